// The caller side of the boundary for the Granite-4.0 hybrid: parameter
// storage (model/model.cpp:959-1160), the KV cache (inference/kv_cache.*),
// the prefill (inference/generator.cpp:627-983) and the greedy decode loop
// (:221-443, :985-1098), written against the backend's own entry points.
//
// The decode step keeps all of its control state on the device (token,
// cache length, ring start, slot), so the whole step -- embedding, 6 layers,
// lm_head, argmax -- can be captured once into a hipGraph and replayed per
// token without host round trips (the reference synchronises per MoE layer
// and per sampled token, cuda/moe.cu:709-729).
#include <map>
#include <string>
#include <vector>

#include "gemv_fuse.h"
#include "decode_persistent.h"

namespace gh {

int linear_any(const float* x, const void* w, float* y, int M, int K, int N, int kind);
int launch_f32_to_f16(const float* s, uint16_t* d, int64_t n);
int launch_argmax(const float* l, int V, int32_t* out_dev);
int launch_argmax_record(const float* l, int V, int32_t* out_dev, int32_t* step, int32_t* ids, int cap);
int attn_decode_partials_devctl(const float* q, const uint16_t* kc, const uint16_t* vc, int H, int KV, int hd,
                                int cache_max, const int32_t* ctl, float scale, const float** o_part,
                                const float** ml, int* splits);
int mamba_step_fused(const float* x, const float* nw, float norm_eps, const void* w_in, const float* conv_w,
                     const float* conv_b, const float* dt_bias, const float* a_log, const float* D,
                     const float* norm_w, const void* w_out, float* conv_state, float* ssm_state, float* out,
                     bool add, int d, int d_inner, int conv_dim, int n_heads, int d_head, int d_state, int k,
                     float eps, int kind, const GmFuse* begin = nullptr);
int moe_decode_fused(float* xres, const float* nw, float eps, const float* rw, const float* bias, const void* gates,
                     const void* ups, const void* downs, const void* sh_g, const void* sh_u, const void* sh_d, int N,
                     int d, int E, int ne, int K, int SH, int qkind);
int attention_prefill(const float* q, const float* k, const float* v, float* out, int B, int T, int H, int KV, int hd,
                      float scale, int window);
int attn_decode_devctl(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int H, int KV, int hd,
                       int cache_max, const int32_t* ctl, float scale);
int mamba_forward_impl(const float* x, const void* w_in, const float* conv_w, const float* conv_b,
                       const float* dt_bias, const float* a_log, const float* D, const float* norm_w, const void* w_out,
                       float* state, float* conv_state, float* out, int T, int d, int d_inner, int conv_dim,
                       int n_heads, int d_head, int d_state, int k, float eps, int kind, bool accumulate,
                       const float* pre_nw, float pre_eps);
int linear_norm_skinny(const float* x, int mode, const float* nw, float eps, const void* w, float* y, int M, int K,
                       int N, int kind, int accumulate);  // gemm.hip
int linear_multi_skinny(const float* x, int mode, const float* nw, float eps, int nseg, const void* const* w,
                        float* const* y, uint16_t* const* y16, const int* n, int M, int K, int kind);  // gemm.hip
int linear_acc(const float* x, const void* w, float* y, int M, int K, int N, int kind);  // y += x W^T

// decode control block (device ints)
// ctl[CTL_AMAX..+1]: a 64-bit running argmax key (8-byte aligned), ctl[CTL_AMAX_CNT]: blocks
// done, ctl[CTL_AMAX_NEG0]: logit 0 is -inf; all zero between launches of k_head_argmax.
enum {
    CTL_TOKEN = 0, CTL_LEN = 1, CTL_START = 2, CTL_PINNED = 3, CTL_CAP = 4, CTL_SLOT = 5, CTL_STEP = 6,
    CTL_AMAX = 8, CTL_AMAX_CNT = 10, CTL_AMAX_NEG0 = 11, CTL_N = 12
};
static_assert(CTL_TOKEN == 0 && CTL_LEN == 1 && CTL_START == 2 && CTL_PINNED == 3 && CTL_CAP == 4 && CTL_SLOT == 5,
              "decode_alloc_slot (gemv_fuse.h) indexes the control block by these positions");

// KVCache::allocate_slot (inference/kv_cache.h:74-92) on the device.
__global__ void k_alloc_slot(int32_t* ctl) { decode_alloc_slot(ctl); }

// K/V of one token -> fp16 cache rows at the slot chosen by k_alloc_slot.
__global__ void k_store_kv(const float* __restrict__ k, const float* __restrict__ v, uint16_t* __restrict__ kc,
                           uint16_t* __restrict__ vc, const int32_t* __restrict__ ctl, int kvd) {
    const size_t base = (size_t)ctl[CTL_SLOT] * kvd;
    for (int i = threadIdx.x; i < kvd; i += blockDim.x) {
        kc[base + i] = f32_to_f16(k[i]);
        vc[base + i] = f32_to_f16(v[i]);
    }
}

// token -> ids[step++] after the argmax wrote ctl[CTL_TOKEN]
__global__ void k_record_token(int32_t* ctl, int32_t* ids, int cap) {
    const int s = ctl[CTL_STEP];
    if (s < cap) ids[s] = ctl[CTL_TOKEN];
    ctl[CTL_STEP] = s + 1;
}

// Start of a decode step: the cache slot of the new token (k_alloc_slot)
// and its embedding row (elementwise.hip k_embed_half) in one launch.
__global__ void k_step_begin(int32_t* ctl, const uint16_t* __restrict__ tab, float* __restrict__ x, int dim,
                             int vocab) {
    if (threadIdx.x == 0) decode_alloc_slot(ctl);
    const int id = ctl[CTL_TOKEN];
    for (int i = threadIdx.x; i < dim; i += blockDim.x)
        x[i] = (id < 0 || id >= vocab) ? 0.f : f16_to_f32(tab[(size_t)id * dim + i]);
}


// Argmax key of logit v at index i, ordered like core/math_cpu.cpp:710-723
// (first finite maximum, strict '>', so the lower index wins ties; -0 counts
// as +0, they compare equal there): a finite value becomes an order-preserving
// unsigned number (>= 0x00800000) above ~i. +inf gets 0 above ~i, so the largest
// key is a finite maximum if there is one, else the first +inf; NaN and -inf
// get 0 = "none".
__device__ __forceinline__ uint64_t amax_key(float v, int i) {
    const uint32_t lo = ~(uint32_t)i;
    if (v == __builtin_inff()) return lo;
    if (!isfinite(v)) return 0;
    const uint32_t u = __builtin_bit_cast(uint32_t, v == 0.f ? 0.f : v);
    const uint32_t hi = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)hi << 32) | lo;
}

// End of a decode step in one launch: final RMSNorm (k_rmsnorm's arithmetic,
// so the normalised row is bit-identical), the tied fp16 lm head
// (model/model.cpp:1087-1160) and, with `argmax`, the greedy pick recorded as
// k_argmax + k_record_token do. Wave w of block b owns RPW consecutive rows
// (block b rows 4 RPW b ..); lane l holds 8-value pieces l, l + 64, ... of x and
// of each row. For d <= 512 a wave takes 16 rows: a quarter of the blocks, so a
// quarter of the device-scope atomics meeting on the key and the counter
// (+1% decode tokens/s on c1 against 4 rows per wave). Every
// block recomputes the norm (d floats from L2) while its weight rows stream in.
// The blocks' best keys meet in a 64-bit atomicMax; the block whose count
// arrives last takes the key, resets it and the counter, and writes the token.
// Device-scope atomics are ordered by waiting for each one's return before the
// next is issued (no cache write-back fence: the logits themselves are not
// read back). With no finite logit the reference's serial scan returns the
// first +inf when l[0] is -inf and 0 otherwise; the block of row 0 reports
// whether l[0] is -inf through ctl[CTL_AMAX_NEG0].
template <int CHM, int RPW>
__global__ void __launch_bounds__(256) k_head_argmax(const float* __restrict__ x, const float* __restrict__ nw,
                                                     float eps, const uint16_t* __restrict__ tab,
                                                     float* __restrict__ logits, int d, int V, int32_t* ctl,
                                                     int32_t* ids, int cap, int argmax) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nch = d >> 3;
    const int row0 = (blockIdx.x * 4 + wave) * RPW;
    // every load issued before the first wait: x pieces + norm weights, weight rows, x for the sum
    float4 xv[CHM][2], nv[CHM][2];
    uint4 wr[RPW][CHM];
#pragma unroll
    for (int i = 0; i < CHM; ++i) {
        const int c = lane + 64 * i;
        if (c < nch) {
            xv[i][0] = ((const float4*)x)[2 * c];
            xv[i][1] = ((const float4*)x)[2 * c + 1];
            nv[i][0] = ((const float4*)nw)[2 * c];
            nv[i][1] = ((const float4*)nw)[2 * c + 1];
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int n = row0 + r < V ? row0 + r : V - 1;
        const uint4* wrow = (const uint4*)(tab + (size_t)n * d);
#pragma unroll
        for (int i = 0; i < CHM; ++i) {
            const int c = lane + 64 * i;
            if (c < nch) wr[r][i] = wrow[c];
        }
    }
    float xs[CHM * 2];
#pragma unroll
    for (int j = 0; j < CHM * 2; ++j)
        if (tid + 256 * j < d) xs[j] = x[tid + 256 * j];
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < CHM * 2; ++j)
        if (tid + 256 * j < d) ss += (double)xs[j] * xs[j];
    __shared__ double red[4];
    __shared__ uint64_t skey[4];
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // LDS only: the weight loads stay in flight
    __builtin_amdgcn_s_barrier();
    const double tot = red[0] + red[1] + red[2] + red[3];
    const double invd = 1.0 / sqrt(tot / (double)d + (double)eps);
    const float inv = isfinite(invd) ? (float)invd : 0.0f;
    float xn[CHM][8];
#pragma unroll
    for (int i = 0; i < CHM; ++i) {
        const float a[8] = {xv[i][0].x, xv[i][0].y, xv[i][0].z, xv[i][0].w,
                            xv[i][1].x, xv[i][1].y, xv[i][1].z, xv[i][1].w};
        const float b[8] = {nv[i][0].x, nv[i][0].y, nv[i][0].z, nv[i][0].w,
                            nv[i][1].x, nv[i][1].y, nv[i][1].z, nv[i][1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) xn[i][e] = a[e] * inv * b[e];
    }
    uint64_t best = 0;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < CHM; ++i) {
            if (lane + 64 * i < nch) {
                const uint32_t wd[4] = {wr[r][i].x, wr[r][i].y, wr[r][i].z, wr[r][i].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc = fmaf(xn[i][2 * e], f16_to_f32((uint16_t)(wd[e] & 0xFFFF)), acc);
                    acc = fmaf(xn[i][2 * e + 1], f16_to_f32((uint16_t)(wd[e] >> 16)), acc);
                }
            }
        }
        acc = wave_total63(acc);
        const int n = row0 + r;
        if (lane == 63 && n < V) {
            logits[n] = acc;
            const uint64_t k = amax_key(acc, n);
            best = k > best ? k : best;
            if (argmax && n == 0 && acc == -__builtin_inff()) {
                (void)__hip_atomic_fetch_or(ctl + CTL_AMAX_NEG0, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): performed before the block's count
            }
        }
    }
    if (!argmax) return;
    if (lane == 63) skey[wave] = best;
    __syncthreads();
    if (tid == 0) {
        uint64_t k = skey[0];
#pragma unroll
        for (int w = 1; w < 4; ++w) k = skey[w] > k ? skey[w] : k;
        unsigned long long* keyp = (unsigned long long*)(ctl + CTL_AMAX);
        unsigned int* cntp = (unsigned int*)(ctl + CTL_AMAX_CNT);
        if (k) {
            (void)__hip_atomic_fetch_max(keyp, (unsigned long long)k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0x0F70);
        }
        if (__hip_atomic_fetch_add(cntp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1) {
            const uint64_t fin = __hip_atomic_exchange(keyp, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int neg0 = __hip_atomic_exchange(ctl + CTL_AMAX_NEG0, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            (void)__hip_atomic_exchange(cntp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            int bi = 0;
            if (fin >> 32) bi = (int)~(uint32_t)fin;                // finite maximum
            else if (fin && neg0) bi = (int)~(uint32_t)fin;        // no finite value: first +inf after l[0] = -inf
            ctl[CTL_TOKEN] = bi;
            if (ids) {
                const int s = ctl[CTL_STEP];
                if (s < cap) ids[s] = bi;
                ctl[CTL_STEP] = s + 1;
            }
        }
    }
}

// After a prefill of P tokens: cache length P, ring start 0, decode step 0.
__global__ void k_ctl_prefilled(int32_t* ctl, int P) {
    if (threadIdx.x == 0) {
        ctl[CTL_LEN] = P;
        ctl[CTL_START] = 0;
        ctl[CTL_STEP] = 0;
    }
}

// Returns 1 if launched (fp16 table, d a multiple of 8 up to 2048, 16-byte aligned rows).
static int launch_head_argmax(const float* x, const float* nw, float eps, const uint16_t* tab, float* logits, int d,
                              int V, int32_t* ctl, int32_t* ids, int cap, bool argmax) {
    if (d % 8 || d > 2048 || (((uintptr_t)x | (uintptr_t)nw | (uintptr_t)tab) & 15)) return 0;
    const dim3 blk(256);
    if (d <= 512)
        hipLaunchKernelGGL((k_head_argmax<1, 16>), dim3(cdiv(V, 4 * 16)), blk, 0, stream(), x, nw, eps, tab, logits, d, V, ctl, ids, cap, argmax);
    else if (d <= 1024)
        hipLaunchKernelGGL((k_head_argmax<2, 4>), dim3(cdiv(V, 16)), blk, 0, stream(), x, nw, eps, tab, logits, d, V, ctl, ids, cap, argmax);
    else
        hipLaunchKernelGGL((k_head_argmax<4, 4>), dim3(cdiv(V, 16)), blk, 0, stream(), x, nw, eps, tab, logits, d, V, ctl, ids, cap, argmax);
    GH_LAUNCHED("k_head_argmax");
    return 1;
}
}  // namespace gh

using namespace gh;

struct Param {
    std::string name;
    int64_t numel;
    int storage;  // 0 packed (qkind), 1 fp16, 2 fp32
    size_t nbytes, off;
};

static const char* const STATE_INVALID_MSG =
    "the model state is invalid after an aborted persistent decode (call gh_granite_reset, then prefill again)";

struct gh_granite {
    int V, d, L, H, KV, hd, E, ne, K, SH, di, mh, mdh, mds, ck, qkind;
    std::vector<int> lt;
    float eps, scale;
    // Granite multipliers (model/model.cpp:2431-2432, 2531; inference/generator.cpp:248, 266, 440):
    // embeddings x emb_mult, every branch output x res_mult before its residual add, logits x
    // (1 / logits_scaling). tied: the lm head is tok_embeddings, else its own fp16 "lm_head"
    // [V, d] (model/model.cpp:1160). aux_free: per-layer router bias "layers.N.moe_bias" [ne]
    // added to the probabilities for the selection (model/model.cpp:179-194).
    float emb_mult = 1.0f, res_mult = 1.0f, logits_scaling = 1.0f;
    bool tied = true, aux_free = false;
    bool plain_multipliers() const { return emb_mult == 1.0f && res_mult == 1.0f; }
    const char* head_name() const { return tied ? "tok_embeddings" : "lm_head"; }
    int max_ctx, conv_dim, proj, qd, kvd, pinned_cfg;
    std::vector<Param> params;
    std::map<std::string, size_t> by_name;
    uint8_t* wbuf = nullptr;
    size_t wbytes = 0;
    // state
    std::map<int, float*> conv, ssm;
    std::map<int, uint16_t*> kc, vc;
    float* state_buf = nullptr;
    // activations (prefill sized)
    float *x = nullptr, *xb = nullptr, *pr = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr,
          *logits = nullptr;
    int32_t *ids = nullptr, *ctl = nullptr, *gen_ids = nullptr;
    int act_rows = 0;
    int host_len = 0;  // cache length mirror
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    hipStream_t cap_stream = nullptr;  // the stream the graph was captured on; lives as long as the graph
    uint64_t graph_ws_gen = 0;         // workspace generation the graph's buffer addresses belong to
    // persistent decode loop: its model description (device copy) and hand-over buffers
    PdModel* pd_dev = nullptr;
    uint8_t* pd_buf = nullptr;
    size_t pd_zero_bytes = 0;  // bytes of pd_buf zeroed before each launch (all of it)
    // An aborted persistent launch leaves the recurrent state, the KV cache and the generated
    // ids partly advanced: the model refuses every call that reads that state until a reset.
    bool state_invalid = false;
    int32_t* ids_pin = nullptr;  // pinned host staging of a prompt's ids (an asynchronous H2D copy)
    int ids_pin_cap = 0;
    bool pd_force_abort = false;  // test hook: the next persistent launch starts aborted

    const void* W(const std::string& n) const {
        auto it = by_name.find(n);
        return it == by_name.end() ? nullptr : wbuf + params[it->second].off;
    }
    const float* F(const std::string& n) const { return (const float*)W(n); }
};

static void add_param(gh_granite* g, const std::string& name, int64_t numel, int storage) {
    Param p;
    p.name = name;
    p.numel = numel;
    p.storage = storage;
    if (storage == 0) p.nbytes = (size_t)(numel / block_values(g->qkind)) * block_bytes(g->qkind);
    else p.nbytes = (size_t)numel * (storage == 1 ? 2 : 4);
    p.off = 0;
    g->by_name[name] = g->params.size();
    g->params.push_back(p);
}

static void free_all(gh_granite* g) {
    if (g->graph_exec) (void)hipGraphExecDestroy(g->graph_exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    if (g->cap_stream) {
        (void)hipStreamSynchronize(g->cap_stream);
        (void)hipStreamDestroy(g->cap_stream);
    }
    if (g->pd_dev) (void)hipFree(g->pd_dev);
    if (g->pd_buf) (void)hipFree(g->pd_buf);
    if (g->ids_pin) (void)hipHostFree(g->ids_pin);
    void* ptrs[] = {g->wbuf, g->state_buf, g->x, g->ids, g->ctl, g->gen_ids};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
}

static int ensure_acts(gh_granite* g, int rows) {
    if (rows <= g->act_rows) return GH_OK;
    if (g->x) GH_HIP(hipFree(g->x));
    const size_t d = g->d;
    const size_t per = 2 * d + d + (size_t)g->qd + 2 * (size_t)g->kvd + g->qd;
    size_t n = (size_t)rows * per + g->V + 64;
    GH_HIP(hipMalloc(&g->x, n * 4));
    g->xb = g->x + rows * d;
    g->pr = g->xb + rows * d;
    g->q = g->pr + rows * d;
    g->k = g->q + (size_t)rows * g->qd;
    g->v = g->k + (size_t)rows * g->kvd;
    g->att = g->v + (size_t)rows * g->kvd;
    g->logits = g->att + (size_t)rows * g->qd;
    g->act_rows = rows;
    return GH_OK;
}

#define GHC(call)                      \
    do {                               \
        int rc_ = (call);              \
        if (rc_) return rc_;           \
    } while (0)

// Model::moe_bias_ptr (model/model.cpp:192-199): the layer's router bias, or null
static const float* moe_bias(const gh_granite* g, int l) {
    return g->aux_free ? g->F("layers." + std::to_string(l) + ".moe_bias") : nullptr;
}

// x += res_mult * branch (inference/generator.cpp:266-268: scale_inplace, then add_inplace;
// two roundings, as the reference does them)
static int add_branch(gh_granite* g, float* branch, int64_t n) {
    if (g->res_mult != 1.0f) GHC(gh_scale_inplace(branch, g->res_mult, n));
    return gh_add_inplace(g->x, branch, n);
}

// final norm output -> logits (inference/generator.cpp:438-441)
static int lm_head(gh_granite* g, const float* xb) {
    GHC(linear_any(xb, g->W(g->head_name()), g->logits, 1, g->d, g->V, 4));
    if (g->logits_scaling != 1.0f) GHC(gh_scale_inplace(g->logits, 1.0f / g->logits_scaling, g->V));
    return GH_OK;
}

static int moe_layer(gh_granite* g, int l, const float* xb, float* out, int n) {
    const std::string pre = "layers." + std::to_string(l) + ".";
    return gh_moe_forward_bias_half(xb, g->F(pre + "moe_router"), moe_bias(g, l), g->W(pre + "moe_gate"), g->W(pre + "moe_up"),
                                    g->W(pre + "moe_down"), g->W(pre + "moe_sh_gate"), g->W(pre + "moe_sh_up"),
                                    g->W(pre + "moe_sh_down"), out, nullptr, nullptr, nullptr, nullptr, nullptr,
                                    nullptr, n, g->d, g->E, g->ne, g->K, g->SH, g->qkind);
}

static int mamba_step(gh_granite* g, int l, const float* xin, float* out) {
    const std::string mp = "layers." + std::to_string(l) + ".mamba.";
    return gh_mamba2_step_half(xin, g->W(mp + "in_proj"), g->F(mp + "conv1d.weight"), g->F(mp + "conv1d.bias"),
                               g->F(mp + "dt_bias"), g->F(mp + "A_log"), g->F(mp + "D"), g->F(mp + "norm.weight"),
                               g->W(mp + "out_proj"), g->conv[l], g->ssm[l], out, g->d, g->di, g->conv_dim, g->mh,
                               g->mdh, g->mds, g->ck, g->eps, g->qkind);
}

// One decode step for the token in ctl[CTL_TOKEN] (inference/generator.cpp:221-443),
// ending with the greedy argmax written back to ctl[CTL_TOKEN] and recorded.
static int decode_step_dev(gh_granite* g, bool argmax) {
    const int d = g->d;
    hipLaunchKernelGGL(k_alloc_slot, dim3(1), dim3(1), 0, stream(), g->ctl);
    GHC(gh_embedding_forward_half(g->ctl + CTL_TOKEN, (const uint16_t*)g->W("tok_embeddings"), g->x, 1, d, g->V));
    if (g->emb_mult != 1.0f) GHC(gh_scale_inplace(g->x, g->emb_mult, d));
    for (int l = 0; l < g->L; ++l) {
        const std::string pre = "layers." + std::to_string(l) + ".";
        GHC(gh_rmsnorm_forward(g->x, g->F(pre + "attn_norm"), g->xb, nullptr, 1, d, g->eps));
        if (g->lt[l] == 0) {
            GHC(mamba_step(g, l, g->xb, g->pr));
        } else {
            GHC(linear_any(g->xb, g->W(pre + "wq"), g->q, 1, d, g->qd, g->qkind));
            GHC(linear_any(g->xb, g->W(pre + "wk"), g->k, 1, d, g->kvd, g->qkind));
            GHC(linear_any(g->xb, g->W(pre + "wv"), g->v, 1, d, g->kvd, g->qkind));
            hipLaunchKernelGGL(k_store_kv, dim3(1), dim3(256), 0, stream(), g->k, g->v, g->kc[l], g->vc[l], g->ctl,
                               g->kvd);
            GHC(attn_decode_devctl(g->q, g->kc[l], g->vc[l], g->att, g->H, g->KV, g->hd, g->max_ctx, g->ctl, g->scale));
            GHC(linear_any(g->att, g->W(pre + "wo"), g->pr, 1, g->qd, d, g->qkind));
        }
        GHC(add_branch(g, g->pr, d));
        GHC(gh_rmsnorm_forward(g->x, g->F(pre + "ffn_norm"), g->xb, nullptr, 1, d, g->eps));
        GHC(moe_layer(g, l, g->xb, g->pr, 1));
        GHC(add_branch(g, g->pr, d));
    }
    GHC(gh_rmsnorm_forward(g->x, g->F("final_norm"), g->xb, nullptr, 1, d, g->eps));
    GHC(lm_head(g, g->xb));
    if (argmax) {
        GHC(launch_argmax(g->logits, g->V, g->ctl + CTL_TOKEN));
        hipLaunchKernelGGL(k_record_token, dim3(1), dim3(1), 0, stream(), g->ctl, g->gen_ids, g->max_ctx);
    }
    GH_LAUNCHED("decode_step");
    return GH_OK;
}

// The same step with every sub-layer fused into few launches: per Mamba
// layer 3 ([norm+in_proj+conv], scan, [gated norm+out_proj+residual]), per
// attention layer 3 ([norm+q/k/v+cache store], split-K partials,
// [merge+wo+residual]), per MoE 3 ([norm+route], gate/up, [down+combine+
// residual]); begin, lm head and argmax+record around them. Returns
// GH_EUNSUPPORTED before launching anything if a shape does not fit.
namespace gh {
int attn_chunk_min();
int moe_forward_acc(const float* x, const float* router_w, const float* router_bias, const void* gates,
                    const void* ups, const void* downs, const void* sh_g, const void* sh_u, const void* sh_d,
                    float* out, float* acc_dst, int* added, float* probs_cache, int32_t* idx_cache, float* w_cache,
                    int64_t N, int d, int E, int ne, int K, int SH, int qkind, const float* nw, float eps,
                    float* xn);
}
static bool fused_supported(const gh_granite* g) {
    const int k = g->qkind;
    if (k != 2 && k != 3) return false;
    // the fused launches add branch outputs into the residual stream unscaled and take the
    // embedding row as is: other multipliers run the step launch by launch
    if (!g->plain_multipliers()) return false;
    if (g->d % 256 || g->di % 256 || g->qd % 256 || g->qd % 16 || g->kvd % 16) return false;
    if (g->mds != 64 && g->mds != 128) return false;
    const int chunk_min = attn_chunk_min();
    if ((g->max_ctx + chunk_min - 1) / chunk_min > 64) return false;  // attention merge in the wo prologue
    return true;
}

static int decode_step_fused(gh_granite* g, bool argmax) {
    const int d = g->d;
    // the step's start (slot + embedding row) runs inside layer 0's first GEMV when its path
    // takes it; otherwise (GH_EUNSUPPORTED before any launch) as k_step_begin
    GmFuse begin;
    begin.emb = (const uint16_t*)g->W("tok_embeddings");
    begin.emb_out = g->x;
    begin.bctl = g->ctl;
    begin.vocab = g->V;
    bool begun = false;
    auto launch_begin = [&]() -> int {
        hipLaunchKernelGGL(k_step_begin, dim3(1), dim3(256), 0, stream(), g->ctl, begin.emb, g->x, d, g->V);
        GH_LAUNCHED("k_step_begin");
        begun = true;
        return GH_OK;
    };
    for (int l = 0; l < g->L; ++l) {
        const std::string pre = "layers." + std::to_string(l) + ".";
        if (g->lt[l] == 0) {
            const std::string mp = pre + "mamba.";
            auto run = [&](const GmFuse* b) {
                return mamba_step_fused(g->x, g->F(pre + "attn_norm"), g->eps, g->W(mp + "in_proj"),
                                        g->F(mp + "conv1d.weight"), g->F(mp + "conv1d.bias"), g->F(mp + "dt_bias"),
                                        g->F(mp + "A_log"), g->F(mp + "D"), g->F(mp + "norm.weight"),
                                        g->W(mp + "out_proj"), g->conv[l], g->ssm[l], g->x, true, d, g->di,
                                        g->conv_dim, g->mh, g->mdh, g->mds, g->ck, g->eps, g->qkind, b);
            };
            if (!begun) {
                const int rc = run(&begin);
                if (rc == GH_OK) {
                    begun = true;
                } else {
                    if (rc != GH_EUNSUPPORTED) return rc;
                    GHC(launch_begin());
                    GHC(run(nullptr));
                }
            } else {
                GHC(run(nullptr));
            }
        } else {
            if (!begun) GHC(launch_begin());
            GmFuse f1;
            f1.pro = GM_PRO_RMSNORM;
            f1.pw = g->F(pre + "attn_norm");
            f1.eps = g->eps;
            f1.w1 = g->W(pre + "wk");
            f1.w2 = g->W(pre + "wv");
            f1.n0 = g->qd;
            f1.n1 = g->kvd;
            f1.epi = GM_EPI_QKV;
            f1.kc = g->kc[l];
            f1.vc = g->vc[l];
            f1.slot = g->ctl + CTL_SLOT;
            f1.kvd = g->kvd;
            GHC(gemv_fused(g->x, g->W(pre + "wq"), g->q, d, g->qd + 2 * g->kvd, g->qkind, f1));
            GmFuse f3;
            GHC(attn_decode_partials_devctl(g->q, g->kc[l], g->vc[l], g->H, g->KV, g->hd, g->max_ctx, g->ctl, g->scale,
                                            &f3.o_part, &f3.ml, &f3.splits));
            f3.pro = GM_PRO_ATTN;
            f3.H = g->H;
            f3.KV = g->KV;
            f3.G = g->H / g->KV;
            f3.hd = g->hd;
            f3.epi = GM_EPI_ADD;
            GHC(gemv_fused(g->q, g->W(pre + "wo"), g->x, g->qd, d, g->qkind, f3));
        }
        GHC(moe_decode_fused(g->x, g->F(pre + "ffn_norm"), g->eps, g->F(pre + "moe_router"), moe_bias(g, l),
                             g->W(pre + "moe_gate"), g->W(pre + "moe_up"), g->W(pre + "moe_down"),
                             g->W(pre + "moe_sh_gate"), g->W(pre + "moe_sh_up"), g->W(pre + "moe_sh_down"), 1, d, g->E,
                             g->ne, g->K, g->SH, g->qkind));
    }
    // the one-launch tail picks the id from unscaled logits: with a logits_scaling it runs as
    // norm, head, scale and argmax launches (the scaled values decide ties, as in the reference)
    if (g->logits_scaling == 1.0f &&
        launch_head_argmax(g->x, g->F("final_norm"), g->eps, (const uint16_t*)g->W(g->head_name()), g->logits, d,
                           g->V, g->ctl, g->gen_ids, g->max_ctx, argmax)) {
        GH_LAUNCHED("decode_step");
        return GH_OK;
    }
    GHC(gh_rmsnorm_forward(g->x, g->F("final_norm"), g->xb, nullptr, 1, d, g->eps));
    GHC(lm_head(g, g->xb));
    if (argmax)
        GHC(launch_argmax_record(g->logits, g->V, g->ctl + CTL_TOKEN, g->ctl + CTL_STEP, g->gen_ids, g->max_ctx));
    GH_LAUNCHED("decode_step");
    return GH_OK;
}

static int decode_step(gh_granite* g, bool argmax) {
    if (fused_supported(g)) return decode_step_fused(g, argmax);
    return decode_step_dev(g, argmax);
}

extern "C" {

// Final norm + tied fp16 lm head + greedy id in one launch (the tail of a
// decode step), for callers outside a model; the id goes to a device int.
int gh_lm_head_greedy_dev(const float* x, const float* norm_w, float eps, const uint16_t* tab, float* logits, int d,
                          int V, int32_t* out_dev) {
    GH_REQUIRE(x && norm_w && tab && logits && out_dev && d > 0 && V > 0, "lm_head_greedy: bad arguments");
    int32_t* ctl = (int32_t*)workspace(WS_HEAD_CTL, CTL_N * 4);
    if (!ctl) return fail(GH_ENOMEM, "lm_head_greedy: workspace");
    // a fill kernel, not a memset node: this entry point is meant for captured graphs
    const int zrc = gh_zero((float*)ctl, CTL_N);
    if (zrc) return zrc;
    if (!launch_head_argmax(x, norm_w, eps, tab, logits, d, V, ctl, nullptr, 0, true))
        return fail(GH_EUNSUPPORTED, "lm_head_greedy: d=%d (needs d %% 8 == 0, d <= 2048, 16-byte aligned rows)", d);
    GH_HIP(hipMemcpyAsync(out_dev, ctl + CTL_TOKEN, 4, hipMemcpyDeviceToDevice, stream()));
    return GH_OK;
}

int gh_granite_create(const int32_t* cfg, const float* fcfg, int max_ctx, gh_granite** out) {
    GH_REQUIRE(cfg && fcfg && out, "granite_create: null argument");
    GH_REQUIRE(cfg[2] > 0 && cfg[2] <= 1024, "granite_create: bad layer count %d", cfg[2]);
    return gh_granite_create_ex(cfg, 16 + cfg[2], fcfg, 2, max_ctx, out);
}

int gh_granite_create_ex(const int32_t* cfg, int ncfg, const float* fcfg, int nfcfg, int max_ctx, gh_granite** out) {
    GH_REQUIRE(cfg && fcfg && out && ncfg >= 17 && nfcfg >= 2, "granite_create: null argument or short arrays");
    GH_REQUIRE(cfg[2] > 0 && cfg[2] <= 1024 && ncfg >= 16 + cfg[2], "granite_create: bad layer count %d", cfg[2]);
    const int L0 = cfg[2];
    const float emb_mult = nfcfg > 2 ? fcfg[2] : 1.0f, res_mult = nfcfg > 3 ? fcfg[3] : 1.0f,
                logits_scaling = nfcfg > 4 ? fcfg[4] : 1.0f;
    // model/model.cpp:360-366: logits_scaling is a divisor, the multipliers must be finite
    GH_REQUIRE(std::isfinite(logits_scaling) && logits_scaling > 0.0f,
               "granite_create: logits_scaling must be finite and > 0");
    GH_REQUIRE(std::isfinite(emb_mult) && std::isfinite(res_mult), "granite_create: multipliers must be finite");
    gh_granite* g = new gh_granite();
    g->emb_mult = emb_mult;
    g->res_mult = res_mult;
    g->logits_scaling = logits_scaling;
    g->tied = ncfg > 16 + L0 ? cfg[16 + L0] != 0 : true;
    g->aux_free = ncfg > 17 + L0 ? cfg[17 + L0] != 0 : false;
    g->V = cfg[0]; g->d = cfg[1]; g->L = cfg[2]; g->H = cfg[3]; g->KV = cfg[4]; g->hd = cfg[5]; g->E = cfg[6];
    g->ne = cfg[7]; g->K = cfg[8]; g->SH = cfg[9]; g->di = cfg[10]; g->mh = cfg[11]; g->mdh = cfg[12];
    g->mds = cfg[13]; g->ck = cfg[14]; g->qkind = cfg[15];
    g->lt.assign(cfg + 16, cfg + 16 + g->L);
    g->eps = fcfg[0];
    g->scale = fcfg[1];
    g->max_ctx = max_ctx;
    g->conv_dim = g->di + 2 * g->mds;
    g->proj = g->di + g->conv_dim + g->mh;
    g->qd = g->H * g->hd;
    g->kvd = g->KV * g->hd;
    g->pinned_cfg = max_ctx - 1 < 8 ? (max_ctx - 1 > 0 ? max_ctx - 1 : 0) : 8;  // generator.cpp:94
    if (!valid_kind(g->qkind) || max_ctx < 2 || g->L <= 0 || g->H % g->KV) {
        delete g;
        return fail(GH_EINVAL, "granite_create: bad configuration");
    }
    // parameter table, model/model.cpp:1087-1160
    const int64_t d = g->d;
    add_param(g, "tok_embeddings", (int64_t)g->V * d, 1);
    for (int i = 0; i < g->L; ++i) {
        const std::string pre = "layers." + std::to_string(i) + ".";
        add_param(g, pre + "attn_norm", d, 2);
        add_param(g, pre + "ffn_norm", d, 2);
        if (g->lt[i] == 0) {
            const std::string mp = pre + "mamba.";
            add_param(g, mp + "in_proj", (int64_t)g->proj * d, 0);
            add_param(g, mp + "conv1d.weight", (int64_t)g->conv_dim * g->ck, 2);
            add_param(g, mp + "conv1d.bias", g->conv_dim, 2);
            add_param(g, mp + "dt_bias", g->mh, 2);
            add_param(g, mp + "A_log", g->mh, 2);
            add_param(g, mp + "D", g->mh, 2);
            add_param(g, mp + "norm.weight", g->di, 2);
            add_param(g, mp + "out_proj", d * g->di, 0);
        } else {
            add_param(g, pre + "wq", (int64_t)g->qd * d, 0);
            add_param(g, pre + "wk", (int64_t)g->kvd * d, 0);
            add_param(g, pre + "wv", (int64_t)g->kvd * d, 0);
            add_param(g, pre + "wo", d * g->qd, 0);
        }
        add_param(g, pre + "moe_router", (int64_t)g->ne * d, 2);
        add_param(g, pre + "moe_gate", (int64_t)g->ne * g->E * d, 0);
        add_param(g, pre + "moe_up", (int64_t)g->ne * g->E * d, 0);
        add_param(g, pre + "moe_down", (int64_t)g->ne * d * g->E, 0);
        add_param(g, pre + "moe_sh_gate", (int64_t)g->SH * d, 0);
        add_param(g, pre + "moe_sh_up", (int64_t)g->SH * d, 0);
        add_param(g, pre + "moe_sh_down", d * g->SH, 0);
        if (g->aux_free) add_param(g, pre + "moe_bias", g->ne, 2);
    }
    add_param(g, "final_norm", d, 2);
    if (!g->tied) add_param(g, "lm_head", (int64_t)g->V * d, 1);  // fp16, like tok_embeddings
    size_t off = 0;
    for (Param& p : g->params) {
        p.off = off;
        off += (p.nbytes + 255) & ~(size_t)255;
    }
    g->wbytes = off;
    hipError_t e = hipMalloc(&g->wbuf, off);
    if (e != hipSuccess) {
        delete g;
        return fail(GH_ENOMEM, "granite_create: %zu bytes of weights: %s", off, hipGetErrorString(e));
    }
    // recurrent state + KV caches in one allocation
    size_t sbytes = 0;
    for (int l = 0; l < g->L; ++l) {
        if (g->lt[l] == 0) sbytes += ((size_t)g->conv_dim * (g->ck - 1) + (size_t)g->mh * g->mdh * g->mds) * 4;
        else sbytes += (size_t)2 * g->max_ctx * g->kvd * 2;
    }
    e = hipMalloc(&g->state_buf, sbytes + 256);
    if (e == hipSuccess) e = hipMalloc(&g->ids, (size_t)1024 * 4);
    if (e == hipSuccess) e = hipMalloc(&g->ctl, CTL_N * 4);
    if (e == hipSuccess) e = hipMalloc(&g->gen_ids, (size_t)(g->max_ctx + 1) * 4);
    if (e != hipSuccess) {
        free_all(g);
        delete g;
        return fail(GH_ENOMEM, "granite_create: state allocation failed");
    }
    uint8_t* sp = (uint8_t*)g->state_buf;
    for (int l = 0; l < g->L; ++l) {
        if (g->lt[l] == 0) {
            g->conv[l] = (float*)sp;
            sp += (size_t)g->conv_dim * (g->ck - 1) * 4;
            g->ssm[l] = (float*)sp;
            sp += (size_t)g->mh * g->mdh * g->mds * 4;
        } else {
            g->kc[l] = (uint16_t*)sp;
            sp += (size_t)g->max_ctx * g->kvd * 2;
            g->vc[l] = (uint16_t*)sp;
            sp += (size_t)g->max_ctx * g->kvd * 2;
        }
    }
    int rc = ensure_acts(g, 1);
    if (rc == GH_OK) rc = gh_granite_reset(g);
    if (rc) {
        free_all(g);
        delete g;
        return rc;
    }
    *out = g;
    return GH_OK;
}

int gh_granite_destroy(gh_granite* g) {
    if (!g) return GH_OK;
    (void)hipStreamSynchronize(stream());
    free_all(g);
    delete g;
    return GH_OK;
}

int gh_granite_param_count(gh_granite* g) { return g ? (int)g->params.size() : 0; }

int gh_granite_param_name(gh_granite* g, int i, const char** name, size_t* nbytes) {
    GH_REQUIRE(g && i >= 0 && i < (int)g->params.size() && name && nbytes, "granite_param_name: bad arguments");
    *name = g->params[(size_t)i].name.c_str();
    *nbytes = g->params[(size_t)i].nbytes;
    return GH_OK;
}

int gh_granite_set_param(gh_granite* g, const char* name, const void* host, size_t nbytes) {
    GH_REQUIRE(g && name && host, "granite_set_param: null argument");
    auto it = g->by_name.find(name);
    GH_REQUIRE(it != g->by_name.end(), "granite_set_param: unknown parameter %s", name);
    const Param& p = g->params[it->second];
    GH_REQUIRE(nbytes == p.nbytes, "granite_set_param: %s expects %zu bytes, got %zu", name, p.nbytes, nbytes);
    GH_HIP(hipMemcpy(g->wbuf + p.off, host, nbytes, hipMemcpyHostToDevice));
    return GH_OK;
}

int gh_granite_load_gguf(gh_granite* g, const gh_gguf* f) {
    GH_REQUIRE(g && f, "granite_load_gguf: null argument");
    for (const Param& p : g->params) {
        const bool is_bias = p.name.size() > 9 && p.name.compare(p.name.size() - 9, 9, ".moe_bias") == 0;
        std::string src = p.name;
        int64_t ti = gh_gguf_find_tensor(f, src.c_str());
        if (ti < 0 && p.name == "lm_head") {
            // no output projection in the file: the token embedding serves as the lm head
            // (format/gguf_codec.cpp:1517-1523)
            src = "tok_embeddings";
            ti = gh_gguf_find_tensor(f, src.c_str());
        }
        if (ti < 0 && is_bias) {
            // a router bias absent from the file stays zero (format/gguf_codec.cpp:1549-1556)
            GH_HIP(hipMemset(g->wbuf + p.off, 0, p.nbytes));
            continue;
        }
        GH_REQUIRE(ti >= 0, "granite_load_gguf: tensor not found: %s", p.name.c_str());
        int nd = 0;
        uint64_t dims[8], nb = 0;
        GHC(gh_gguf_tensor_info(f, ti, nullptr, nullptr, &nd, dims, &nb));
        uint64_t numel = 1;
        for (int i = 0; i < nd; ++i) numel *= dims[i];
        GH_REQUIRE(numel == (uint64_t)p.numel, "granite_load_gguf: %s has %llu values, the model needs %lld",
                   p.name.c_str(), (unsigned long long)numel, (long long)p.numel);
        void* dst = g->wbuf + p.off;
        if (p.storage == 0) GHC(gh_gguf_read_packed(f, src.c_str(), g->qkind, dst, GH_DEV_GPU, p.nbytes));
        else if (p.storage == 1) GHC(gh_gguf_read_f16(f, src.c_str(), (uint16_t*)dst, GH_DEV_GPU, (size_t)p.numel));
        else GHC(gh_gguf_read_f32(f, src.c_str(), (float*)dst, GH_DEV_GPU, (size_t)p.numel));
    }
    return GH_OK;
}

int gh_granite_open_gguf(const char* path, int qkind, int max_ctx, gh_granite** out) {
    GH_REQUIRE(path && out, "granite_open_gguf: null argument");
    *out = nullptr;
    gh_gguf* f = nullptr;
    int rc = gh_gguf_open(path, &f);
    if (rc != GH_OK) return rc;
    int32_t cfg[18 + 1024];
    float fcfg[5];
    int ncfg = 0;
    gh_granite* g = nullptr;
    rc = gh_gguf_granite_config(f, qkind, cfg, (int)(sizeof cfg / sizeof cfg[0]), fcfg, 5, &ncfg);
    if (rc == GH_OK) rc = gh_granite_create_ex(cfg, ncfg, fcfg, 5, max_ctx, &g);
    if (rc == GH_OK) rc = gh_granite_load_gguf(g, f);
    gh_gguf_close(f);
    if (rc != GH_OK) {
        if (g) gh_granite_destroy(g);  // keeps the first failure's message: destroy does not fail here
        return rc;
    }
    *out = g;
    return GH_OK;
}

int gh_granite_get_param(gh_granite* g, const char* name, void* host, size_t nbytes) {
    GH_REQUIRE(g && name && host, "granite_get_param: null argument");
    auto it = g->by_name.find(name);
    GH_REQUIRE(it != g->by_name.end(), "granite_get_param: unknown parameter %s", name);
    const Param& p = g->params[it->second];
    GH_REQUIRE(nbytes == p.nbytes, "granite_get_param: %s has %zu bytes", name, p.nbytes);
    GH_HIP(hipMemcpy(host, g->wbuf + p.off, nbytes, hipMemcpyDeviceToHost));
    return GH_OK;
}

int gh_granite_init_synthetic(gh_granite* g, uint64_t seed) {
    GH_REQUIRE(g != nullptr, "granite_init_synthetic: null model");
    std::vector<float> f;
    std::vector<uint8_t> b;
    for (const Param& p : g->params) {
        f.resize((size_t)p.numel);
        GHC(gh_synth_param_f32(p.name.c_str(), seed, f.data(), p.numel));
        b.resize(p.nbytes);
        if (p.storage == 0) {
            GHC(gh_quantize_host(g->qkind, f.data(), b.data(), p.numel));
        } else if (p.storage == 1) {
            uint16_t* h = (uint16_t*)b.data();
            for (int64_t i = 0; i < p.numel; ++i) h[i] = f32_to_f16(f[(size_t)i]);
        } else {
            memcpy(b.data(), f.data(), p.nbytes);
        }
        GHC(gh_granite_set_param(g, p.name.c_str(), b.data(), p.nbytes));
    }
    return GH_OK;
}

int gh_granite_test_force_abort(gh_granite* g) {
    GH_REQUIRE(g != nullptr, "granite_test_force_abort: null model");
    g->pd_force_abort = true;
    return GH_OK;
}

int gh_granite_reset(gh_granite* g) {
    GH_REQUIRE(g != nullptr, "granite_reset: null model");
    size_t sbytes = 0;
    for (int l = 0; l < g->L; ++l) {
        if (g->lt[l] == 0) sbytes += ((size_t)g->conv_dim * (g->ck - 1) + (size_t)g->mh * g->mdh * g->mds) * 4;
        else sbytes += (size_t)2 * g->max_ctx * g->kvd * 2;
    }
    GH_HIP(hipMemsetAsync(g->state_buf, 0, sbytes, stream()));
    const int32_t ctl[CTL_N] = {0, 0, 0, g->pinned_cfg, g->max_ctx, 0, 0, 0, 0, 0, 0, 0};
    GH_HIP(hipMemcpyAsync(g->ctl, ctl, sizeof ctl, hipMemcpyHostToDevice, stream()));
    GH_HIP(hipStreamSynchronize(stream()));
    g->host_len = 0;
    g->state_invalid = false;
    return GH_OK;
}

int gh_granite_prefill(gh_granite* g, const int32_t* ids_host, int P, float* logits_host, int mamba_mode) {
    GH_REQUIRE(g && ids_host && P > 0, "granite_prefill: bad arguments");
    GH_REQUIRE(!g->state_invalid, "granite_prefill: %s", STATE_INVALID_MSG);
    GH_REQUIRE(g->host_len == 0, "granite_prefill: the cache is not empty (reset first)");
    GH_REQUIRE(P <= 1024 && P < g->max_ctx, "granite_prefill: %d tokens (batched prefill takes <= 1024 and < ctx)", P);
    const int d = g->d;
    GHC(ensure_acts(g, P));
    // the ids through pinned host memory: a DMA the host does not wait for (the staging buffer is
    // reused only after this call's closing synchronisation)
    if (g->ids_pin_cap < P) {
        if (g->ids_pin) GH_HIP(hipHostFree(g->ids_pin));
        g->ids_pin = nullptr;
        g->ids_pin_cap = 0;
        GH_HIP(hipHostMalloc((void**)&g->ids_pin, (size_t)1024 * 4, hipHostMallocDefault));
        g->ids_pin_cap = 1024;
    }
    memcpy(g->ids_pin, ids_host, (size_t)P * 4);
    GH_HIP(hipMemcpyAsync(g->ids, g->ids_pin, (size_t)P * 4, hipMemcpyHostToDevice, stream()));
    GHC(gh_embedding_forward_half(g->ids, (const uint16_t*)g->W("tok_embeddings"), g->x, P, d, g->V));
    if (g->emb_mult != 1.0f) GHC(gh_scale_inplace(g->x, g->emb_mult, (int64_t)P * d));
    // with a residual multiplier every branch lands in pr first and is scaled there
    const bool acc = g->res_mult == 1.0f;
    for (int l = 0; l < g->L; ++l) {
        const std::string pre = "layers." + std::to_string(l) + ".";
        // the layer's input norm: on the row prologue of the projections that read it where the
        // skinny GEMM takes them, else one k_rmsnorm launch into xb (made at most once)
        bool xb_made = false;
        auto make_xb = [&]() -> int {
            if (!xb_made) GHC(gh_rmsnorm_forward(g->x, g->F(pre + "attn_norm"), g->xb, nullptr, P, d, g->eps));
            xb_made = true;
            return GH_OK;
        };
        auto proj_normed = [&](const void* w, float* y, int N) -> int {
            const int rc = linear_norm_skinny(g->x, 1, g->F(pre + "attn_norm"), g->eps, w, y, P, d, N, g->qkind, 0);
            if (rc != GH_EUNSUPPORTED) return rc;
            GHC(make_xb());
            return linear_any(g->xb, w, y, P, d, N, g->qkind);
        };
        if (g->lt[l] == 0) {
            if (mamba_mode == 0) {
                GHC(make_xb());
                // token by token, the reference's order (inference/generator.cpp:743-760)
                for (int t = 0; t < P; ++t) GHC(mamba_step(g, l, g->xb + (size_t)t * d, g->pr + (size_t)t * d));
            } else {
                const std::string mp = pre + "mamba.";
                // the residual add is folded into out_proj (x += ...)
                GHC(mamba_forward_impl(g->x, g->W(mp + "in_proj"), g->F(mp + "conv1d.weight"),
                                       g->F(mp + "conv1d.bias"), g->F(mp + "dt_bias"), g->F(mp + "A_log"),
                                       g->F(mp + "D"), g->F(mp + "norm.weight"), g->W(mp + "out_proj"), g->ssm[l],
                                       g->conv[l], acc ? g->x : g->pr, P, d, g->di, g->conv_dim, g->mh, g->mdh,
                                       g->mds, g->ck, g->eps, g->qkind, acc, g->F(pre + "attn_norm"), g->eps));
                if (!acc) GHC(add_branch(g, g->pr, (int64_t)P * d));
            }
        } else {
            // q, k, v in one launch with the norm as its row prologue and the fp16 KV-cache copies
            // of k and v in its epilogue (the cache starts at position 0); else one by one
            const void* wqkv[3] = {g->W(pre + "wq"), g->W(pre + "wk"), g->W(pre + "wv")};
            float* yqkv[3] = {g->q, g->k, g->v};
            uint16_t* y16[3] = {nullptr, g->kc[l], g->vc[l]};
            const int nqkv[3] = {g->qd, g->kvd, g->kvd};
            const int rc = linear_multi_skinny(g->x, 1, g->F(pre + "attn_norm"), g->eps, 3, wqkv, yqkv, y16, nqkv, P, d,
                                               g->qkind);
            if (rc != GH_EUNSUPPORTED) {
                GHC(rc);
            } else {
                GHC(proj_normed(wqkv[0], g->q, g->qd));
                GHC(proj_normed(wqkv[1], g->k, g->kvd));
                GHC(proj_normed(wqkv[2], g->v, g->kvd));
                GHC(launch_f32_to_f16(g->k, g->kc[l], (int64_t)P * g->kvd));
                GHC(launch_f32_to_f16(g->v, g->vc[l], (int64_t)P * g->kvd));
            }
            GHC(attention_prefill(g->q, g->k, g->v, g->att, 1, P, g->H, g->KV, g->hd, g->scale, 0));
            if (acc) {
                GHC(linear_acc(g->att, g->W(pre + "wo"), g->x, P, g->qd, d, g->qkind));  // x += attn W_o^T
            } else {
                GHC(linear_any(g->att, g->W(pre + "wo"), g->pr, P, g->qd, d, g->qkind));
                GHC(add_branch(g, g->pr, (int64_t)P * d));
            }
        }
        if (g->lt[l] == 0 && mamba_mode == 0) GHC(add_branch(g, g->pr, (int64_t)P * d));
        // x += moe(ffn_norm(x)): the norm rides on the router launch (normalised rows into xb); the
        // residual add on the combine launch when the path has one, else here
        int added = 0;
        GHC(moe_forward_acc(g->x, g->F(pre + "moe_router"), moe_bias(g, l), g->W(pre + "moe_gate"),
                            g->W(pre + "moe_up"), g->W(pre + "moe_down"), g->W(pre + "moe_sh_gate"),
                            g->W(pre + "moe_sh_up"), g->W(pre + "moe_sh_down"), g->pr, acc ? g->x : nullptr, &added, nullptr, nullptr, nullptr, P, d, g->E,
                            g->ne, g->K, g->SH, g->qkind, g->F(pre + "ffn_norm"), g->eps, g->xb));
        if (!added) GHC(add_branch(g, g->pr, (int64_t)P * d));
    }
    // cache length P, ring start 0 (KVCache::set_length), decode step 0: one small launch
    hipLaunchKernelGGL(k_ctl_prefilled, dim3(1), dim3(64), 0, stream(), g->ctl, P);
    GH_LAUNCHED("k_ctl_prefilled");
    g->host_len = P;
    // final norm of the last row + lm head: one launch (k_head_argmax without the pick) where it
    // fits and the logits are unscaled, else the norm and the head GEMV
    if (g->logits_scaling != 1.0f ||
        !launch_head_argmax(g->x + (size_t)(P - 1) * d, g->F("final_norm"), g->eps,
                            (const uint16_t*)g->W(g->head_name()), g->logits, d, g->V, g->ctl, nullptr, 0, false)) {
        GHC(gh_rmsnorm_forward(g->x + (size_t)(P - 1) * d, g->F("final_norm"), g->xb, nullptr, 1, d, g->eps));
        GHC(lm_head(g, g->xb));
    }
    if (logits_host) {
        GH_HIP(hipMemcpyAsync(logits_host, g->logits, (size_t)g->V * 4, hipMemcpyDeviceToHost, stream()));
    }
    GH_HIP(hipStreamSynchronize(stream()));
    return GH_OK;
}

int gh_granite_decode(gh_granite* g, int32_t token, float* logits_host) {
    GH_REQUIRE(g != nullptr, "granite_decode: null model");
    GH_REQUIRE(!g->state_invalid, "granite_decode: %s", STATE_INVALID_MSG);
    GH_HIP(hipMemcpyAsync(g->ctl + CTL_TOKEN, &token, 4, hipMemcpyHostToDevice, stream()));
    GHC(decode_step(g, false));
    g->host_len = g->host_len < g->max_ctx ? g->host_len + 1 : g->host_len;
    if (logits_host) GH_HIP(hipMemcpyAsync(logits_host, g->logits, (size_t)g->V * 4, hipMemcpyDeviceToHost, stream()));
    GH_HIP(hipStreamSynchronize(stream()));
    return GH_OK;
}

// The persistent decode loop's description of this model (host copy); buffers not set.
static PdModel pd_describe(gh_granite* g) {
    PdModel m;
    memset(&m, 0, sizeof m);
    m.L = g->L; m.d = g->d; m.V = g->V; m.H = g->H; m.KV = g->KV; m.hd = g->hd; m.E = g->E; m.ne = g->ne;
    m.K = g->K; m.SH = g->SH; m.di = g->di; m.mh = g->mh; m.mdh = g->mdh; m.mds = g->mds; m.ck = g->ck;
    m.kind = g->qkind; m.max_ctx = g->max_ctx; m.eps = g->eps; m.scale = g->scale;
    m.emb = pd_g((const uint16_t*)g->W("tok_embeddings"));
    m.final_norm = pd_g(g->F("final_norm"));
    for (int l = 0; l < g->L && l < PD_MAX_LAYERS; ++l) {
        const std::string pre = "layers." + std::to_string(l) + ".";
        PdLayer& y = m.layers[l];
        y.type = g->lt[l];
        y.attn_norm = pd_g(g->F(pre + "attn_norm"));
        y.ffn_norm = pd_g(g->F(pre + "ffn_norm"));
        if (y.type == 0) {
            const std::string mp = pre + "mamba.";
            y.in_proj = pd_g((const uint8_t*)g->W(mp + "in_proj"));
            y.conv_w = pd_g(g->F(mp + "conv1d.weight"));
            y.conv_b = pd_g(g->F(mp + "conv1d.bias"));
            y.dt_bias = pd_g(g->F(mp + "dt_bias"));
            y.a_log = pd_g(g->F(mp + "A_log"));
            y.Dp = pd_g(g->F(mp + "D"));
            y.gnorm_w = pd_g(g->F(mp + "norm.weight"));
            y.out_proj = pd_g((const uint8_t*)g->W(mp + "out_proj"));
            y.conv_state = pd_g(g->conv[l]);
            y.ssm_state = pd_g(g->ssm[l]);
        } else {
            y.wq = pd_g((const uint8_t*)g->W(pre + "wq"));
            y.wk = pd_g((const uint8_t*)g->W(pre + "wk"));
            y.wv = pd_g((const uint8_t*)g->W(pre + "wv"));
            y.wo = pd_g((const uint8_t*)g->W(pre + "wo"));
            y.kc = pd_g(g->kc[l]);
            y.vc = pd_g(g->vc[l]);
        }
        y.router = pd_g(g->F(pre + "moe_router"));
        y.gate = pd_g((const uint8_t*)g->W(pre + "moe_gate"));
        y.up = pd_g((const uint8_t*)g->W(pre + "moe_up"));
        y.down = pd_g((const uint8_t*)g->W(pre + "moe_down"));
        y.sh_gate = pd_g((const uint8_t*)g->W(pre + "moe_sh_gate"));
        y.sh_up = pd_g((const uint8_t*)g->W(pre + "moe_sh_up"));
        y.sh_down = pd_g((const uint8_t*)g->W(pre + "moe_sh_down"));
    }
    return m;
}

// n_steps decode steps (each: the token in ctl[CTL_TOKEN] -> greedy id recorded at
// gen_ids[step0 + i]) in one launch of the persistent loop. GH_EUNSUPPORTED (nothing
// launched) if the model or context does not fit it.
static int pd_generate(gh_granite* g, int step0, int n_steps) {
    PdModel m = pd_describe(g);
    const char* why = nullptr;
    if (!pd_supported(m, g->host_len, n_steps, &why)) return GH_EUNSUPPORTED;
    // hand-over buffers: tagged words, then keys, neg0 flags, counters
    const int conv_dim = g->di + 2 * g->mds;
    const size_t w_x = (size_t)g->d, w_proj = (size_t)g->di + conv_dim + g->mh, w_y = (size_t)g->di,
                 w_q = (size_t)g->H * g->hd, w_kv = (size_t)2 * g->KV * g->hd,
                 w_part = (size_t)g->H * PD_MAX_SPLITS * (g->hd + 2), w_act = (size_t)g->ne * g->E + g->SH,
                 w_route = (size_t)2 * g->K;
    // each vector in PD_REP replicas; the extra 64 words put consecutive replicas on
    // different memory channels
    auto stride = [](size_t words) { return (words + 31) / 32 * 32 + 64; };
    const size_t sizes[8] = {w_x, w_proj, w_y, w_q, w_kv, w_part, w_act, w_route};
    size_t tag_words = 0;
    for (size_t w : sizes) tag_words += stride(w) * PD_REP;
    const size_t bytes = tag_words * 8 + (size_t)g->max_ctx * 8 + (size_t)g->max_ctx * 4 + 256;
    if (!g->pd_buf) {
        GH_HIP(hipMalloc(&g->pd_buf, bytes));
        GH_HIP(hipMalloc(&g->pd_dev, sizeof(PdModel)));
        g->pd_zero_bytes = bytes;
    }
    uint64_t* t = (uint64_t*)g->pd_buf;
    PdBuf* bufs[8] = {&m.tx, &m.tproj, &m.ty, &m.tq, &m.tkv, &m.tpart, &m.tact, &m.troute};
    for (int i = 0; i < 8; ++i) {
        bufs[i]->p = pd_g(t);
        bufs[i]->stride = (int)stride(sizes[i]);
        t += stride(sizes[i]) * PD_REP;
    }
    m.tag_words = tag_words;
    m.keys = pd_g((unsigned long long*)t);
    m.neg0 = pd_g((int32_t*)((unsigned long long*)t + g->max_ctx));
    m.done = pd_g((uint32_t*)((int32_t*)((unsigned long long*)t + g->max_ctx) + g->max_ctx));
    int32_t* abort_flag = (int32_t*)((uint32_t*)((int32_t*)((unsigned long long*)t + g->max_ctx) + g->max_ctx) + 1);
    m.abort = pd_g(abort_flag);
    m.ctl = pd_g(g->ctl);
    m.gen_ids = pd_g(g->gen_ids);
    m.logits = pd_g(g->logits);
    GH_HIP(hipMemcpyAsync(g->pd_dev, &m, sizeof m, hipMemcpyHostToDevice, stream()));
    GH_HIP(hipMemsetAsync(g->pd_buf, 0, g->pd_zero_bytes, stream()));
    if (g->pd_force_abort) {
        // every wait that misses sees the flag and returns; the launch still runs to its end
        const int32_t one = 1;
        GH_HIP(hipMemcpyAsync(abort_flag, &one, 4, hipMemcpyHostToDevice, stream()));
        g->pd_force_abort = false;
    }
    GHC(pd_launch(m, g->pd_dev, g->host_len, step0, n_steps));
    int32_t aborted = 0;
    GH_HIP(hipMemcpyAsync(&aborted, abort_flag, 4, hipMemcpyDeviceToHost, stream()));
    GH_HIP(hipStreamSynchronize(stream()));
    if (aborted) {
        g->state_invalid = true;
        return fail(GH_EHIP, "persistent decode: a hand-over wait ran out (launch aborted); %s", STATE_INVALID_MSG);
    }
    return GH_OK;
}

int gh_granite_generate_greedy(gh_granite* g, int n_new, int32_t* ids_host, int use_graph) {
    GH_REQUIRE(g && ids_host && n_new >= 0, "granite_generate: bad arguments");
    GH_REQUIRE(!g->state_invalid, "granite_generate: %s", STATE_INVALID_MSG);
    GH_REQUIRE(g->host_len + n_new <= g->max_ctx, "granite_generate: %d + %d tokens exceed the context %d",
               g->host_len, n_new, g->max_ctx);
    if (n_new == 0) return GH_OK;
    const int32_t zero = 0;
    GH_HIP(hipMemcpyAsync(g->ctl + CTL_STEP, &zero, 4, hipMemcpyHostToDevice, stream()));
    // first id from the prefill logits
    GHC(launch_argmax(g->logits, g->V, g->ctl + CTL_TOKEN));
    hipLaunchKernelGGL(k_record_token, dim3(1), dim3(1), 0, stream(), g->ctl, g->gen_ids, g->max_ctx);
    int done = 1;
    // the persistent kernel implements the plain c1-style sequence (tied head, no router bias,
    // unit multipliers); other models decode through the graph
    const bool pd_model = g->tied && !g->aux_free && g->plain_multipliers() && g->logits_scaling == 1.0f;
    if (use_graph == 2 && n_new > 1 && pd_model) {
        // the whole loop in one persistent launch when the model fits it
        const int rc = pd_generate(g, 1, n_new - 1);
        if (rc == GH_OK) {
            GH_HIP(hipMemcpyAsync(ids_host, g->gen_ids, (size_t)n_new * 4, hipMemcpyDeviceToHost, stream()));
            GH_HIP(hipStreamSynchronize(stream()));
            g->host_len += n_new - 1;
            return GH_OK;
        }
        if (rc != GH_EUNSUPPORTED) return rc;
    }
    if (n_new > 1) {
        // one plain step (also sizes every workspace before a capture)
        GHC(decode_step(g, true));
        ++done;
    }
    if (use_graph >= 1 && done < n_new) {
        if (g->graph_exec && g->graph_ws_gen != workspace_generation()) {
            // a workspace buffer the graph reads or writes was replaced since the capture (a
            // larger prefill grew it): the captured addresses are stale, capture again
            GH_HIP(hipStreamSynchronize(stream()));
            (void)hipGraphExecDestroy(g->graph_exec);
            (void)hipGraphDestroy(g->graph);
            g->graph_exec = nullptr;
            g->graph = nullptr;
        }
        if (!g->graph_exec) {
            // Capture needs a non-null stream. When the backend stream is the null stream, the
            // capture runs on a stream the model owns and keeps until the graph is destroyed
            // (gh_granite_destroy), so no captured node can outlive the stream it was recorded on.
            hipStream_t s = stream();
            const bool own = s == nullptr;
            if (own) {
                if (!g->cap_stream) GH_HIP(hipStreamCreate(&g->cap_stream));
                s = g->cap_stream;
                GH_HIP(hipStreamSynchronize(nullptr));  // prior null-stream work before the capture
                gh_set_stream((void*)s);
            }
            GH_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            int rc = decode_step(g, true);
            hipGraph_t graph = nullptr;
            hipError_t e = hipStreamEndCapture(s, &graph);
            if (own) gh_set_stream(nullptr);
            if (rc) {
                if (graph) (void)hipGraphDestroy(graph);
                return rc;
            }
            if (e != hipSuccess) return fail(GH_EHIP, "decode graph capture: %s", hipGetErrorString(e));
            g->graph = graph;
            GH_HIP(hipGraphInstantiate(&g->graph_exec, graph, nullptr, nullptr, 0));
            g->graph_ws_gen = workspace_generation();
        }
        for (; done < n_new; ++done) GH_HIP(hipGraphLaunch(g->graph_exec, stream()));
    } else {
        for (; done < n_new; ++done) GHC(decode_step(g, true));
    }
    GH_HIP(hipMemcpyAsync(ids_host, g->gen_ids, (size_t)n_new * 4, hipMemcpyDeviceToHost, stream()));
    GH_HIP(hipStreamSynchronize(stream()));
    g->host_len += n_new - 1;
    return GH_OK;
}

}  // extern "C"
