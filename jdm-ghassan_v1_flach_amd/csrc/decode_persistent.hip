// The greedy decode loop of the Granite hybrid as ONE cooperative launch.
//
// The reference runs a decode step (inference/generator.cpp:221-443) as a
// sequence of ops, each its own kernel; the captured-graph path of this
// backend (granite.hip) fuses them into ~30 launches per token, which then
// cost more in launch and completion latency than in memory traffic (the c1
// model is 12 MB). Here one launch of co-resident blocks (hipLaunchCooperativeKernel)
// runs all n steps: per token, the sub-layers are phases of independent jobs
// (16-64 weight rows each, or one attention split, or the router), and every
// phase hands its outputs to the next through "tagged" words: a 64-bit word holds
// the fp32 value and the epoch (step x phase) that produced it, written and read
// at agent scope (global_store / global_load with sc1: through the non-coherent
// per-XCD L2s to the coherent memory side). A consumer spins on the words it needs
// until every one carries the expected epoch -- one memory round trip per
// hand-over instead of the three of a counter barrier (arrive, poll, then load).
// Every phase's jobs depend on all jobs of the phase before (each needs a whole
// vector), so a buffer is never overwritten before its last reader has read it.
// Weights are read-only and stay cached: the job -> block assignment is the same
// every token, so each XCD's L2 keeps its blocks' rows; a job requests its weight
// rows before it waits for its inputs. State that only one job touches (the
// Mamba conv window and SSM state rows, the argmax keys) uses ordinary accesses.
// Every wait is bounded: a wait that runs out sets an abort flag that every
// other wait checks, so all blocks leave and the host reports an error.
//
// Per token and layer: Mamba-2 [norm + in_proj + conv step] -> [state update]
// -> [gated norm + out_proj + residual]; attention [norm + q/k/v + cache store]
// -> [split attention partials] -> [merge + wo + residual]; MoE [norm + gate/up
// of every expert and the shared expert, router in its own job] -> [down of the
// selected experts + shared + ordered combine + residual]; then [final norm + tied
// lm head + argmax] whose key meets in a 64-bit atomicMax.
#include "decode_persistent.h"
#include "gemv_tasks.h"
#include "route.h"

namespace gh {

namespace {

constexpr int PD_T = 256;
constexpr int PD_SM = 8192;               // floats of the activation area
constexpr int PD_HD_MAX = 128;            // head_dim bound of the attention tiles
constexpr uint32_t PD_SPIN = 1u << 20;    // polls before a wait gives up (~1 s)
#ifndef PD_SLEEP
#define PD_SLEEP 1
#endif
constexpr int CTL_TOKEN = 0, CTL_LEN = 1, CTL_SLOT = 5, CTL_STEP = 6;
constexpr int PD_NW = 8;                  // norm weights per thread: vectors of at most 2048
// LDS pointers kept in structs stay LDS pointers (ds_* instructions, not flat ones)
#if defined(__HIP_DEVICE_COMPILE__)
#define PD_L __attribute__((address_space(3)))
#else
#define PD_L
#endif

// Activations as GEMV operands live in LDS padded by 4 floats per 64 (value k at
// k + 4 floor(k / 64)), so the lanes of a row, reading slices 64 values apart, hit distinct banks.
__device__ __forceinline__ int pd_padi(int k) { return k + ((k >> 6) << 2); }


__device__ __forceinline__ void tput1(PD_G uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// word i of a hand-over vector, into every replica
__device__ __forceinline__ void tput(const PdBuf& b, int i, float v, uint32_t tag) {
#pragma unroll
    for (int r = 0; r < PD_REP; ++r) tput1(b.p + (size_t)r * b.stride + i, v, tag);
}
// this block's replica of a hand-over vector, from word i
__device__ __forceinline__ const PD_G uint64_t* tsrc(const PdBuf& b, int i) {
    return b.p + (size_t)(blockIdx.x % PD_REP) * b.stride + i;
}

// A run of tagged words to wait for: n words at src, expected epoch tag, values to dst (LDS).
struct PdRange {
    const PD_G uint64_t* src;
    int n;
    uint32_t tag;
    PD_L float* dst;
};

// LDS staging of the polled words (16-byte chunks, filled by direct global -> LDS transfers).
constexpr int PD_STAGE = 4096;  // words

// Block-wide: once every word of the NR ranges carries its range's tag, the values are in
// their dst (LDS). A poll moves every chunk still missing straight into the LDS staging area
// (global_load_lds_dwordx4 with sc1: from the coherent memory side, no registers), all in
// flight at once, then each lane checks the chunks it moved; chunks that arrived complete are
// not requested again. Ranges start at even words (16-byte aligned). The chunks are taken in
// windows of at most PD_STAGE / 2 (the staging area's capacity), one window after the other,
// so any total fits. false if the launch is aborting.
#ifdef GH_PD_TRACE
__device__ uint32_t pd_last_spins;
#endif
constexpr int PD_WIN = PD_STAGE / 2;  // chunks per window
static_assert(PD_WIN / PD_T <= 32, "the per-lane done mask holds one bit per chunk slot");
template <int NR>
__device__ bool pd_wait_n(const PdRange (&r)[NR], PD_G int32_t* abort, PD_L uint64_t* stage) {
    __shared__ int s_abort;
    const int wave_base = threadIdx.x & ~63;
    int total = 0;
#pragma unroll
    for (int q = 0; q < NR; ++q) total += (r[q].n + 1) / 2;
    for (int base = 0; base < total; base += PD_WIN) {
        const int cnt = min(total - base, PD_WIN);
        const int nj = (cnt + PD_T - 1) / PD_T;  // <= PD_WIN / PD_T
        uint32_t done = 0;
        for (uint32_t spin = 0;; ++spin) {
            // request the missing chunks: chunk base + c, c = PD_T j + tid, lands at stage[2 c]
            for (int j = 0; j < nj; ++j) {
                const int c = PD_T * j + threadIdx.x;
                if (c < cnt && !((done >> j) & 1u)) {
                    int cc = base + c;
                    const PD_G uint64_t* g = nullptr;
#pragma unroll
                    for (int q = 0; q < NR; ++q) {
                        const int nq = (r[q].n + 1) / 2;
                        if (!g && cc < nq) g = r[q].src + 2 * cc;
                        else if (!g) cc -= nq;
                    }
                    const uint32_t lds = (uint32_t)(uintptr_t)(stage + 2 * (PD_T * j + wave_base));
                    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off sc1" ::"v"(g),
                                 "s"(__builtin_amdgcn_readfirstlane(lds))
                                 : "memory");
                }
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            int miss = 0;
            for (int j = 0; j < nj; ++j) {
                const int c = PD_T * j + threadIdx.x;
                if (c >= cnt || ((done >> j) & 1u)) continue;
                int cc = base + c;
                bool found = false, ok = true;
#pragma unroll
                for (int q = 0; q < NR; ++q) {
                    const int nq = (r[q].n + 1) / 2;
                    if (!found && cc < nq) {
                        found = true;
                        const int k = 2 * cc;
                        const uint64_t v0 = stage[2 * c], v1 = stage[2 * c + 1];
                        const bool two = k + 1 < r[q].n;
                        ok = (uint32_t)(v0 >> 32) == r[q].tag && (!two || (uint32_t)(v1 >> 32) == r[q].tag);
                        if (ok) {
                            r[q].dst[k] = __builtin_bit_cast(float, (uint32_t)v0);
                            if (two) r[q].dst[k + 1] = __builtin_bit_cast(float, (uint32_t)v1);
                        }
                    } else if (!found) {
                        cc -= nq;
                    }
                }
                if (ok) done |= 1u << j;
                else miss = 1;
            }
            // the barrier also keeps the next window's transfers behind every lane's reads
            if (!__syncthreads_or(miss)) {
#ifdef GH_PD_TRACE
                if (threadIdx.x == 0) __hip_atomic_store(&pd_last_spins, spin, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#endif
                break;
            }
            if (threadIdx.x == 0) {
                int a = __hip_atomic_load(abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (!a && spin >= PD_SPIN) {
                    __hip_atomic_store(abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    a = 1;
                }
                s_abort = a;
            }
            __syncthreads();
            if (s_abort) return false;
            __builtin_amdgcn_s_sleep(PD_SLEEP);
        }
    }
    return true;
}
__device__ bool pd_wait(const PD_G uint64_t* src, int n, uint32_t tag, PD_L float* dst, PD_G int32_t* abort,
                        PD_L uint64_t* stage) {
    const PdRange r[1] = {{src, n, tag, dst}};
    return pd_wait_n<1>(r, abort, stage);
}

// sx (padded) <- x * inv * w, inv = k_rmsnorm's statistic (double sum of squares; the sum
// over this thread's elements i = tid + 256 j, then the waves: k_rmsnorm's order, so the
// normalised row is bit-identical to the multi-kernel path). x (LDS): the thread's own
// elements need no barrier; wr: the thread's norm weights (pd_nw_load).
__device__ void pd_rmsnorm_pad(const PD_L float* x, int n, const float* wr, float eps, PD_L float* sx) {
    __shared__ double red[4];
    const int tid = threadIdx.x;
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < PD_NW; ++j) {
        const int i = tid + PD_T * j;
        if (i < n) ss += (double)x[i] * x[i];
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const double tot = red[0] + red[1] + red[2] + red[3];
    const double invd = 1.0 / sqrt(tot / (double)n + (double)eps);
    const float inv = isfinite(invd) ? (float)invd : 0.0f;
#pragma unroll
    for (int j = 0; j < PD_NW; ++j) {
        const int i = tid + PD_T * j;
        if (i < n) sx[pd_padi(i)] = x[i] * inv * wr[j];
    }
    __syncthreads();
}

// Mamba-2 gated norm (mamba.hip k_gated_norm) into sx (padded): rmsnorm(y * silu(z)) * w,
// y (LDS [n]) and z at y + n; double variance, float rsqrt.
__device__ void pd_gated_norm_pad(PD_L float* y, int n, const float* wr, float eps, PD_L float* sx) {
    __shared__ double red[4];
    const int tid = threadIdx.x;
    const PD_L float* z = y + n;
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < PD_NW; ++j) {
        const int i = tid + PD_T * j;
        if (i < n) {
            const float zv = z[i];
            const float v = y[i] * (zv / (1.0f + expf(-zv)));
            y[i] = v;
            ss += (double)v * v;
        }
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const double tot = red[0] + red[1] + red[2] + red[3];
    const float inv = 1.0f / sqrtf((float)(tot / (double)n) + eps);
#pragma unroll
    for (int j = 0; j < PD_NW; ++j) {
        const int i = tid + PD_T * j;
        if (i < n) sx[pd_padi(i)] = y[i] * inv * wr[j];
    }
    __syncthreads();
}

template <int KIND>
__device__ __forceinline__ size_t pd_rowb(int K) {
    if constexpr (KIND == KF16) return (size_t)K * 2;
    else return (size_t)(K / block_values(KIND)) * block_bytes(KIND);
}

// A lane's share of a weight row, a "slice": 32 values of a Q4_K or fp16 row (half of a 64-value
// task), or a whole 64-value Q8_0 task (two 34-byte blocks; halves would not be 4-byte aligned).
template <int KIND> struct Slice;
template <> struct Slice<3> { static constexpr int V = 32, DW = 8; };
template <> struct Slice<2> { static constexpr int V = 64, DW = 17; };
template <> struct Slice<KF16> { static constexpr int V = 32, DW = 16; };

// Slice s of a row into registers (cached loads: the rows stay in L2).
template <int KIND>
__device__ __forceinline__ void pd_load(const PD_G uint8_t* row, int s, uint32_t* w) {
    if constexpr (KIND == 3) {
        // task t = s / 2 (values 64 t ..), half h: qs bytes 16 h .. 16 h + 15 of the task's 32
        const int t = s >> 1, h = s & 1;
        const PD_G uint8_t* sb = row + (size_t)(t >> 2) * 144;
        const uint4 hd = *(const PD_G uint4*)sb;
        const uint4 q = *(const PD_G uint4*)(sb + 16 + 32 * (t & 3) + 16 * h);
        w[0] = hd.x; w[1] = hd.y; w[2] = hd.z; w[3] = hd.w;
        w[4] = q.x; w[5] = q.y; w[6] = q.z; w[7] = q.w;
    } else if constexpr (KIND == KF16) {
        const PD_G uint4* src = (const PD_G uint4*)(row + (size_t)s * 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 v = src[i];
            w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
        }
    } else {
        const PD_G uint32_t* src = (const PD_G uint32_t*)(row + (size_t)s * 68);
#pragma unroll
        for (int i = 0; i < 17; ++i) w[i] = src[i];
    }
}


// dst (padded) <- src[0..n) (unpadded LDS); block-wide.
__device__ __forceinline__ void pd_pad(const PD_L float* src, int n, PD_L float* dst) {
    for (int i = threadIdx.x; i < n; i += PD_T) dst[pd_padi(i)] = src[i];
    __syncthreads();
}

__device__ __forceinline__ void pd_ld16(const PD_L float* p, float* v) {
    const PD_L float4* q = (const PD_L float4*)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 a = q[i];
        v[4 * i] = a.x; v[4 * i + 1] = a.y; v[4 * i + 2] = a.z; v[4 * i + 3] = a.w;
    }
}

// The dot of slice s (loaded into w) with its activations in the padded operand sx.
template <int KIND>
__device__ __forceinline__ float pd_dot(const uint32_t* w, const PD_L float* sx, int s) {
    if constexpr (KIND == 3) {
#pragma clang fp contract(fast)
        const int t = s >> 1, h = s & 1;
        float xa[16], xb[16];
        pd_ld16(sx + 68 * t + 16 * h, xa);       // sub-block 2p,   values 16 h ..
        pd_ld16(sx + 68 * t + 32 + 16 * h, xb);  // sub-block 2p+1, values 16 h ..
        float sa = 0.f, sb = 0.f, qa = 0.f, qb = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = w[4 + i] & 0x0F0F0F0Fu, hi = (w[4 + i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                qa = fmaf(xa[4 * i + b], ub(lo, b), qa);
                qb = fmaf(xb[4 * i + b], ub(hi, b), qb);
                sa += xa[4 * i + b];
                sb += xb[4 * i + b];
            }
        }
        auto scb = [&](int i) { return (int)((w[1 + (i >> 2)] >> (8 * (i & 3))) & 0xFF); };
        auto scale_min = [&](int j, int& sc, int& m) {
            if (j < 4) {
                sc = scb(j) & 63;
                m = scb(j + 4) & 63;
            } else {
                sc = (scb(j + 4) & 0xF) | ((scb(j - 4) >> 6) << 4);
                m = (scb(j + 4) >> 4) | ((scb(j) >> 6) << 4);
            }
        };
        const int p = t & 3;
        int sc0, m0, sc1, m1;
        scale_min(2 * p, sc0, m0);
        scale_min(2 * p + 1, sc1, m1);
        const float d = f16_to_f32((uint16_t)(w[0] & 0xFFFF)), dmin = f16_to_f32((uint16_t)(w[0] >> 16));
        return d * ((float)sc0 * qa + (float)sc1 * qb) - dmin * ((float)m0 * sa + (float)m1 * sb);
    } else if constexpr (KIND == KF16) {
        const int t = s >> 1, h = s & 1;
        float x[32];
        pd_ld16(sx + 68 * t + 32 * h, x);
        pd_ld16(sx + 68 * t + 32 * h + 16, x + 16);
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            acc = fmaf(x[2 * i], f16_to_f32((uint16_t)(w[i] & 0xFFFF)), acc);
            acc = fmaf(x[2 * i + 1], f16_to_f32((uint16_t)(w[i] >> 16)), acc);
        }
        return acc;
    } else {
        float xv[64];
#pragma unroll
        for (int i = 0; i < 4; ++i) pd_ld16(sx + 68 * s + 16 * i, xv + 16 * i);
        float s2[2];
        task_xsum<KIND>(xv, s2);
        return task_dot<KIND>(w, xv, s2, s);
    }
}

// Norm weights of this thread's elements (i = tid + 256 j) into registers.
__device__ __forceinline__ void pd_nw_load(const PD_G float* __restrict__ w, int n, float* r) {
#pragma unroll
    for (int j = 0; j < PD_NW; ++j) {
        const int i = threadIdx.x + PD_T * j;
        if (i < n) r[j] = w[i];
    }
}

struct PdCtx {
    const PdModel* M;
    PD_G int32_t* abort;
    PD_L float* sm;       // LDS work area [PD_SM]
    PD_L float* sx;       // LDS padded GEMV operand [PD_SM / 64 * 68]
    PD_L float* xo;       // LDS residual rows of the current job [PD_T]
    PD_L uint64_t* stage; // LDS staging of polled tagged words [PD_STAGE]
    int token;       // the token of the current step
    uint32_t ex;     // epoch of the last residual-stream write this step (0: the embedding row)
    int t;           // step
    uint32_t ep0;    // epoch before the step's first phase
};

#ifdef GH_PD_TRACE
// Experiment builds only: thread 0 of each block stamps the real-time clock (100 MHz) at
// points of its first job in every phase of step PD_TRACE_STEP: [4 (phase) + 0] job start,
// + 1 inputs ready, + 2 outputs stored; event 127: the step's token known.
constexpr int PD_TRACE_STEP = 20, PD_TRACE_EV = 256;
__device__ uint64_t pd_trace[256][PD_TRACE_EV];
#define PD_SUB(c, ep, sub, j)                                                                             \
    do {                                                                                                  \
        const int ev_ = 8 * (int)((ep) - (c).ep0 - 1) + (sub);                                           \
        if ((c).t == PD_TRACE_STEP && threadIdx.x == 0 && (j) == (int)blockIdx.x && blockIdx.x < 256 &&    \
            ev_ < PD_TRACE_EV)                                                                            \
            pd_trace[blockIdx.x][ev_] = __builtin_amdgcn_s_memrealtime();                               \
    } while (0)
#else
#define PD_SUB(c, ep, sub, j) \
    do {                      \
    } while (0)
#endif

// The residual-stream wait of a job as a range (n = 0 when the stream is the embedding row,
// which pd_emb_rows / pd_emb_x read directly).
__device__ __forceinline__ PdRange pd_x_range(const PdCtx& c, int r0, int n, PD_L float* dst) {
    return PdRange{tsrc(c.M->tx, r0), c.ex ? n : 0, c.ex, dst};
}
__device__ __forceinline__ float pd_emb(const PdCtx& c, int i) {
    const PdModel& M = *c.M;
    return (c.token < 0 || c.token >= M.V) ? 0.f : f16_to_f32(M.emb[(size_t)c.token * M.d + i]);
}
// The whole residual stream into dst when it is the embedding row (block-wide; no-op otherwise).
__device__ __forceinline__ void pd_emb_x(const PdCtx& c, PD_L float* dst) {
    if (c.ex) return;
    for (int i = threadIdx.x; i < c.M->d; i += PD_T) dst[i] = pd_emb(c, i);
    __syncthreads();
}
// Rows [r0, r0 + n) of the residual stream into xo when it is the embedding row.
__device__ __forceinline__ void pd_emb_rows(const PdCtx& c, int r0, int n) {
    if (c.ex) return;
    for (int i = threadIdx.x; i < n; i += PD_T) c.xo[i] = r0 + i < c.M->d ? pd_emb(c, r0 + i) : 0.f;
    __syncthreads();
}

// Rows per job of a one-slice-per-lane GEMV over K inputs.
template <int KIND>
__device__ __forceinline__ int pd_rpj(int K) { return PD_T / (K / Slice<KIND>::V); }

// ---------------------------------------------------------------- phases
// Mamba-2 [norm + in_proj + conv step + SiLU]: rows z | xBC | dt of in_proj.
template <int KIND>
__device__ bool ph_mamba_in(PdCtx& c, const PdLayer& Ly, uint32_t ep) {
    const PdModel& M = *c.M;
    const int d = M.d, conv_dim = M.di + 2 * M.mds, proj = M.di + conv_dim + M.mh;
    const int LPR = d / Slice<KIND>::V, rpj = PD_T / LPR, jobs = cdiv(proj, rpj);
    const size_t rowb = pd_rowb<KIND>(d);
    for (int j = blockIdx.x; j < jobs; j += gridDim.x) {
        PD_SUB(c, ep, 0, j);
        const int sub = threadIdx.x % LPR, r = j * rpj + threadIdx.x / LPR;
        const int rr = r < proj ? r : proj - 1;
        uint32_t w[Slice<KIND>::DW];
        pd_load<KIND>(Ly.in_proj + (size_t)rr * rowb, sub, w);
        float nw[PD_NW];
        pd_nw_load(Ly.attn_norm, d, nw);
        // the conv operands of an xBC row, requested with the weights
        const bool conv = sub == 0 && r >= M.di && r < M.di + conv_dim;
        const int ch = r - M.di, wl = M.ck - 1;
        float cw[8], win[8], cb = 0.f;
        if (conv) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                if (q <= wl) cw[q] = Ly.conv_w[(size_t)ch * M.ck + q];
                if (q < wl) win[q] = Ly.conv_state[(size_t)ch * wl + q];
            }
            cb = Ly.conv_b ? Ly.conv_b[ch] : 0.0f;
        }
        const PdRange rg[1] = {pd_x_range(c, 0, d, c.sm)};
        if (!pd_wait_n<1>(rg, c.abort, c.stage)) return false;
        pd_emb_x(c, c.sm);
        pd_rmsnorm_pad(c.sm, d, nw, M.eps, c.sx);
        PD_SUB(c, ep, 1, j);
        float v = pd_dot<KIND>(w, c.sx, sub);
        v = group_sum(v, LPR);
        if (sub == 0 && r < proj) {
            float out = v;
            if (conv) {
#pragma clang fp contract(off)
                float acc = cb;
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    if (q < wl) acc += cw[q] * win[q];
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    if (q == wl) acc += cw[q] * v;
                PD_G float* ws = Ly.conv_state + (size_t)ch * wl;
#pragma unroll
                for (int q = 0; q < 7; ++q)
                    if (q + 1 < wl) ws[q] = win[q + 1];
                if (wl > 0) ws[wl - 1] = v;
                out = acc / (1.0f + expf(-acc));
            }
            tput(M.tproj, r, out, ep);
        }
        PD_SUB(c, ep, 2, j);
        __syncthreads();
    }
    return true;
}

// Mamba-2 single-token state update (mamba.hip k_step_scan arithmetic): job = (head, rows).
__device__ bool ph_mamba_scan(PdCtx& c, const PdLayer& Ly, uint32_t ep_in, uint32_t ep) {
    const PdModel& M = *c.M;
    const int N = M.mds, P = M.mdh, di = M.di;
    const int TPR = N / 8, ROWS = PD_T / TPR, cpj = cdiv(P, ROWS), jobs = M.mh * cpj;
    PD_L float* sm = c.sm;
    for (int j = blockIdx.x; j < jobs; j += gridDim.x) {
        PD_SUB(c, ep, 0, j);
        const int h = j / cpj, r0 = (j % cpj) * ROWS;
        const int nr = min(ROWS, P - r0);
        const int tr = threadIdx.x / TPR, tc = threadIdx.x % TPR, p = r0 + tr;
        const int i = h * P + p;
        const bool act = tr < nr;
        float s[8];
        if (act) {
            const PD_G float4* sp = (const PD_G float4*)(Ly.ssm_state + (size_t)i * N + tc * 8);
            const float4 a = sp[0], b = sp[1];
            s[0] = a.x; s[1] = a.y; s[2] = a.z; s[3] = a.w; s[4] = b.x; s[5] = b.y; s[6] = b.z; s[7] = b.w;
        }
        const float a_log = Ly.a_log[h], dt_b = Ly.dt_bias[h], Dh = Ly.Dp[h];
        // x rows of this job, B | C, and the head's raw dt
        const PdRange rg[3] = {{tsrc(M.tproj, di + h * P + r0), nr, ep_in, sm},
                               {tsrc(M.tproj, 2 * di), 2 * N, ep_in, sm + 256},
                               {tsrc(M.tproj, 2 * di + 2 * N), M.mh, ep_in, sm + 512}};
        if (!pd_wait_n<3>(rg, c.abort, c.stage)) return false;
        PD_SUB(c, ep, 1, j);
        const float a = -expf(a_log);
        const float dtb = sm[512 + h] + dt_b;
        const float dt = (dtb > 20.0f) ? dtb : log1pf(expf(dtb));
        const float dA = expf(a * dt);
        const float xv = act ? sm[tr] : 0.f;
        const PD_L float* Bm = sm + 256;
        const PD_L float* Cm = Bm + N;
        float acc = 0.f;
        if (act) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int n = tc * 8 + q;
                s[q] = dA * s[q] + (Bm[n] * dt) * xv;
                acc = fmaf(Cm[n], s[q], acc);
            }
            PD_G float4* sp = (PD_G float4*)(Ly.ssm_state + (size_t)i * N + tc * 8);
            sp[0] = make_float4(s[0], s[1], s[2], s[3]);
            sp[1] = make_float4(s[4], s[5], s[6], s[7]);
        }
        acc = group_sum(acc, TPR);
        if (act && tc == 0) tput(M.ty, i, acc + Dh * xv, ep);
        PD_SUB(c, ep, 2, j);
        __syncthreads();
    }
    return true;
}

// Mamba-2 [gated norm + out_proj + residual]: x[r] += (W_out rmsnorm(y silu(z)) w)[r].
template <int KIND>
__device__ bool ph_mamba_out(PdCtx& c, const PdLayer& Ly, uint32_t ep_z, uint32_t ep_y, uint32_t ep) {
    const PdModel& M = *c.M;
    const int d = M.d, K = M.di, LPR = K / Slice<KIND>::V, rpj = PD_T / LPR, jobs = cdiv(d, rpj);
    const size_t rowb = pd_rowb<KIND>(K);
    for (int j = blockIdx.x; j < jobs; j += gridDim.x) {
        PD_SUB(c, ep, 0, j);
        const int r0 = j * rpj, sub = threadIdx.x % LPR, r = r0 + threadIdx.x / LPR;
        const int rr = r < d ? r : d - 1;
        uint32_t w[Slice<KIND>::DW];
        pd_load<KIND>(Ly.out_proj + (size_t)rr * rowb, sub, w);
        float nw[PD_NW];
        pd_nw_load(Ly.gnorm_w, K, nw);
        const PdRange rg[3] = {{tsrc(M.ty, 0), K, ep_y, c.sm}, {tsrc(M.tproj, 0), K, ep_z, c.sm + K},
                               pd_x_range(c, r0, min(rpj, d - r0), c.xo)};
        if (!pd_wait_n<3>(rg, c.abort, c.stage)) return false;
        PD_SUB(c, ep, 3, j);
#ifdef GH_PD_TRACE
        if (c.t == PD_TRACE_STEP && threadIdx.x == 0 && j == (int)blockIdx.x) pd_trace[blockIdx.x][8 * (int)(ep - c.ep0 - 1) + 7] = pd_last_spins;
#endif
        pd_emb_rows(c, r0, min(rpj, d - r0));
        PD_SUB(c, ep, 4, j);
        pd_gated_norm_pad(c.sm, K, nw, M.eps, c.sx);
        PD_SUB(c, ep, 1, j);
        float v = pd_dot<KIND>(w, c.sx, sub);
        v = group_sum(v, LPR);
        if (sub == 0 && r < d) tput(M.tx, r, c.xo[r - r0] + v, ep);
        PD_SUB(c, ep, 2, j);
        __syncthreads();
    }
    return true;
}

// Attention [norm + q | k | v]: k and v go to the cache slot as fp16 and, rounded the same
// way, to the tagged hand-over for this step's attention jobs.
template <int KIND>
__device__ bool ph_attn_qkv(PdCtx& c, const PdLayer& Ly, int slot, uint32_t ep) {
    const PdModel& M = *c.M;
    const int d = M.d, qd = M.H * M.hd, kvd = M.KV * M.hd, rows = qd + 2 * kvd;
    const int LPR = d / Slice<KIND>::V, rpj = PD_T / LPR, jobs = cdiv(rows, rpj);
    const size_t rowb = pd_rowb<KIND>(d);
    for (int j = blockIdx.x; j < jobs; j += gridDim.x) {
        PD_SUB(c, ep, 0, j);
        const int sub = threadIdx.x % LPR, r = j * rpj + threadIdx.x / LPR;
        const int rr = r < rows ? r : rows - 1;
        const PD_G uint8_t* row = rr < qd ? Ly.wq + (size_t)rr * rowb
                             : rr < qd + kvd ? Ly.wk + (size_t)(rr - qd) * rowb
                                             : Ly.wv + (size_t)(rr - qd - kvd) * rowb;
        uint32_t w[Slice<KIND>::DW];
        pd_load<KIND>(row, sub, w);
        float nw[PD_NW];
        pd_nw_load(Ly.attn_norm, d, nw);
        const PdRange rg[1] = {pd_x_range(c, 0, d, c.sm)};
        if (!pd_wait_n<1>(rg, c.abort, c.stage)) return false;
        pd_emb_x(c, c.sm);
        pd_rmsnorm_pad(c.sm, d, nw, M.eps, c.sx);
        PD_SUB(c, ep, 1, j);
        float v = pd_dot<KIND>(w, c.sx, sub);
        v = group_sum(v, LPR);
        if (sub == 0 && r < rows) {
            if (r < qd) {
                tput(M.tq, r, v, ep);
            } else {
                const int cix = r - qd;  // [0, 2 kvd): k then v
                const uint16_t h16 = f32_to_f16(v);
                PD_G uint16_t* cache = cix < kvd ? Ly.kc : Ly.vc;
                const int cc = cix < kvd ? cix : cix - kvd;
                __hip_atomic_store(cache + (size_t)slot * kvd + cc, h16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                tput(M.tkv, cix, f16_to_f32(h16), ep);
            }
        }
        PD_SUB(c, ep, 2, j);
        __syncthreads();
    }
    return true;
}

// Attention partials: job = (kv head, run of PD_POS positions); wave g < G takes q head
// kvh * G + g, lane = position. Writes (o[hd], running max, sum) per head and split.
// K / V tile rows are padded by 2 halves so the lanes of a score read distinct banks.
constexpr int PD_KS = PD_HD_MAX + 2;
__device__ bool ph_attn_part(PdCtx& c, const PdLayer& Ly, int len, uint32_t ep_in, uint32_t ep, PD_L uint16_t* kt,
                             PD_L uint16_t* vt) {
    const PdModel& M = *c.M;
    const int hd = M.hd, G = M.H / M.KV, kvd = M.KV * hd, total = len + 1;
    const int nsplit = cdiv(total, PD_POS), jobs = M.KV * nsplit, hw = hd / 2;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    PD_L float* sm = c.sm;
    for (int j = blockIdx.x; j < jobs; j += gridDim.x) {
        PD_SUB(c, ep, 0, j);
        const int kvh = j / nsplit, s = j % nsplit;
        const int p0 = s * PD_POS, np = min(PD_POS, total - p0);
        const bool has_new = p0 + np == total;  // the new token's position is in this run
        // cached rows of this run (written by earlier steps' jobs or the prefill)
        const int nold = has_new ? np - 1 : np;
        for (int e = threadIdx.x; e < nold * hw; e += PD_T) {
            const int jp = e / hw, q = e % hw;
            const size_t off = (size_t)(p0 + jp) * kvd + (size_t)kvh * hd + 2 * q;
            const uint32_t kw = __hip_atomic_load((PD_G uint32_t*)(Ly.kc + off), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint32_t vw = __hip_atomic_load((PD_G uint32_t*)(Ly.vc + off), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ((PD_L uint32_t*)kt)[jp * (PD_KS / 2) + q] = kw;
            ((PD_L uint32_t*)vt)[jp * (PD_KS / 2) + q] = vw;
        }
        const PdRange rg[3] = {{tsrc(M.tq, (size_t)kvh * G * hd), G * hd, ep_in, sm},
                               {tsrc(M.tkv, (size_t)kvh * hd), has_new ? hd : 0, ep_in, sm + G * hd},
                               {tsrc(M.tkv, kvd + (size_t)kvh * hd), has_new ? hd : 0, ep_in, sm + G * hd + hd}};
        if (!pd_wait_n<3>(rg, c.abort, c.stage)) return false;
        if (has_new) {
            for (int q = threadIdx.x; q < hd; q += PD_T) {
                kt[(np - 1) * PD_KS + q] = f32_to_f16(sm[G * hd + q]);
                vt[(np - 1) * PD_KS + q] = f32_to_f16(sm[G * hd + hd + q]);
            }
        }
        __syncthreads();
        PD_SUB(c, ep, 1, j);
        if (wave < G) {
            const PD_L float* qv = sm + wave * hd;
            float sc = -INFINITY;
            if (lane < np) {
                float acc = 0.f;
                const PD_L uint32_t* kr = (const PD_L uint32_t*)(kt + lane * PD_KS);
                for (int q = 0; q < hw; ++q) {
                    const uint32_t kk = kr[q];
                    acc = fmaf(qv[2 * q], f16_to_f32((uint16_t)(kk & 0xFFFF)), acc);
                    acc = fmaf(qv[2 * q + 1], f16_to_f32((uint16_t)(kk >> 16)), acc);
                }
                sc = acc * M.scale;
            }
            const float mx = wave_max(sc);
            const float pv = lane < np ? expf(sc - mx) : 0.f;
            const float l = wave_sum(pv);
            float o0 = 0.f, o1 = 0.f;
            for (int jp = 0; jp < np; ++jp) {
                const float pj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv), jp));
                o0 = fmaf(pj, f16_to_f32(vt[jp * PD_KS + lane]), o0);
                if (hd > 64) o1 = fmaf(pj, f16_to_f32(vt[jp * PD_KS + 64 + lane]), o1);
            }
            const int h = kvh * G + wave;
            const int base = (h * nsplit + s) * (hd + 2);
            tput(M.tpart, base + lane, o0, ep);
            if (hd > 64) tput(M.tpart, base + 64 + lane, o1, ep);
            if (lane == 0) {
                tput(M.tpart, base + hd, mx, ep);
                tput(M.tpart, base + hd + 1, l, ep);
            }
        }
        PD_SUB(c, ep, 2, j);
        __syncthreads();
    }
    return true;
}

// Attention [merge of the partials + wo + residual].
template <int KIND>
__device__ bool ph_attn_out(PdCtx& c, const PdLayer& Ly, int len, uint32_t ep_in, uint32_t ep) {
    const PdModel& M = *c.M;
    const int d = M.d, hd = M.hd, H = M.H, K = H * hd, nsplit = cdiv(len + 1, PD_POS);
    const int LPR = K / Slice<KIND>::V, rpj = PD_T / LPR, jobs = cdiv(d, rpj);
    const size_t rowb = pd_rowb<KIND>(K);
    PD_L float* part = c.sm + K;
    for (int j = blockIdx.x; j < jobs; j += gridDim.x) {
        PD_SUB(c, ep, 0, j);
        const int r0 = j * rpj, sub = threadIdx.x % LPR, r = r0 + threadIdx.x / LPR;
        const int rr = r < d ? r : d - 1;
        uint32_t w[Slice<KIND>::DW];
        pd_load<KIND>(Ly.wo + (size_t)rr * rowb, sub, w);
        const PdRange rg[2] = {{tsrc(M.tpart, 0), H * nsplit * (hd + 2), ep_in, part},
                               pd_x_range(c, r0, min(rpj, d - r0), c.xo)};
        if (!pd_wait_n<2>(rg, c.abort, c.stage)) return false;
        pd_emb_rows(c, r0, min(rpj, d - r0));
        for (int e = threadIdx.x; e < K; e += PD_T) {
            const int h = e / hd, q = e % hd;
            const PD_L float* ph = part + (size_t)h * nsplit * (hd + 2);
            float mx = -INFINITY;
            for (int sp = 0; sp < nsplit; ++sp) mx = fmaxf(mx, ph[sp * (hd + 2) + hd]);
            float L = 0.f, o = 0.f;
            for (int sp = 0; sp < nsplit; ++sp) {
                const PD_L float* pp = ph + sp * (hd + 2);
                const float f = pp[hd] == -INFINITY ? 0.f : expf(pp[hd] - mx);
                L += pp[hd + 1] * f;
                o += pp[q] * f;
            }
            c.sx[pd_padi(e)] = L > 0.f ? o * (1.0f / L) : 0.f;
        }
        __syncthreads();
        PD_SUB(c, ep, 1, j);
        float v = pd_dot<KIND>(w, c.sx, sub);
        v = group_sum(v, LPR);
        if (sub == 0 && r < d) tput(M.tx, r, c.xo[r - r0] + v, ep);
        PD_SUB(c, ep, 2, j);
        __syncthreads();
    }
    return true;
}

// MoE [norm + gate/up + SwiGLU of every expert and the shared expert]; job 0 routes.
template <int KIND>
__device__ bool ph_moe_up(PdCtx& c, const PdLayer& Ly, uint32_t ep, PD_L float* term) {
    const PdModel& M = *c.M;
    const int d = M.d, LPR = d / Slice<KIND>::V, rpj = PD_T / LPR;
    const int rows = M.ne * M.E + M.SH, jobs = 1 + cdiv(rows, rpj);
    const size_t rowb = pd_rowb<KIND>(d);
    __shared__ int sel[8];
    __shared__ float wsel[8];
    for (int j = blockIdx.x; j < jobs; j += gridDim.x) {
        PD_SUB(c, ep, 0, j);
        float nw[PD_NW];
        pd_nw_load(Ly.ffn_norm, d, nw);
        if (j == 0) {
            const PdRange rg[1] = {pd_x_range(c, 0, d, c.sm)};
            if (!pd_wait_n<1>(rg, c.abort, c.stage)) return false;
            pd_emb_x(c, c.sm);
            pd_rmsnorm_pad(c.sm, d, nw, M.eps, c.sx);
            for (int i = threadIdx.x; i < d; i += PD_T) c.sm[i] = c.sx[pd_padi(i)];
            __syncthreads();
            const int GW = min(d / 4, (PD_POS * PD_KS / 2) / M.ne - 1);
            route_token(c.sm, Ly.router, nullptr, nullptr, nullptr, nullptr, d, M.ne, M.K, nullptr, 0.f, nullptr, GW,
                        0, c.sm, term, sel, wsel);
            if (threadIdx.x < M.K) {
                tput(M.troute, threadIdx.x, (float)sel[threadIdx.x], ep);
                tput(M.troute, M.K + threadIdx.x, wsel[threadIdx.x], ep);
            }
            __syncthreads();
            continue;
        }
        const int sub = threadIdx.x % LPR, r = (j - 1) * rpj + threadIdx.x / LPR;
        const int rr = r < rows ? r : rows - 1;
        const PD_G uint8_t *rg_, *ru;
        if (rr < M.ne * M.E) {
            rg_ = Ly.gate + (size_t)rr * rowb;
            ru = Ly.up + (size_t)rr * rowb;
        } else {
            rg_ = Ly.sh_gate + (size_t)(rr - M.ne * M.E) * rowb;
            ru = Ly.sh_up + (size_t)(rr - M.ne * M.E) * rowb;
        }
        uint32_t wg[Slice<KIND>::DW], wu[Slice<KIND>::DW];
        pd_load<KIND>(rg_, sub, wg);
        pd_load<KIND>(ru, sub, wu);
        const PdRange rg[1] = {pd_x_range(c, 0, d, c.sm)};
        if (!pd_wait_n<1>(rg, c.abort, c.stage)) return false;
        PD_SUB(c, ep, 3, j);
        pd_emb_x(c, c.sm);
        pd_rmsnorm_pad(c.sm, d, nw, M.eps, c.sx);
        PD_SUB(c, ep, 4, j);
        PD_SUB(c, ep, 1, j);
        float g = pd_dot<KIND>(wg, c.sx, sub);
        float u = pd_dot<KIND>(wu, c.sx, sub);
        PD_SUB(c, ep, 5, j);
        g = group_sum(g, LPR);
        u = group_sum(u, LPR);
        PD_SUB(c, ep, 6, j);
        if (sub == 0 && r < rows) tput(M.tact, r, g / (1.0f + expf(-g)) * u, ep);
        PD_SUB(c, ep, 2, j);
        __syncthreads();
    }
    return true;
}

// MoE [down of the shared and the selected experts + combine + residual]: row r's lanes
// hold the tasks of shared down row r (SH inputs), then of each selected expert's down row
// (E inputs each); the combine is shared + w_0 y_0 + w_1 y_1 + ... (moe.hip k_moe_down_par).
template <int KIND>
__device__ bool ph_moe_down(PdCtx& c, const PdLayer& Ly, uint32_t ep_in, uint32_t ep, PD_L float* tdot) {
    const PdModel& M = *c.M;
    const int d = M.d, E = M.E, SH = M.SH, K = M.K;
    const int ts = SH / Slice<KIND>::V, te = E / Slice<KIND>::V, LPR = ts + K * te, rpj = PD_T / LPR, jobs = cdiv(d, rpj);
    const size_t rowb_s = pd_rowb<KIND>(SH), rowb_e = pd_rowb<KIND>(E);
    __shared__ float rsel[16];
    PD_L float* sm = c.sm;
    for (int j = blockIdx.x; j < jobs; j += gridDim.x) {
        PD_SUB(c, ep, 0, j);
        const int r0 = j * rpj, nrow = min(rpj, d - r0);
        const int sub = threadIdx.x % LPR, rl = threadIdx.x / LPR, r = r0 + rl;
        const int rr = r < d ? r : d - 1;
        const bool active = threadIdx.x < rpj * LPR;
        int seg = 0, t = sub;
        if (sub >= ts) {
            seg = 1 + (sub - ts) / te;
            t = (sub - ts) % te;
        }
        // the shared expert's rows and the residual rows first (independent of the routing)
        uint32_t w[Slice<KIND>::DW];
        if (active && seg == 0) pd_load<KIND>(Ly.sh_down + (size_t)rr * rowb_s, t, w);
        {
            const PdRange rg[2] = {{tsrc(M.troute, 0), 2 * K, ep_in, (PD_L float*)rsel}, pd_x_range(c, r0, nrow, c.xo)};
            if (!pd_wait_n<2>(rg, c.abort, c.stage)) return false;
        }
        pd_emb_rows(c, r0, nrow);
        if (active && seg > 0) pd_load<KIND>(Ly.down + ((size_t)(int)rsel[seg - 1] * d + rr) * rowb_e, t, w);
        // activations: shared expert, then each selected expert
        if (K == 2) {
            const PdRange rg[3] = {{tsrc(M.tact, (size_t)M.ne * E), SH, ep_in, sm},
                                   {tsrc(M.tact, (size_t)(int)rsel[0] * E), E, ep_in, sm + SH},
                                   {tsrc(M.tact, (size_t)(int)rsel[1] * E), E, ep_in, sm + SH + E}};
            if (!pd_wait_n<3>(rg, c.abort, c.stage)) return false;
        } else {
            if (!pd_wait(tsrc(M.tact, (size_t)M.ne * E), SH, ep_in, sm, c.abort, c.stage)) return false;
            for (int k = 0; k < K; ++k)
                if (!pd_wait(tsrc(M.tact, (size_t)(int)rsel[k] * E), E, ep_in, sm + SH + k * E, c.abort, c.stage)) return false;
        }
        pd_pad(sm, SH + K * E, c.sx);
        PD_SUB(c, ep, 1, j);
        if (active) {
            const int o64 = seg == 0 ? 0 : (SH + (seg - 1) * E) / 64;  // segment start in 64-value units
            tdot[rl * LPR + sub] = pd_dot<KIND>(w, c.sx + 68 * o64, t);
        }
        __syncthreads();
        if (threadIdx.x < nrow) {
            const int row = r0 + threadIdx.x;
            const PD_L float* td = tdot + threadIdx.x * LPR;
            float acc = 0.f;
            for (int q = 0; q < ts; ++q) acc += td[q];
            for (int k = 0; k < K; ++k) {
                float y = 0.f;
                for (int q = 0; q < te; ++q) y += td[ts + k * te + q];
                acc += rsel[K + k] * y;
            }
            tput(M.tx, row, c.xo[threadIdx.x] + acc, ep);
        }
        PD_SUB(c, ep, 2, j);
        __syncthreads();
    }
    return true;
}

// Argmax key of logit v at index i (granite.hip amax_key: first finite maximum, lower index on
// ties, -0 == +0; +inf only above "none", NaN / -inf none).
__device__ __forceinline__ uint64_t pd_key(float v, int i) {
    const uint32_t lo = ~(uint32_t)i;
    if (v == __builtin_inff()) return lo;
    if (!isfinite(v)) return 0;
    const uint32_t u = __builtin_bit_cast(uint32_t, v == 0.f ? 0.f : v);
    const uint32_t hi = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)hi << 32) | lo;
}

// [final norm + tied fp16 lm head + argmax]: each job's best key meets the others in
// keys[step] (atomicMax), then the job counts itself done.
__device__ bool ph_head(PdCtx& c, int step, uint32_t ep) {
    const PdModel& M = *c.M;
    const int d = M.d, V = M.V, LPR = d / Slice<KF16>::V, rpj = PD_T / LPR, jobs = cdiv(V, rpj);
    __shared__ unsigned long long bkey[4];
    for (int j = blockIdx.x; j < jobs; j += gridDim.x) {
        PD_SUB(c, ep, 0, j);
        const int sub = threadIdx.x % LPR, r = j * rpj + threadIdx.x / LPR;
        const int rr = r < V ? r : V - 1;
        uint32_t w[Slice<KF16>::DW];
        pd_load<KF16>((const PD_G uint8_t*)(M.emb + (size_t)rr * d), sub, w);
        float nw[PD_NW];
        pd_nw_load(M.final_norm, d, nw);
        const PdRange rg[1] = {pd_x_range(c, 0, d, c.sm)};
        if (!pd_wait_n<1>(rg, c.abort, c.stage)) return false;
        pd_emb_x(c, c.sm);
        pd_rmsnorm_pad(c.sm, d, nw, M.eps, c.sx);
        PD_SUB(c, ep, 1, j);
        float v = pd_dot<KF16>(w, c.sx, sub);
        v = group_sum(v, LPR);
        uint64_t key = 0;
        if (sub == 0 && r < V) {
            M.logits[r] = v;
            key = pd_key(v, r);
            if (r == 0 && v == -__builtin_inff()) {
                (void)__hip_atomic_fetch_or(M.neg0 + step, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): performed before the job counts itself done
            }
        }
        // block maximum of the keys
        uint32_t hi = (uint32_t)(key >> 32), lo = (uint32_t)key;
        for (int o = 32; o >= 1; o >>= 1) {
            const uint32_t oh = __shfl_xor(hi, o, 64), ol = __shfl_xor(lo, o, 64);
            if (oh > hi || (oh == hi && ol > lo)) { hi = oh; lo = ol; }
        }
        if ((threadIdx.x & 63) == 0) bkey[threadIdx.x >> 6] = ((uint64_t)hi << 32) | lo;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long k = bkey[0];
            for (int q = 1; q < 4; ++q) k = bkey[q] > k ? bkey[q] : k;
            if (k) {
                (void)__hip_atomic_fetch_max(M.keys + step, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __builtin_amdgcn_s_waitcnt(0x0F70);
            }
            (void)__hip_atomic_fetch_add(M.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        PD_SUB(c, ep, 2, j);
        __syncthreads();
    }
    return true;
}

// The greedy id of `step` once all its lm-head jobs are done (every thread gets it); -1 if
// aborting.
__device__ int pd_token(const PdCtx& c, int step, int head_jobs) {
    const PdModel& M = *c.M;
    __shared__ int s_tok;
    if (threadIdx.x == 0) {
        const uint32_t need = (uint32_t)(step + 1) * (uint32_t)head_jobs;
        int tok = -1;
        for (uint32_t spin = 0;; ++spin) {
            if (__hip_atomic_load(M.done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= need) {
                const uint64_t fin = __hip_atomic_load(M.keys + step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const int neg0 = __hip_atomic_load(M.neg0 + step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                tok = 0;
                if (fin >> 32) tok = (int)~(uint32_t)fin;        // finite maximum
                else if (fin && neg0) tok = (int)~(uint32_t)fin;  // no finite value: first +inf after l[0] = -inf
                break;
            }
            if ((spin & 255) == 255) {
                if (__hip_atomic_load(c.abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
                if (spin >= PD_SPIN) {
                    __hip_atomic_store(c.abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
            }
            __builtin_amdgcn_s_sleep(1);
        }
        s_tok = tok;
    }
    __syncthreads();
    return s_tok;
}

}  // namespace

template <int KIND>
__global__ void __launch_bounds__(256, 1) k_decode_persistent(const PdModel* __restrict__ Mp, int len0, int step0,
                                                              int n_steps) {
    __shared__ __attribute__((aligned(16))) float sm[PD_SM];
    __shared__ __attribute__((aligned(16))) float sx[PD_SM / 64 * 68];
    __shared__ __attribute__((aligned(16))) float xo[PD_T];
    __shared__ __attribute__((aligned(16))) uint64_t stage[PD_STAGE];
    __shared__ __attribute__((aligned(16))) uint16_t kt[PD_POS * PD_KS], vt[PD_POS * PD_KS];
    const PdModel& M = *Mp;
    PdCtx c;
    c.M = Mp;
    c.abort = M.abort;
    c.sm = (PD_L float*)sm;
    c.sx = (PD_L float*)sx;
    c.xo = (PD_L float*)xo;
    c.stage = (PD_L uint64_t*)stage;
    c.token = M.ctl[CTL_TOKEN];
    c.t = 0;
    c.ep0 = 0;
    const int head_jobs = cdiv(M.V, pd_rpj<KF16>(M.d));
    PD_L float* term = (PD_L float*)(PD_L uint16_t*)kt;  // router group terms, down-projection dots share the tile area
    uint32_t ep = 0;
    for (int t = 0; t < n_steps; ++t) {
        if (t > 0) {
            c.token = pd_token(c, t - 1, head_jobs);
#ifdef GH_PD_TRACE
            if (t == PD_TRACE_STEP && threadIdx.x == 0) {
                pd_trace[blockIdx.x][255] = __builtin_amdgcn_s_memrealtime();
                pd_trace[blockIdx.x][254] = __builtin_amdgcn_s_memtime();
            }
            if (t == PD_TRACE_STEP + 1 && threadIdx.x == 0) {
                pd_trace[blockIdx.x][253] = __builtin_amdgcn_s_memrealtime();
                pd_trace[blockIdx.x][252] = __builtin_amdgcn_s_memtime();
            }
#endif
            if (c.token < 0) return;
            if (blockIdx.x == 0 && threadIdx.x == 0) M.gen_ids[step0 + t - 1] = c.token;
        }
        const int len = len0 + t;  // cache length before this token; its K/V go to slot len
        c.ex = 0;
        c.t = t;
        c.ep0 = ep;
        for (int l = 0; l < M.L; ++l) {
            const PdLayer& Ly = M.layers[l];
            if (Ly.type == 0) {
                const uint32_t e1 = ++ep, e2 = ++ep, e3 = ++ep;
                if (!ph_mamba_in<KIND>(c, Ly, e1)) return;
                if (!ph_mamba_scan(c, Ly, e1, e2)) return;
                if (!ph_mamba_out<KIND>(c, Ly, e1, e2, e3)) return;
                c.ex = e3;
            } else {
                const uint32_t a1 = ++ep, a2 = ++ep, a3 = ++ep;
                if (!ph_attn_qkv<KIND>(c, Ly, len, a1)) return;
                if (!ph_attn_part(c, Ly, len, a1, a2, (PD_L uint16_t*)kt, (PD_L uint16_t*)vt)) return;
                if (!ph_attn_out<KIND>(c, Ly, len, a2, a3)) return;
                c.ex = a3;
            }
            const uint32_t f1 = ++ep, f2 = ++ep;
            if (!ph_moe_up<KIND>(c, Ly, f1, term)) return;
            if (!ph_moe_down<KIND>(c, Ly, f1, f2, term)) return;
            c.ex = f2;
        }
        ++ep;
        if (!ph_head(c, t, ep)) return;
    }
    // the last step's id, and the control block as the per-token path leaves it
    const int last = pd_token(c, n_steps - 1, head_jobs);
    if (blockIdx.x == 0 && threadIdx.x == 0 && last >= 0) {
        M.gen_ids[step0 + n_steps - 1] = last;
        M.ctl[CTL_TOKEN] = last;
        M.ctl[CTL_LEN] = len0 + n_steps;
        M.ctl[CTL_SLOT] = len0 + n_steps - 1;
        M.ctl[CTL_STEP] = step0 + n_steps;
    }
}

#ifdef GH_PD_TRACE
extern "C" int gh_pd_trace_dump(uint64_t* host) {
    GH_HIP(hipMemcpyFromSymbol(host, HIP_SYMBOL(pd_trace), sizeof(pd_trace)));
    return GH_OK;
}
#endif

bool pd_supported(const PdModel& m, int len0, int n_steps, const char** msg) {
    auto no = [&](const char* s) {
        *msg = s;
        return false;
    };
    if (m.kind != 2 && m.kind != 3) return no("weights are not Q8_0 / Q4_K");
    const int bv = m.kind == 3 ? 256 : 64;
    if (m.L < 1 || m.L > PD_MAX_LAYERS) return no("layer count");
    if (m.d % bv || m.d > PD_NW * PD_T || m.d < 64) return no("d");
    const int qd = m.H * m.hd, conv_dim = m.di + 2 * m.mds;
    bool has_m = false, has_a = false;
    for (int l = 0; l < m.L; ++l) (m.layers[l].type == 0 ? has_m : has_a) = true;
    if (has_m) {
        if (m.di % bv || 2 * m.di > PD_SM || m.di > PD_NW * PD_T) return no("d_inner");
        if (m.mds != 64 && m.mds != 128) return no("d_state");
        if (m.mdh > PD_T || m.mh * m.mdh != m.di) return no("Mamba heads");
        if (m.ck < 1 || m.ck > 8) return no("conv kernel");
        (void)conv_dim;
    }
    if (has_a) {
        if (m.hd != 64 && m.hd != 128) return no("head_dim");
        if (m.H % m.KV || m.H / m.KV > 4) return no("GQA group > 4");
        if (qd % bv || qd > 4096) return no("q width");
        const int nsplit = cdiv(len0 + n_steps, PD_POS);
        if (nsplit > PD_MAX_SPLITS) return no("context longer than the persistent attention covers");
        if (qd + m.H * nsplit * (m.hd + 2) > PD_SM) return no("attention partials exceed LDS");
    }
    if (m.ne < 1 || m.ne > 64 || m.K < 1 || m.K > 8 || m.K > m.ne) return no("experts");
    if (m.E % bv || m.SH % bv || m.SH < 64) return no("expert widths (a shared expert is required)");
    if ((m.SH + m.K * m.E) / 64 > 64 || m.SH + m.K * m.E > PD_SM) return no("down inputs");
    if (PD_T / ((m.SH + m.K * m.E) / 64) * ((m.SH + m.K * m.E) / 64) > PD_POS * PD_KS / 2) return no("down task dots");
    if ((size_t)m.ne * m.E * m.d > ((size_t)8 << 20)) return no("expert set too large for the all-expert gate/up");
    if (m.d / 4 + 1 > PD_SM / m.ne) return no("router");
    if (m.ne * (min(m.d / 4, (PD_POS * PD_KS / 2) / m.ne - 1) + 1) > PD_POS * PD_KS / 2) return no("router terms");
    if (len0 + n_steps > m.max_ctx) return no("context");
    if (m.d % 8) return no("lm head rows");
    return true;
}

int pd_launch(const PdModel& host, const PdModel* dev, int len0, int step0, int n_steps) {
    const void* kern = host.kind == 3 ? (const void*)k_decode_persistent<3> : (const void*)k_decode_persistent<2>;
    int per_cu = 0;
    GH_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, PD_T, 0));
    if (per_cu < 1) return fail(GH_EUNSUPPORTED, "persistent decode: kernel does not fit a CU");
    // one block per CU (the jobs of a phase spread over all of them)
    const int nb = min(num_cus(), 256);
    void* args[] = {(void*)&dev, (void*)&len0, (void*)&step0, (void*)&n_steps};
    GH_HIP(hipLaunchCooperativeKernel(kern, dim3(nb), dim3(PD_T), args, 0, stream()));
    return GH_OK;
}

}  // namespace gh
