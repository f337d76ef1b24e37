// Sampling-side ops of the decode loop on the device: top-K candidate
// selection and the repetition / frequency / presence penalties
// (core/ops.h:397-404; CPU semantics core/math_cpu.cpp:695-707 and 725-752,
// limits and messages of the CUDA branch cuda/kernels.cu:1279-1300, 1473-1476).
//
// topk_select: every logit becomes one 64-bit key, an order-preserving form of
// the value above ~index, so that sorting keys in descending order is sorting
// by (value descending, index ascending) -- the reference's comparator -- and
// all keys differ. -0 is keyed as +0 (equal values there); NaN gets value part
// 0, below -inf (the reference's comparator is not an order on NaN). Pass 1:
// one 256-thread block per 512 logits sorts their keys (bitonic, two keys per
// thread in registers, lane shuffles, LDS only for the two farthest steps) and
// keeps the first K; further passes do the same over the survivors until one
// block is left, which writes the K winners (values re-read from the logits,
// so -0 keeps its sign). A bitonic step costs ~30 instructions per key, so
// small sorts spread over many CUs beat one large sort per CU.
//
// apply_rep_penalties: one block. Pass 1 counts the in-range history tokens
// into a per-vocabulary table (device atomics); pass 2 hands each token's
// count to exactly one thread by an atomic exchange with 0, which applies the
// transform once per distinct token and leaves the table zeroed for the next
// call (it is cleared once, when allocated).
#include "gh_common.h"

namespace gh {

constexpr int TK_MAXV = 262144;
constexpr int TK_MAXK = 128;

__device__ __forceinline__ uint64_t tk_key(float v, int i) {
    const uint32_t lo = ~(uint32_t)i;
    if (v != v) return lo;  // NaN: value part 0
    const uint32_t u = __builtin_bit_cast(uint32_t, v == 0.f ? 0.f : v);
    const uint32_t hi = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t tk_shfl_xor(uint64_t v, int m) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
    return ((uint64_t)hi << 32) | lo;
}

template <int E, int J>
__device__ __forceinline__ void tk_cas_local(uint64_t (&v)[E], int k) {
    if constexpr (J < E) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            if ((e & J) == 0) {  // positions p = E t + e and p + J
                const int p = E * threadIdx.x + e;
                const uint64_t a = v[e], b = v[e + J];
                const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
                const bool desc = (p & k) == 0;  // branch-free exchange
                v[e] = desc ? hi : lo;
                v[e + J] = desc ? lo : hi;
            }
        }
    }
}

constexpr int TK_NT = 256;                // threads of a sorting block
constexpr int TK_E = 2;                   // keys per thread
constexpr int TK_C = TK_NT * TK_E;        // keys per block

// Bitonic sort into descending order of the TK_C keys of one block, thread t
// holding positions 2t, 2t + 1 in v[]. A compare-exchange of positions p and
// p ^ j keeps the larger key at the lower position inside blocks with
// (p & k) == 0 and at the higher one elsewhere. Partners closer than 2 are in
// the same thread, closer than 128 in the same wave (lane shuffles); only the
// j >= 128 steps go through LDS (s[] holds TK_C keys), two barriers each.
// Four waves share the work of every step, one per SIMD. With kmax < TK_C only
// the first kmax positions are sorted (pairs never cross a kmax boundary).
__device__ void tk_sort_desc(uint64_t (&v)[TK_E], uint64_t* s, int kmax) {
    const int tid = threadIdx.x;
    for (int k = 2; k <= kmax; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            if (j == 1) {
                tk_cas_local<TK_E, 1>(v, k);
                continue;
            }
            uint64_t o[TK_E];
            if (j < 64 * TK_E) {
#pragma unroll
                for (int e = 0; e < TK_E; ++e) o[e] = tk_shfl_xor(v[e], j / TK_E);
            } else {
                __syncthreads();  // the previous LDS step has been read
#pragma unroll
                for (int e = 0; e < TK_E; ++e) s[TK_E * tid + e] = v[e];
                __syncthreads();
#pragma unroll
                for (int e = 0; e < TK_E; ++e) o[e] = s[(TK_E * tid + e) ^ j];
            }
#pragma unroll
            for (int e = 0; e < TK_E; ++e) {
                const int p = TK_E * tid + e;
                const bool lower = (p & j) == 0, desc = (p & k) == 0;
                const uint64_t a = v[e], b = o[e];
                const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
                v[e] = (lower == desc) ? hi : lo;
            }
        }
    }
}

// One pass: block b sorts keys [512 b, 512 b + 512) -- made from the logits
// (FROM_LOGITS) or taken from the previous pass -- and keeps the first K; a
// single-block pass writes the final values and ids instead.
template <bool FROM_LOGITS>
__global__ void __launch_bounds__(TK_NT) k_topk_pass(const float* __restrict__ l, const uint64_t* __restrict__ in,
                                                     int n, int K, uint64_t* __restrict__ out,
                                                     float* __restrict__ vals, int32_t* __restrict__ ids) {
    __shared__ uint64_t s[TK_C];
    uint64_t v[TK_E];
    const int base = blockIdx.x * TK_C + TK_E * threadIdx.x;
#pragma unroll
    for (int e = 0; e < TK_E; ++e) {
        const int i = base + e;
        if (FROM_LOGITS) v[e] = i < n ? tk_key(l[i], i) : 0ull;  // padding sorts last
        else v[e] = i < n ? in[i] : 0ull;
    }
    int kmax = TK_C;  // a single block sorts only the power of two that holds its n keys
    if (gridDim.x == 1)
        while (kmax > 2 && kmax / 2 >= n) kmax >>= 1;
    tk_sort_desc(v, s, kmax);
#pragma unroll
    for (int e = 0; e < TK_E; ++e) {
        const int k = TK_E * threadIdx.x + e;
        if (k >= K) break;
        if (gridDim.x == 1) {
            const int id = (int)~(uint32_t)v[e];
            ids[k] = id;
            vals[k] = l[id];
        } else {
            out[(size_t)blockIdx.x * K + k] = v[e];
        }
    }
}

__global__ void __launch_bounds__(1024) k_rep_penalties(float* __restrict__ l, int V, const int32_t* __restrict__ hist,
                                                        int n, float rep, float freq, float pres,
                                                        int* __restrict__ cnt) {
#pragma clang fp contract(off)
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int t = hist[i];
        if (t >= 0 && t < V) (void)__hip_atomic_fetch_add(cnt + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): every count has been performed
    __syncthreads();
    const bool use_rep = rep > 0.0f && rep != 1.0f, use_freq = freq != 0.0f, use_pres = pres != 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int t = hist[i];
        if (t < 0 || t >= V) continue;
        const int c = __hip_atomic_exchange(cnt + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (c <= 0) continue;
        float v = l[t];
        if (use_rep) v = v > 0.0f ? v / rep : v * rep;
        if (use_freq) v -= freq * (float)c;
        if (use_pres) v -= pres;
        l[t] = v;
    }
}

}  // namespace gh

using namespace gh;

extern "C" {

int gh_topk_select(const float* logits, int V, int K, float* out_vals, int32_t* out_ids) {
    GH_REQUIRE(logits && out_vals && out_ids, "topk_select: null argument");
    GH_REQUIRE(K >= 1 && K <= TK_MAXK, "topk_select: K out of range [1,128]");
    GH_REQUIRE(V >= K, "topk_select: vocab too small for K");
    GH_REQUIRE(V <= TK_MAXV, "topk_select: vocab exceeds maximum supported size (262,144)");
    // pass 1 over the logits, then passes over the survivors until one block is left
    int G = (V + TK_C - 1) / TK_C;
    const size_t cap = (size_t)G * K;
    uint64_t* buf = nullptr;
    if (G > 1) {
        buf = (uint64_t*)workspace(WS_TOPK, 2 * cap * 8);
        if (!buf) return fail(GH_ENOMEM, "topk_select: workspace");
    }
    hipLaunchKernelGGL(k_topk_pass<true>, dim3(G), dim3(TK_NT), 0, stream(), logits, nullptr, V, K, buf, out_vals,
                       out_ids);
    GH_LAUNCHED("k_topk_pass");
    int half = 0;
    while (G > 1) {
        const int n = G * K;
        G = (n + TK_C - 1) / TK_C;
        hipLaunchKernelGGL(k_topk_pass<false>, dim3(G), dim3(TK_NT), 0, stream(), logits, buf + half * cap, n, K,
                           buf + (half ^ 1) * cap, out_vals, out_ids);
        GH_LAUNCHED("k_topk_pass");
        half ^= 1;
    }
    return GH_OK;
}

int gh_apply_rep_penalties(float* logits, int V, const int32_t* hist, int hist_n, float rep, float freq,
                           float pres) {
    if (hist_n <= 0 || V <= 0) return GH_OK;
    if (!(rep > 0.0f && rep != 1.0f) && freq == 0.0f && pres == 0.0f) return GH_OK;
    GH_REQUIRE(logits && hist, "apply_rep_penalties: null argument");
    // the count table: zeroed once when (re)allocated, left zeroed by every call
    static int* cnt = nullptr;
    static int cap = 0;
    if (cap < V) {
        GH_HIP(hipStreamSynchronize(stream()));
        if (cnt) GH_HIP(hipFree(cnt));
        cnt = nullptr;
        cap = 0;
        GH_HIP(hipMalloc(&cnt, (size_t)V * 4));
        GH_HIP(hipMemsetAsync(cnt, 0, (size_t)V * 4, stream()));
        cap = V;
    }
    int32_t* hd = (int32_t*)workspace(WS_PEN_HIST, (size_t)hist_n * 4);
    if (!hd) return fail(GH_ENOMEM, "apply_rep_penalties: workspace");
    // the history is a host array (the reference passes Generator::history_)
    GH_HIP(hipMemcpyAsync(hd, hist, (size_t)hist_n * 4, hipMemcpyHostToDevice, stream()));
    hipLaunchKernelGGL(k_rep_penalties, dim3(1), dim3(1024), 0, stream(), logits, V, hd, hist_n, rep, freq, pres, cnt);
    GH_LAUNCHED("k_rep_penalties");
    return GH_OK;
}

}  // extern "C"
