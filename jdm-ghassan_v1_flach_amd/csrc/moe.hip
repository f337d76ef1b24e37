// Mixture-of-experts FFN: router top-k, deterministic token permutation,
// grouped expert GEMV (decode) / grouped MFMA GEMM (prefill) with the SwiGLU
// fused into the gate/up epilogue, and an ordered combine.
//
// Replaces cuda/moe.cu:170-905: there the grouping is an atomic counting
// sort (non-deterministic slot order), the offsets are copied to the host
// (a sync per layer), every expert is one GEMV/GEMM launch per matrix and the
// combine is an atomicAdd scatter. Here the whole FFN is 6-7 launches with
// no host sync, independent of the expert count, and every output is
// bit-reproducible run to run.
#include "gemm_tile.h"
#include "gemv_tasks.h"
#include "route.h"

namespace gh {

__global__ void __launch_bounds__(256) k_route(const float* __restrict__ x, const float* __restrict__ rw,
                                               const float* __restrict__ bias, float* __restrict__ probs,
                                               int32_t* __restrict__ idx, float* __restrict__ wout, int d, int ne,
                                               int K, const float* __restrict__ nw, float eps,
                                               float* __restrict__ xn, int GW) {
    extern __shared__ float route_sm[];
    route_token(x, rw, bias, probs, idx, wout, d, ne, K, nw, eps, xn, GW, blockIdx.x, route_sm, route_sm + d, nullptr);
}

// window of router groups whose terms fit 60 KB of LDS next to the token;
// for many tokens (one block each) a 64-group window keeps blocks small
static int route_window(int d, int ne, int N) {
    const int budget = 60 * 1024 / 4 - d;  // floats, leaving room for the static arrays
    int gw = budget / ne - 1;
    if (N > 8 && gw > 64) gw = 64;
    if (gw > d / 4) gw = d / 4;
    return gw < 1 ? 1 : gw;
}
static size_t route_lds(int d, int ne, int N) {
    return ((size_t)d + (size_t)ne * (route_window(d, ne, N) + 1)) * 4;
}

// Router logits of a large expert set for few tokens: one wave per (expert e, token t). Lane
// l holds the group terms of groups l, l + 64, ... (the reference's group term
// ((x0 w0 + x1 w1) + x2 w2) + x3 w3, core/moe_cpu.cpp:76-83, no fused multiply-add), read
// with coalesced 16-byte loads; the sequential sum over the groups in order then runs as one
// chain of adds whose operands come by readlane (no memory round trip inside the chain).
// With `nw` the token row is RMS-normalised first (double sum of squares, the k_rmsnorm
// statistic) and the wave of expert 0 writes the normalised row to xn. Requires d % 4 == 0
// and d <= 4096.
constexpr int RC_J = 16;  // groups per lane (d <= 4096)
__global__ void __launch_bounds__(64) k_route_chain(const float* __restrict__ x, const float* __restrict__ rw,
                                                    float* __restrict__ logits, int d, int ne,
                                                    const float* __restrict__ nw, float eps,
                                                    float* __restrict__ xn) {
#pragma clang fp contract(off)
    const int e = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int G = d / 4, J = (G + 63) / 64;
    const float4* x4 = (const float4*)(x + (size_t)t * d);
    const float4* w4 = (const float4*)(rw + (size_t)e * d);
    float4 xv[RC_J], wv[RC_J];
#pragma unroll
    for (int j = 0; j < RC_J; ++j) {
        const int g = 64 * j + lane;
        if (j < J) {
            xv[j] = g < G ? x4[g] : make_float4(0.f, 0.f, 0.f, 0.f);
            wv[j] = g < G ? w4[g] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    if (nw) {
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < RC_J; ++j)
            if (j < J) ss += (double)xv[j].x * xv[j].x + (double)xv[j].y * xv[j].y + (double)xv[j].z * xv[j].z +
                             (double)xv[j].w * xv[j].w;
        const double tot = wave_sum(ss);
        const double invd = 1.0 / sqrt(tot / (double)d + (double)eps);
        const float inv = isfinite(invd) ? (float)invd : 0.0f;
        const float4* n4 = (const float4*)nw;
#pragma unroll
        for (int j = 0; j < RC_J; ++j) {
            const int g = 64 * j + lane;
            if (j < J && g < G) {
                const float4 wn = n4[g];
                xv[j] = make_float4(xv[j].x * inv * wn.x, xv[j].y * inv * wn.y, xv[j].z * inv * wn.z,
                                    xv[j].w * inv * wn.w);
                if (e == 0 && xn) ((float4*)(xn + (size_t)t * d))[g] = xv[j];
            }
        }
    }
    float term[RC_J];
#pragma unroll
    for (int j = 0; j < RC_J; ++j)
        if (j < J) {
            const float p0 = xv[j].x * wv[j].x, p1 = xv[j].y * wv[j].y, p2 = xv[j].z * wv[j].z, p3 = xv[j].w * wv[j].w;
            term[j] = ((p0 + p1) + p2) + p3;
        }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < RC_J; ++j) {
        if (j < J) {
            const int cnt = min(64, G - 64 * j);  // wave-uniform
            const int tb = __builtin_bit_cast(int, term[j]);
            if (cnt == 64) {
#pragma unroll
                for (int l = 0; l < 64; ++l) s += __builtin_bit_cast(float, __builtin_amdgcn_readlane(tb, l));
            } else {
                // a partial last run: readlane needs a wave-uniform lane index, here a loop counter
                for (int l = 0; l < cnt; ++l) s += __builtin_bit_cast(float, __builtin_amdgcn_readlane(tb, l));
            }
        }
    }
    if (lane == 0) logits[(size_t)t * ne + e] = s;
}

// Router of many tokens (prefill), no norm, in two kernels.
// k_route_logits: block (expert slice j, token tile i) keeps the router rows
// of experts 16j..16j+15 in LDS for the whole K range (rows padded by one
// float4, so the 16 rows a wave reads fall in distinct banks) and computes
// their logits for 32 tokens: lane (token t = l / 16, expert e = l % 16) of
// wave w runs the chain of token 32i + 4w + t, expert 16j + e: the
// reference's group term ((x0 w0 + x1 w1) + x2 w2) + x3 w3
// (core/moe_cpu.cpp:76-83) added in group order -- the same arithmetic as
// k_route. Activations stream from global (4 tokens per wave, prefetched a
// batch of groups ahead). k_route_finish then softmaxes and selects per
// token (one wave each).
constexpr int RL_E = 16, RL_T = 32, RL_B = 8;  // experts per block, tokens per block, groups per batch
__global__ void __launch_bounds__(512) k_route_logits(const float* __restrict__ x, const float* __restrict__ rw,
                                                      float* __restrict__ logits, int N, int d, int ne) {
#pragma clang fp contract(off)
    extern __shared__ float4 rl_w[];  // [RL_E][ngroups + 1]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ngroups = d / 4, rs = ngroups + 1;
    const int e0 = blockIdx.x * RL_E;
    const float4* rw4 = (const float4*)rw;
    for (int q = tid; q < RL_E * ngroups; q += 512) {
        const int r = q / ngroups, g = q - r * ngroups;
        const int e = min(e0 + r, ne - 1);
        rl_w[r * rs + g] = rw4[(size_t)e * ngroups + g];
    }
    const int el = lane & 15, tl = lane >> 4;
    const int t = blockIdx.y * RL_T + wave * 4 + tl;
    const float4* xr = (const float4*)x + (size_t)min(t, N - 1) * ngroups;
    const float4* wr = rl_w + el * rs;
    float4 xa[RL_B], xb[RL_B];
#pragma unroll
    for (int j = 0; j < RL_B; ++j) xa[j] = j < ngroups ? xr[j] : float4{0.f, 0.f, 0.f, 0.f};
    __syncthreads();
    float s = 0.0f;
    int g = 0;
    auto batch = [&](const float4 (&xv)[RL_B], int gb) {
        float term[RL_B];
#pragma unroll
        for (int j = 0; j < RL_B; ++j) {
            const float4 w4 = wr[gb + j];
            const float p0 = xv[j].x * w4.x, p1 = xv[j].y * w4.y, p2 = xv[j].z * w4.z, p3 = xv[j].w * w4.w;
            term[j] = ((p0 + p1) + p2) + p3;
        }
#pragma unroll
        for (int j = 0; j < RL_B; ++j) s += term[j];
    };
    for (; g + 2 * RL_B <= ngroups; g += 2 * RL_B) {
#pragma unroll
        for (int j = 0; j < RL_B; ++j) xb[j] = xr[g + RL_B + j];
        batch(xa, g);
        if (g + 3 * RL_B <= ngroups) {
#pragma unroll
            for (int j = 0; j < RL_B; ++j) xa[j] = xr[g + 2 * RL_B + j];
        }
        batch(xb, g + RL_B);
    }
    if (g + RL_B <= ngroups) {  // xa holds groups g..g+RL_B-1
        batch(xa, g);
        g += RL_B;
    }
    for (; g < ngroups; ++g) {  // the last < RL_B groups
        const float4 xv = xr[g], w4 = wr[g];
        const float p0 = xv.x * w4.x, p1 = xv.y * w4.y, p2 = xv.z * w4.z, p3 = xv.w * w4.w;
        s += ((p0 + p1) + p2) + p3;
    }
    if (t < N && e0 + el < ne) logits[(size_t)t * ne + e0 + el] = s;
}

__global__ void __launch_bounds__(256) k_route_finish(const float* __restrict__ logits, const float* __restrict__ bias,
                                                      float* __restrict__ probs, int32_t* __restrict__ idx,
                                                      float* __restrict__ wout, int N, int ne, int K) {
    __shared__ float sp_all[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave;
    if (t >= N) return;  // whole wave (route_finish is wave-local)
    float* sp = sp_all[wave];
    if (lane < ne) sp[lane] = logits[(size_t)t * ne + lane];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    route_finish(sp, bias, ne, K, t, idx, wout, probs);
}

// router launch: one block per token, or the two-kernel form for a large
// router matrix and few tokens
static int launch_route(const float* x, const float* rw, const float* bias, float* probs, int32_t* idx, float* w,
                        int N, int d, int ne, int K, const float* nw, float eps, float* xn) {
    if (N <= 8 && (size_t)ne * d > 16384 && ne <= 64 && d % 4 == 0 && d <= 4096) {
        float* lg = (float*)workspace(WS_MOE_TERMS, (size_t)N * ne * 4);
        if (!lg) return fail(GH_ENOMEM, "moe route: workspace");
        hipLaunchKernelGGL(k_route_chain, dim3(ne, N), dim3(64), 0, stream(), x, rw, lg, d, ne, nw, eps, xn);
        hipLaunchKernelGGL(k_route_finish, dim3(cdiv(N, 4)), dim3(256), 0, stream(), lg, bias, probs, idx, w, N, ne,
                           K);
        GH_LAUNCHED("k_route_chain/finish");
        return GH_OK;
    }
    const size_t rl_lds = (size_t)RL_E * (d / 4 + 1) * 16;
    // below 16 experts (c1: 8) a 16-expert slice leaves half the lanes idle and a 128-token
    // prefill fills 4 blocks; one block per token (k_route) is faster there (c1 prefill +5 %)
    if (N > 8 && !nw && ne <= 64 && ne >= 16 && K <= 8 && d % 4 == 0 && rl_lds <= 160 * 1024) {
        static bool configured = false;
        if (!configured) {
            const hipError_t e = hipFuncSetAttribute((const void*)k_route_logits,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            if (e != hipSuccess) return fail(GH_EHIP, "k_route_logits LDS attribute: %s", hipGetErrorString(e));
            configured = true;
        }
        float* lg = (float*)workspace(WS_MOE_TERMS, (size_t)N * ne * 4);
        if (!lg) return fail(GH_ENOMEM, "moe route: workspace");
        hipLaunchKernelGGL(k_route_logits, dim3(cdiv(ne, RL_E), cdiv(N, RL_T)), dim3(512), rl_lds, stream(), x, rw,
                           lg, N, d, ne);
        hipLaunchKernelGGL(k_route_finish, dim3(cdiv(N, 4)), dim3(256), 0, stream(), lg, bias, probs, idx, w, N, ne,
                           K);
        GH_LAUNCHED("k_route_logits/finish");
        return GH_OK;
    }
    hipLaunchKernelGGL(k_route, dim3(N), dim3(256), route_lds(d, ne, N), stream(), x, rw, bias, probs, idx, w, d, ne,
                       K, nw, eps, xn, route_window(d, ne, N));
    GH_LAUNCHED("k_route");
    return GH_OK;
}

// ========================================================== permutation
// Stable counting sort of slot ids s = t*K+k by expert, in three
// deterministic passes over 256-slot chunks (wave ballots give each lane its
// rank among equal experts of lower lanes; lower waves come first).
constexpr int PERM_CHUNK = 256, PERM_MAX_CHUNKS = 256;

__device__ __forceinline__ void chunk_ranks(const int32_t* idx, int S, int ne, int c, int* wc /*[4][64] LDS*/,
                                            int& e_l, int& rank) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int s = c * PERM_CHUNK + threadIdx.x;
    e_l = s < S ? idx[s] : -1;
    const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    rank = 0;
    for (int e = 0; e < ne; ++e) {
        const unsigned long long m = __ballot(e_l == e);
        if (e_l == e) rank = __popcll(m & below);
        if (lane == e) wc[wave * 64 + e] = __popcll(m);
    }
    __syncthreads();
}

__global__ void __launch_bounds__(256) k_perm_count(const int32_t* __restrict__ idx, int S, int ne,
                                                    int32_t* __restrict__ counts) {
    __shared__ int wc[4 * 64];
    int e_l, rank;
    chunk_ranks(idx, S, ne, blockIdx.x, wc, e_l, rank);
    if (threadIdx.x < ne)
        counts[(size_t)blockIdx.x * ne + threadIdx.x] =
            wc[threadIdx.x] + wc[64 + threadIdx.x] + wc[128 + threadIdx.x] + wc[192 + threadIdx.x];
}

// counts[c][e] -> base[c][e] (first grouped position of expert e's slots in
// chunk c); offsets = exclusive scan of the totals; tile table for the
// grouped GEMM (tiles of `bm` rows per expert segment, experts in order). Wave w scans its
// quarter of the chunks per expert, the earlier quarters' totals are added after; the tile
// table is written by every thread (tile j belongs to the last expert whose first tile is
// <= j).
__global__ void __launch_bounds__(256) k_perm_scan(int32_t* __restrict__ counts, int nchunks, int ne, int S,
                                                   int32_t* __restrict__ offsets, int32_t* __restrict__ tiles,
                                                   int bm) {
    __shared__ int cnt[PERM_MAX_CHUNKS * 64];
    __shared__ int part[4][64];
    __shared__ int offs[65], tfirst[65];
    const int n = nchunks * ne, tid = threadIdx.x, wave = tid >> 6, e = tid & 63;
    for (int i = tid; i < n; i += 256) cnt[i] = counts[i];
    __syncthreads();
    const int q = (nchunks + 3) / 4, c0 = min(nchunks, wave * q), c1 = min(nchunks, c0 + q);
    int run = 0;
    if (e < ne)
        for (int c = c0; c < c1; ++c) {
            const int v = cnt[c * ne + e];
            cnt[c * ne + e] = run;
            run += v;
        }
    part[wave][e] = run;
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += part[w][e];
    if (e < ne && before)
        for (int c = c0; c < c1; ++c) cnt[c * ne + e] += before;
    if (wave == 0) {
        const int tot = e < ne ? part[0][e] + part[1][e] + part[2][e] + part[3][e] : 0;
        const int nt = bm > 0 ? (tot + bm - 1) / bm : 0;
        int incl = tot, tincl = nt;
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o, 64), tv = __shfl_up(tincl, o, 64);
            if (e >= o) {
                incl += v;
                tincl += tv;
            }
        }
        if (e < ne) {
            offs[e] = incl - tot;
            tfirst[e] = tincl - nt;
        }
        if (e == ne - 1) {
            offs[ne] = S;
            tfirst[ne] = tincl;
        }
    }
    __syncthreads();
    for (int i = tid; i < n; i += 256) counts[i] = cnt[i] + offs[i % ne];
    for (int i = tid; i <= ne; i += 256) offsets[i] = offs[i];
    if (tiles) {
        const int ntiles = tfirst[ne];
        for (int j = tid; j < ntiles; j += 256) {
            int lo = 0, hi = ne - 1;  // the last g with tfirst[g] <= j
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (tfirst[mid] <= j) lo = mid;
                else hi = mid - 1;
            }
            tiles[1 + 2 * j] = lo;
            tiles[2 + 2 * j] = offs[lo] + (j - tfirst[lo]) * bm;
        }
        if (tid == 0) tiles[0] = ntiles;
    }
}

__global__ void __launch_bounds__(256) k_perm_scatter(const int32_t* __restrict__ idx, int S, int ne,
                                                      const int32_t* __restrict__ base, int32_t* __restrict__ grouped,
                                                      int32_t* __restrict__ pos_of_slot) {
    __shared__ int wc[4 * 64];
    int e_l, rank;
    chunk_ranks(idx, S, ne, blockIdx.x, wc, e_l, rank);
    const int s = blockIdx.x * PERM_CHUNK + threadIdx.x;
    if (s < S) {
        const int wave = threadIdx.x >> 6;
        int before = 0;
        for (int w = 0; w < wave; ++w) before += wc[w * 64 + e_l];
        const int pos = base[(size_t)blockIdx.x * ne + e_l] + before + rank;
        grouped[pos] = s;
        if (pos_of_slot) pos_of_slot[s] = pos;
    }
}

// The three passes in one block when every slot fits one chunk (S <= 256).
__global__ void __launch_bounds__(256) k_perm_small(const int32_t* __restrict__ idx, int S, int ne,
                                                    int32_t* __restrict__ grouped, int32_t* __restrict__ offsets,
                                                    int32_t* __restrict__ pos_of_slot, int32_t* __restrict__ tiles,
                                                    int bm) {
    __shared__ int wc[4 * 64];
    __shared__ int offs[65];
    int e_l, rank;
    chunk_ranks(idx, S, ne, 0, wc, e_l, rank);
    if (threadIdx.x < 64) {
        const int e = threadIdx.x;
        const int tot = e < ne ? wc[e] + wc[64 + e] + wc[128 + e] + wc[192 + e] : 0;
        int incl = tot;
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o, 64);
            if (e >= o) incl += v;
        }
        if (e < ne) offs[e] = incl - tot;
        if (e == 0) offs[ne] = S;
    }
    __syncthreads();
    const int s = threadIdx.x;
    if (s < S) {
        const int wave = threadIdx.x >> 6;
        int before = 0;
        for (int w = 0; w < wave; ++w) before += wc[w * 64 + e_l];
        const int pos = offs[e_l] + before + rank;
        grouped[pos] = s;
        if (pos_of_slot) pos_of_slot[s] = pos;
    }
    for (int i = threadIdx.x; i <= ne; i += 256) offsets[i] = offs[i];
    if (threadIdx.x == 0 && tiles) {
        int nt = 0;
        for (int g = 0; g < ne; ++g)
            for (int m0 = offs[g]; m0 < offs[g + 1]; m0 += bm) {
                tiles[1 + 2 * nt] = g;
                tiles[2 + 2 * nt] = m0;
                ++nt;
            }
        tiles[0] = nt;
    }
}

static int permute(const int32_t* idx, int S, int ne, int32_t* grouped, int32_t* offsets, int32_t* pos_of_slot,
                   int32_t* tiles, int bm) {
    if (S <= PERM_CHUNK) {
        hipLaunchKernelGGL(k_perm_small, dim3(1), dim3(256), 0, stream(), idx, S, ne, grouped, offsets, pos_of_slot,
                           tiles, bm);
        GH_LAUNCHED("k_perm_small");
        return GH_OK;
    }
    const int nch = cdiv(S > 0 ? S : 1, PERM_CHUNK);
    if (nch > PERM_MAX_CHUNKS) return fail(GH_EUNSUPPORTED, "moe permute: %d slots (max %d)", S, PERM_CHUNK * PERM_MAX_CHUNKS);
    int32_t* counts = (int32_t*)workspace(WS_MOE_PERM, (size_t)nch * ne * 4);
    if (!counts) return fail(GH_ENOMEM, "moe permute: workspace");
    hipLaunchKernelGGL(k_perm_count, dim3(nch), dim3(256), 0, stream(), idx, S, ne, counts);
    hipLaunchKernelGGL(k_perm_scan, dim3(1), dim3(256), 0, stream(), counts, nch, ne, S, offsets, tiles, bm);
    hipLaunchKernelGGL(k_perm_scatter, dim3(nch), dim3(256), 0, stream(), idx, S, ne, counts, grouped, pos_of_slot);
    GH_LAUNCHED("k_perm_*");
    return GH_OK;
}

// ====================================================== decode: grouped GEMV
// Jobs 0..S-1 are routed slots (token s/K, expert idx[s]), jobs S..S+N-1 the
// shared expert of token j-S. A wave computes RP rows of gate AND up of one
// job with one activation chunk in registers, then writes silu(g)*u.
struct GemvJobs {
    const float* x;          // [N][d] (gate/up) or activations (down)
    const int32_t* idx;      // [S]
    int S, N, K, d;          // K = top-k
    const uint8_t* wa;       // routed gate (or down) base
    const uint8_t* wb;       // routed up base (gate/up only)
    size_t estride;          // bytes per expert matrix
    const uint8_t* sa;       // shared gate (or down), may be null
    const uint8_t* sb;       // shared up
    int rows_r, rows_s;      // rows of routed / shared matrices
    int kin_r, kin_s;        // input length (K dim) of routed / shared
    size_t rowb_r, rowb_s;   // bytes per weight row
    float* out_r;            // [S][rows_r]
    float* out_s;            // [N][rows_s]
    const float* in_s;       // shared input (down: shared act)
    // routing in the gate/up kernel itself (k_moe_gemv<.., true>): the raw token rows, the
    // router and its norm; idx / w are written by the first block of each token
    const float* rx;
    const float* rw;
    const float* rbias;
    const float* rnw;
    float reps;
    int ne, gw;
    int32_t* ridx;
    float* rwout;
    const float* rlogits;  // router logits [N][ne] (k_moe_gemv<.., LOGITS>)
    float* rprobs;         // probabilities out [N][ne] (LOGITS, may be null)
    // gate/up of EVERY expert (small expert sets): activations [N][ne][rows_r]; the down
    // kernel then gathers the rows of the selected experts (0: rows in slot order)
    int gather_ne;
};

// ALLEXP (small expert sets, decode): jobs 0..N*ne-1 are (token j/ne, expert
// j%ne) for every expert, N*ne.. the shared experts, and the last N rows of
// blocks route token j (block x = 0 only, writing idx / w): the routing runs
// beside the GEMVs instead of in front of them, and the down kernel gathers
// the selected experts' activations.
// LOGITS (large routers, decode): the router logits come from k_route_chain; every routed
// block picks its token's experts from them itself (route_finish, one wave), the first block
// of each token writing idx / w for the down kernel, so no launch sits between the router and
// the expert weights. Shared-expert blocks start at once.
template <int KIND, bool DUAL, bool ROUTE = false, bool ALLEXP = false, bool LOGITS = false>
__global__ void __launch_bounds__(256) k_moe_gemv(GemvJobs J) {
    int job = blockIdx.y;
    if constexpr (ALLEXP) {
        const int nall = J.N * J.ne;  // J.N = tokens here (shared experts required)
        if (job >= nall + J.N) {
            if (blockIdx.x != 0) return;
            extern __shared__ float msm_r[];
            const int token = job - nall - J.N;
            route_token(J.rx, J.rw, J.rbias, nullptr, J.ridx, J.rwout, J.d, J.ne, J.K, J.rnw, J.reps, nullptr, J.gw,
                        token, msm_r, msm_r + J.d, nullptr);
            return;
        }
    }
    const bool shared = ALLEXP ? job >= J.N * J.ne : job >= J.S;
    extern __shared__ float msm[];  // ROUTE: token row [d] | router terms
    __shared__ int ssel[8];
    if (ALLEXP && shared) job = J.S + (job - J.N * J.ne);  // shared jobs keep their usual numbering
    const int rows = shared ? J.rows_s : J.rows_r;
    const int kin = shared ? J.kin_s : J.kin_r;
    const size_t rowb = shared ? J.rowb_s : J.rowb_r;
    const int T = kin / 64;
    int LPR = 64;
    while (LPR > 1 && LPR > T) LPR >>= 1;
    const int RP = 64 / LPR;
    if (ALLEXP) {
        if (blockIdx.x * 4 * RP >= rows) return;
        extern __shared__ float msm_n[];
        route_norm(J.rx, shared ? job - J.S : job / J.ne, J.d, J.rnw, J.reps, nullptr, msm_n);
    }
    if (LOGITS && !shared) {
        if (blockIdx.x * 4 * RP >= rows) return;
        __shared__ float slg[64];
        const int token = job / J.K;
        const bool writer = blockIdx.x == 0 && job % J.K == 0;
        if (threadIdx.x < 64) {
            if (threadIdx.x < J.ne) slg[threadIdx.x] = J.rlogits[(size_t)token * J.ne + threadIdx.x];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            route_finish(slg, J.rbias, J.ne, J.K, token, writer ? J.ridx : nullptr, writer ? J.rwout : nullptr,
                         writer ? J.rprobs : nullptr, ssel);
        }
        __syncthreads();
    }
    if (ROUTE) {
        if (blockIdx.x * 4 * RP >= rows) return;  // no rows here (block 0, the writer, always has some)
        // every block routes its token (identical arithmetic, so all agree); the normalised row
        // stays in LDS as the GEMV input
        const int token = shared ? job - J.S : job / J.K;
        const bool writer = !shared && blockIdx.x == 0 && job % J.K == 0;
        route_token(J.rx, J.rw, J.rbias, nullptr, writer ? J.ridx : nullptr, writer ? J.rwout : nullptr, J.d, J.ne,
                    J.K, J.rnw, J.reps, nullptr, J.gw, token, msm, msm + J.d, ssel);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, rp = lane / LPR;
    const int row = (blockIdx.x * 4 + wave) * RP + rp;
    if ((blockIdx.x * 4 + wave) * RP >= rows) return;  // whole wave idle (uniform)
    const int rr = row < rows ? row : rows - 1;
    const float* xin;
    const uint8_t *Wa, *Wb = nullptr;
    if (shared) {
        const int t = job - J.S;
        xin = (ROUTE || ALLEXP) ? msm : (DUAL ? J.x + (size_t)t * J.d : J.in_s + (size_t)t * kin);
        Wa = J.sa;
        if (DUAL) Wb = J.sb;
    } else {
        const int e = ALLEXP ? job % J.ne : (ROUTE || LOGITS) ? ssel[job % J.K] : J.idx[job];
        const int tok = ALLEXP ? job / J.ne : job / J.K;
        xin = (ROUTE || ALLEXP) ? msm : (DUAL ? J.x + (size_t)tok * J.d : J.x + (size_t)job * kin);
        Wa = J.wa + (size_t)e * J.estride;
        if (DUAL) Wb = J.wb + (size_t)e * J.estride;
    }
    float ga = 0.f, ub = 0.f;
    for (int t = sub; t < T; t += LPR) {
        uint32_t w0[Task<KIND>::DW], w1[Task<KIND>::DW];
        load_task<KIND>(Wa + (size_t)rr * rowb, t, w0);
        if (DUAL) load_task<KIND>(Wb + (size_t)rr * rowb, t, w1);
        float xv[64];
        const float4* xp = (const float4*)(xin + (size_t)t * 64);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 v = xp[i];
            xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
        }
        float xs[2];
        task_xsum<KIND>(xv, xs);
        ga += task_dot<KIND>(w0, xv, xs, t);
        if (DUAL) ub += task_dot<KIND>(w1, xv, xs, t);
    }
    ga = group_sum(ga, LPR);
    if (DUAL) ub = group_sum(ub, LPR);
    if (sub == 0 && row < rows) {
        const float v = DUAL ? ga / (1.0f + expf(-ga)) * ub : ga;
        if (shared) J.out_s[(size_t)(job - J.S) * rows + row] = v;
        else J.out_r[(size_t)job * rows + row] = v;
    }
}

// Down projections of all K routed experts and the shared expert of token
// blockIdx.y, merged in the combine order (shared first, then k = 0..K-1,
// core/moe_cpu.cpp:265-287) and added to the residual row:
// xres[t][row] += shared + sum_k w[t,k] * down_k (or = without `accumulate`).
// One wave owns RP rows for every job, so the merge happens in registers
// (no per-expert outputs). Latency: the token's activation rows are staged
// in LDS while the routing is read, and the next job's weight bytes are
// requested while the current job is multiplied.
constexpr int DC_TPJ = 4;  // tasks per lane per job held in registers
template <int KIND>
__global__ void __launch_bounds__(256) k_moe_down_combine(GemvJobs J, const float* __restrict__ wroute,
                                                          float* __restrict__ xres, int LPR, int accumulate) {
    constexpr int DW = Task<KIND>::DW;
    extern __shared__ float dc_act[];  // shared [kin_s] | routed k [kin_r] each
    const int tok = blockIdx.y, K = J.K;
    const bool has_sh = J.N > 0;
    const int RP = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, rp = lane / LPR;
    const int rows = J.rows_r;  // = d for both routed and shared down matrices
    const int row = (blockIdx.x * 4 + wave) * RP + rp;
    const int rr = row < rows ? row : rows - 1;
    const bool active = (blockIdx.x * 4 + wave) * RP < rows;
    int ek[8];
    float wk[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
        if (k < K) {
            ek[k] = J.idx[tok * K + k];
            wk[k] = wroute[tok * K + k];
        }
    const int sh_len = has_sh ? J.kin_s : 0;
    {
        const float4* src_s = (const float4*)(J.in_s + (size_t)tok * J.kin_s);
        const int kq = J.kin_r / 4;
        const int n4s = sh_len / 4, n4 = n4s + K * kq;
        for (int i = threadIdx.x; i < n4; i += 256) {
            if (i < n4s) {
                ((float4*)dc_act)[i] = src_s[i];
            } else {
                // routed k: its slot's row, or (all experts computed) the row of its expert
                const int q = i - n4s, kk = q / kq, o = q - kk * kq;
                const size_t r = J.gather_ne ? (size_t)tok * J.gather_ne + J.idx[tok * K + kk] : (size_t)tok * K + kk;
                ((float4*)dc_act)[i] = ((const float4*)(J.x + r * J.kin_r))[o];
            }
        }
    }
    auto load_job = [&](int j, uint32_t (*w)[DW]) {
        const bool shared = j < 0;
        const int T = (shared ? J.kin_s : J.kin_r) / 64;
        const size_t rowb = shared ? J.rowb_s : J.rowb_r;
        const uint8_t* base = (shared ? J.sa : J.wa + (size_t)ek[j] * J.estride) + (size_t)rr * rowb;
#pragma unroll
        for (int q = 0; q < DC_TPJ; ++q) {
            const int t = sub + q * LPR;
            if (t < T) load_task<KIND>(base, t, w[q]);
        }
    };
    uint32_t wa[DC_TPJ][DW], wb[DC_TPJ][DW];
    const int first = has_sh ? -1 : 0;
    if (active) load_job(first, wa);
    __syncthreads();
    if (!active) return;
    float acc = 0.f;
    for (int j = first; j < K; ++j) {
        if (j + 1 < K) load_job(j + 1, wb);
        const bool shared = j < 0;
        const int T = (shared ? J.kin_s : J.kin_r) / 64;
        const float* xin = shared ? dc_act : dc_act + sh_len + (size_t)j * J.kin_r;
        float ga = 0.f;
#pragma unroll
        for (int q = 0; q < DC_TPJ; ++q) {
            const int t = sub + q * LPR;
            if (t < T) {
                float xv[64];
                const float4* xp = (const float4*)(xin + (size_t)t * 64);
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float4 v = xp[i];
                    xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
                }
                float xs[2];
                task_xsum<KIND>(xv, xs);
                ga += task_dot<KIND>(wa[q], xv, xs, t);
            }
        }
        ga = group_sum(ga, LPR);
        if (shared) acc = ga;
        else acc += wk[j] * ga;
#pragma unroll
        for (int q = 0; q < DC_TPJ; ++q)
#pragma unroll
            for (int i = 0; i < DW; ++i) wa[q][i] = wb[q][i];
    }
    if (sub == 0 && row < rows) {
        float* o = xres + (size_t)tok * rows + row;
        *o = accumulate ? *o + acc : acc;
    }
}

// Down projections with the jobs side by side: block = (16 output rows,
// token), wave 0 = the shared expert, wave 1 + k = routed slot k. Every wave
// requests its own weight bytes as soon as it knows its expert (the shared
// wave at once), multiplies 16 rows x its job's K range (4 lanes per row,
// DP_TPL tasks per lane at most), and leaves its 16 row results in LDS; the
// block then merges them in the combine order (shared first, then k = 0..K-1,
// core/moe_cpu.cpp:265-287) and adds the sum to the residual row.
// Activations in LDS: shared [kin_s] | routed k [kin_r] (or, after the
// all-expert gate/up, the selected experts' rows).
constexpr int DP_RB = 16, DP_LPR = 4, DP_TPL = 4;
template <int KIND>
__global__ void __launch_bounds__(576) k_moe_down_par(GemvJobs J, const float* __restrict__ wroute,
                                                      float* __restrict__ xres, int accumulate) {
    constexpr int DW = Task<KIND>::DW;
    extern __shared__ float dp_act[];
    __shared__ float dp_res[9][DP_RB];
    const int tok = blockIdx.y, K = J.K;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % DP_LPR, rloc = lane / DP_LPR;
    const int rows = J.rows_r;
    const int row = blockIdx.x * DP_RB + rloc;
    const int rr = row < rows ? row : rows - 1;
    const bool shared = wave == 0;
    const int k = wave - 1;
    const int e = shared ? 0 : J.idx[tok * K + k];
    const int T = (shared ? J.kin_s : J.kin_r) / 64;
    const size_t rowb = shared ? J.rowb_s : J.rowb_r;
    const uint8_t* base = (shared ? J.sa : J.wa + (size_t)e * J.estride) + (size_t)rr * rowb;
    uint32_t w[DP_TPL][DW];
#pragma unroll
    for (int q = 0; q < DP_TPL; ++q) {
        const int t = sub + q * DP_LPR;
        if (t < T) load_task<KIND>(base, t, w[q]);
    }
    {
        const float4* src_s = (const float4*)(J.in_s + (size_t)tok * J.kin_s);
        const int kq = J.kin_r / 4;
        const int n4s = J.kin_s / 4, n4 = n4s + K * kq;
        for (int i = threadIdx.x; i < n4; i += blockDim.x) {
            if (i < n4s) {
                ((float4*)dp_act)[i] = src_s[i];
            } else {
                const int q = i - n4s, kk = q / kq, o = q - kk * kq;
                const size_t r = J.gather_ne ? (size_t)tok * J.gather_ne + J.idx[tok * K + kk] : (size_t)tok * K + kk;
                ((float4*)dp_act)[i] = ((const float4*)(J.x + r * J.kin_r))[o];
            }
        }
    }
    __syncthreads();
    const float* xin = shared ? dp_act : dp_act + J.kin_s + (size_t)k * J.kin_r;
    float ga = 0.f;
#pragma unroll
    for (int q = 0; q < DP_TPL; ++q) {
        const int t = sub + q * DP_LPR;
        if (t < T) {
            float xv[64];
            const float4* xp = (const float4*)(xin + (size_t)t * 64);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float4 v = xp[i];
                xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
            }
            float xs[2];
            task_xsum<KIND>(xv, xs);
            ga += task_dot<KIND>(w[q], xv, xs, t);
        }
    }
    ga = group_sum(ga, DP_LPR);
    if (sub == 0) dp_res[wave][rloc] = ga;
    __syncthreads();
    if (threadIdx.x < DP_RB) {
        const int r = blockIdx.x * DP_RB + threadIdx.x;
        float acc = dp_res[0][threadIdx.x];
        for (int kk = 0; kk < K; ++kk) acc += wroute[tok * K + kk] * dp_res[1 + kk][threadIdx.x];
        if (r < rows) {
            float* o = xres + (size_t)tok * rows + r;
            *o = accumulate ? *o + acc : acc;
        }
    }
}

template <int KIND>
static bool down_par_fits(bool has_sh, int K, int E, int SH) {
    return KIND != 4 && has_sh && K <= 8 && E % 64 == 0 && SH % 64 == 0 && E / 64 <= DP_LPR * DP_TPL &&
           SH / 64 <= DP_LPR * DP_TPL;
}

// lanes per row of the fused down kernel: the smallest job's task count
// (capped at 64), raised until every job fits DC_TPJ tasks per lane
static int down_lpr(int E, int SH, bool has_sh) {
    const int Tmin = (has_sh && SH < E ? SH : E) / 64, Tmax = (has_sh && SH > E ? SH : E) / 64;
    int LPR = 64;
    while (LPR > 1 && LPR > Tmin) LPR >>= 1;
    while (LPR < 64 && (Tmax + LPR - 1) / LPR > DC_TPJ) LPR <<= 1;
    return LPR;
}

// out[t] = shared[t] + sum_k w[t,k] * y[slot(t,k)], k in order
// (core/moe_cpu.cpp:265-287). pos maps a slot to its row in y (NULL: y is
// in slot order).
__global__ void k_moe_combine(const float* __restrict__ ysh, const float* __restrict__ y,
                              const int32_t* __restrict__ pos, const float* __restrict__ w, float* __restrict__ out,
                              int N, int K, int d, int accumulate) {
    const int t = blockIdx.x;
    for (int j = threadIdx.x; j < d; j += blockDim.x) {
        float acc = ysh ? ysh[(size_t)t * d + j] : 0.f;
        for (int k = 0; k < K; ++k) {
            const int s = t * K + k;
            const int r = pos ? pos[s] : s;
            acc += w[s] * y[(size_t)r * d + j];
        }
        // accumulate: the residual add x + moe(x) of the caller, the same single addition
        out[(size_t)t * d + j] = accumulate ? out[(size_t)t * d + j] + acc : acc;
    }
}

// Target of the ordered combine: the caller's residual stream `acc_dst` when given (the combine
// then adds into it, and *added records that it did), else `out`. Paths without a combine
// launch (decode down kernels) leave *added at 0 and the caller adds `out` itself.
static void combine_target(float* acc_dst, int* added, float*& out, int& acc) {
    acc = acc_dst != nullptr;
    if (acc) {
        out = acc_dst;
        if (added) *added = 1;
    }
}

// ===================================================== prefill: grouped GEMM
// Tiles of 128 grouped rows x (64 outputs, DUAL: gate and up interleaved per
// wave so one lane holds matching g and u) x 64 K. Rows of a group come from
// `gather` (slot ids -> token rows of x) or are contiguous.
struct GroupGemm {
    const float* A;            // activations
    int lda;                   // row length of A (= K)
    const int32_t* gather;     // grouped position -> slot id (row = slot / topk), or null
    int topk;
    const int32_t* tiles;      // [0]=count, then (group, m0)
    const int32_t* offsets;    // group row ranges [g, g+1)
    const uint8_t* W0;         // group g weights at W0 + g*gstride
    const uint8_t* W1;         // DUAL: up
    size_t gstride, rowb;
    int K, N;                  // K = input length, N = output rows per group
    float* out;                // [rows][N], row = grouped position
    const uint16_t* A16;       // v2: fp16 activations (instead of A)
    uint16_t* out16;           // v2 DUAL: fp16 SwiGLU output (instead of out)
    int rows;                  // skinny kernel without a tile table: one group of `rows` rows
    // skinny non-DUAL epilogue = the ordered combine (k_moe_combine's arithmetic): this product
    // is the shared expert's down projection; out row t = [cout +] (shared + sum_k cw[t K + k]
    // cy[cpos[t K + k]]), k in order
    const float* cy;
    const int32_t* cpos;
    const float* cw;
    int cK, caccum;
    float* cout;
};

template <int KIND, bool DUAL>
__global__ void __launch_bounds__(256) k_moe_group_gemm(GroupGemm P) {
    __shared__ __attribute__((aligned(16))) uint16_t sA[BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t sB[BN * LDS_STRIDE];
    const int tile = blockIdx.x;
    if (tile >= P.tiles[0]) return;
    const int g = P.tiles[1 + 2 * tile], m0 = P.tiles[2 + 2 * tile];
    const int mend = P.offsets[g + 1];
    const int NT = DUAL ? 64 : BN;  // output columns per block
    const int n0 = blockIdx.y * NT;
    if (n0 >= P.N) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = tid >> 1, lh = tid & 1;
    const int am = m0 + lr;
    const bool arow_ok = am < mend;
    int arow = arow_ok ? am : m0;
    if (P.gather) arow = P.gather[arow] / P.topk;
    const float* xrow = P.A + (size_t)arow * P.lda;
    // weight row of LDS row lr
    int brow;
    const uint8_t* Wm;
    if (DUAL) {
        const int wn = lr >> 6, r = lr & 63;
        brow = n0 + 32 * wn + (r & 31);
        Wm = (r < 32 ? P.W0 : P.W1) + (size_t)g * P.gstride;
    } else {
        brow = n0 + lr;
        Wm = P.W0 + (size_t)g * P.gstride;
    }
    const bool brow_ok = brow < P.N;
    const uint8_t* wrow = Wm + (size_t)(brow_ok ? brow : 0) * P.rowb;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int T = P.K / BK;
    float4 xa[8];
    WLoad<KIND> wl;
    auto gload = [&](int t) {
        const float4* xp = (const float4*)(xrow + (size_t)t * BK + lh * 32);
#pragma unroll
        for (int i = 0; i < 8; ++i) xa[i] = xp[i];
        wl.load(wrow, t, lh);
    };
    gload(0);
    for (int t = 0; t < T; ++t) {
        {
            float v[32];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v[4 * i] = xa[i].x; v[4 * i + 1] = xa[i].y; v[4 * i + 2] = xa[i].z; v[4 * i + 3] = xa[i].w;
            }
            if (!arow_ok) {
#pragma unroll
                for (int i = 0; i < 32; ++i) v[i] = 0.f;
            }
            store_f16x32(sA + lr * LDS_STRIDE + lh * 32, v);
            wl.decode(v);
            if (!brow_ok) {
#pragma unroll
                for (int i = 0; i < 32; ++i) v[i] = 0.f;
            }
            store_f16x32(sB + lr * LDS_STRIDE + lh * 32, v);
        }
        __syncthreads();
        if (t + 1 < T) gload(t + 1);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int kofs = ks * 16 + (lane >> 5) * 8;
            f16x8 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                a[i] = *(const f16x8*)(sA + (wm + i * 32 + (lane & 31)) * LDS_STRIDE + kofs);
                b[i] = *(const f16x8*)(sB + (wn + i * 32 + (lane & 31)) * LDS_STRIDE + kofs);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int row = m0 + wm + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            if (row >= mend) continue;
            if (DUAL) {
                const int col = n0 + 32 * (wave & 1) + (lane & 31);
                if (col < P.N) {
                    const float gv = acc[i][0][e], uv = acc[i][1][e];
                    P.out[(size_t)row * P.N + col] = gv / (1.0f + expf(-gv)) * uv;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int col = n0 + wn + j * 32 + (lane & 31);
                    if (col < P.N) P.out[(size_t)row * P.N + col] = acc[i][j][e];
                }
            }
        }
    }
}

// v2 of the grouped GEMM (kinds 2, 3, 4): fp16 activations converted once
// (gathered rows are read with 16-byte loads), double-buffered LDS with one
// barrier per K step, and_or/fma_mix weight decode (gemm.hip), the DUAL
// (gate/up) epilogue writes the SwiGLU output as fp16 for the down GEMM.
template <int KIND, bool DUAL>
__global__ void __launch_bounds__(256, 2) k_moe_group_gemm2(GroupGemm P) {
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * LDS_STRIDE];
    const int tile = blockIdx.x;
    if (tile >= P.tiles[0]) return;
    const int g = P.tiles[1 + 2 * tile], m0 = P.tiles[2 + 2 * tile];
    const int mend = P.offsets[g + 1];
    const int NT = DUAL ? 64 : BN;  // output columns per block
    const int n0 = blockIdx.y * NT;
    if (n0 >= P.N) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ar = tid >> 3, ac = (tid & 7) * 8;
    const uint16_t* xrows[4];
    bool aok[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int am = m0 + ar + 32 * i;
        aok[i] = am < mend;
        int arow = aok[i] ? am : m0;
        if (P.gather) arow = P.gather[arow] / P.topk;
        xrows[i] = P.A16 + (size_t)arow * P.lda;
    }
    const int lr = tid >> 1, lh = tid & 1;
    int brow;
    const uint8_t* Wm;
    if (DUAL) {
        const int wn = lr >> 6, r = lr & 63;
        brow = n0 + 32 * wn + (r & 31);
        Wm = (r < 32 ? P.W0 : P.W1) + (size_t)g * P.gstride;
    } else {
        brow = n0 + lr;
        Wm = P.W0 + (size_t)g * P.gstride;
    }
    const bool brow_ok = brow < P.N;
    const uint8_t* wrow = Wm + (size_t)(brow_ok ? brow : 0) * P.rowb;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int T = P.K / BK;
    uint32_t magic = 0x64006400u;
    asm volatile("" : "+v"(magic));
    gh_u32x4v xa[4];
    WLoad<KIND> wl;
#pragma unroll
    for (int i = 0; i < 4; ++i) xa[i] = *(const gh_u32x4v*)(xrows[i] + ac);
    wl.load(wrow, 0, lh);
    int buf = 0;
    for (int t = 0; t < T; ++t, buf ^= 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            gh_u32x4v v = xa[i];
            if (!aok[i]) v = gh_u32x4v{0u, 0u, 0u, 0u};
            *(gh_u32x4v*)(sA[buf] + (ar + 32 * i) * LDS_STRIDE + ac) = v;
        }
        {
            uint16_t* dst = sB[buf] + lr * LDS_STRIDE + lh * 32;
            if (brow_ok) {
                decode16<KIND>(wl, dst, magic);
            } else {
                float z[32];
#pragma unroll
                for (int i = 0; i < 32; ++i) z[i] = 0.f;
                store_f16x32(dst, z);
            }
        }
        __syncthreads();
        if (t + 1 < T) {
#pragma unroll
            for (int i = 0; i < 4; ++i) xa[i] = *(const gh_u32x4v*)(xrows[i] + (size_t)(t + 1) * BK + ac);
            wl.load(wrow, t + 1, lh);
        }
        const uint16_t* cA = sA[buf];
        const uint16_t* cB = sB[buf];
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int kofs = ks * 16 + (lane >> 5) * 8;
            f16x8 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                a[i] = *(const f16x8*)(cA + (wm + i * 32 + (lane & 31)) * LDS_STRIDE + kofs);
                b[i] = *(const f16x8*)(cB + (wn + i * 32 + (lane & 31)) * LDS_STRIDE + kofs);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int row = m0 + wm + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            if (row >= mend) continue;
            if (DUAL) {
                const int col = n0 + 32 * (wave & 1) + (lane & 31);
                if (col < P.N) {
                    const float gv = acc[i][0][e], uv = acc[i][1][e];
                    P.out16[(size_t)row * P.N + col] = f32_to_f16(gv / (1.0f + expf(-gv)) * uv);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int col = n0 + wn + j * 32 + (lane & 31);
                    if (col < P.N) P.out[(size_t)row * P.N + col] = acc[i][j][e];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Skinny grouped GEMM (Q4_K, K = 256 or 512): tiles of 32 grouped rows x 64 weight
// rows (DUAL: 32 gate + the matching 32 up rows, i.e. 32 outputs), the WHOLE K in
// one pass: the block's 32 activation rows (fp16) go to LDS once, and each lane
// requests every weight byte its MFMA B operands need (8 values per k-step of 32,
// plus the super-block headers) before the first multiply, so a block waits for
// memory once instead of once per K step (the 128-row tiles of k_moe_group_gemm2
// spent ~2 us per K step on a group of ~32 rows). Wave w owns weight rows
// 16w..16w+15 of the tile: v_mfma_f32_16x16x32_f16 with the activations as A
// (two 16-row halves) and the lane's dequantised weights as B (lane: weight row
// l % 16, values 8 (l / 16) .. +7 of the k-step, one sub-block of one super-block).
// Weights are rounded to fp16 after dequantisation (d sc q - dmin m in fp32),
// as in the 128-row kernel. KIND 2 (Q8_0): per k-step one 34-byte block, the lane's
// 8 codes and the block scale read as dwords (gemm_tile.h sk_q8_bfrag), q d rounded once.
typedef sk_f16x8 f16x8s;
typedef float f32x4s __attribute__((ext_vector_type(4)));
template <bool DUAL, int KK, int WR, int KIND = 3>
__global__ void __launch_bounds__(512) k_moe_skinny(GroupGemm P0, GroupGemm P1, int ntiles0) {
    // blocks [0, ntiles0) take problem P0, the rest problem P1 (the shared expert beside the
    // routed ones in one launch)
    const bool second = (int)blockIdx.x >= ntiles0;
    const GroupGemm& P = second ? P1 : P0;
    // WR waves own weight rows, 8 / WR wave groups split K (steps kg*NS ..); the groups' sums
    // meet group 0's in LDS, added in group order. DUAL takes WR = 4 (gate rows in waves 0-1,
    // up rows in 2-3); a plain product takes fewer weight-row waves when its grid is small.
    static_assert(!DUAL || WR == 4, "gate/up tiles pair waves 0-1 with 2-3");
    constexpr int NWK = 8 / WR;
    constexpr int SA = KK + 8;  // LDS row stride (fp16)
    constexpr int NS = KK / 32 / NWK;
    static_assert(NS >= 1 && 8 % NS == 0, "a group's K steps stay within one super-block");
    __shared__ __attribute__((aligned(16))) _Float16 sA[32 * SA];
    __shared__ float sU[DUAL ? 32 * 33 : 1];
    __shared__ float sR[(NWK - 1) * WR * 64 * 8];
    const int tile = second ? (int)blockIdx.x - ntiles0 : (int)blockIdx.x;
    const bool table = P.tiles != nullptr;
    if (table && tile >= P.tiles[0]) return;
    const int g = table ? P.tiles[1 + 2 * tile] : 0, m0 = table ? P.tiles[2 + 2 * tile] : 32 * tile;
    const int mend = table ? P.offsets[g + 1] : P.rows;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave % WR, kg = wave / WR;
    constexpr int K = KK;
    // weight row of this lane: DUAL waves 0-1 gate, 2-3 up rows of outputs n0 .. n0+31
    const int NT = DUAL ? 32 : 16 * WR;
    const int n0 = blockIdx.y * NT;
    if (n0 >= P.N) return;  // the other problem's output range is wider
    const int col = lane & 15, kq = lane >> 4;
    const int nrow = DUAL ? n0 + 16 * (wr & 1) + col : n0 + 16 * wr + col;
    const bool nok = nrow < P.N;
    const uint8_t* W = (DUAL && wr >= 2 ? P.W1 : P.W0) + (size_t)g * P.gstride;
    const uint8_t* wrow = W + (size_t)(nok ? nrow : 0) * P.rowb;
    const int s0 = kg * NS;
    // every weight byte of the lane, requested first (Q4_K: the super-block header and 8 code
    // bytes per k-step; Q8_0: per k-step the dwords holding the block scale and codes 8 kq ..)
    uint4 hdr;
    uint2 qb[KIND == 3 ? NS : 1];
    uint32_t q8w[KIND == 2 ? NS : 1][4];
    if constexpr (KIND == 3) {
        hdr = *(const uint4*)(wrow + (size_t)(s0 >> 3) * 144);
#pragma unroll
        for (int s = 0; s < NS; ++s) qb[s] = *(const uint2*)(wrow + sk_q4k_qofs(s0 + s, kq));
    } else {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int ob = 34 * (s0 + s), oc = ob + 2 + 8 * kq;
            const uint32_t* cw = (const uint32_t*)(wrow + (oc & ~3));
            q8w[s][0] = *(const uint32_t*)(wrow + (ob & ~3));
            q8w[s][1] = cw[0];
            q8w[s][2] = cw[1];
            // the third dword only when the codes start mid-dword: otherwise it lies past the
            // block (for a row's last block, past the row and possibly past the allocation)
            q8w[s][3] = (oc & 3) ? cw[2] : 0u;
        }
    }
    // combine epilogue: the rows' slot positions and weights (up to top-2 here), requested now
    constexpr int CKM = 2;
    int cp[2][4][CKM];
    float cwv[2][4][CKM];
    const bool comb = !DUAL && P.cout && P.cK <= CKM && kg == 0;
    if (comb) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int k = 0; k < CKM; ++k) {
                    const int m = m0 + 16 * h + 4 * kq + j;
                    const bool ok = m < mend && k < P.cK;
                    cp[h][j][k] = ok ? P.cpos[m * P.cK + k] : 0;
                    cwv[h][j][k] = ok ? P.cw[m * P.cK + k] : 0.f;
                }
    }
    // the 32 activation rows (grouped positions m0 .. m0+31) into LDS
    const int rq = K / 8;  // 16-byte pieces per row
    for (int e = tid; e < 32 * rq; e += 512) {
        const int r = e / rq, c = e - r * rq, m = m0 + r;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (m < mend) {
            const int arow = P.gather ? P.gather[m] / P.topk : m;
            if (P.A16) {
                v = *(const uint4*)(P.A16 + (size_t)arow * P.lda + 8 * c);
            } else {  // fp32 rows, converted here
                const float4* src = (const float4*)(P.A + (size_t)arow * P.lda + 8 * c);
                const float4 a = src[0], b = src[1];
                f16x8s hv;
                hv[0] = (_Float16)a.x; hv[1] = (_Float16)a.y; hv[2] = (_Float16)a.z; hv[3] = (_Float16)a.w;
                hv[4] = (_Float16)b.x; hv[5] = (_Float16)b.y; hv[6] = (_Float16)b.z; hv[7] = (_Float16)b.w;
                v = __builtin_bit_cast(uint4, hv);
            }
        }
        *(uint4*)(sA + r * SA + 8 * c) = v;
    }
    __syncthreads();
    f32x4s acc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) acc[h] = f32x4s{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        f16x8s bv;
        if constexpr (KIND == 3) {
            bv = sk_q4k_bfrag(hdr, qb[s], (s0 + s) & 7, nok);
        } else {
            const int ob = 34 * (s0 + s), oc = ob + 2 + 8 * kq;
            bv = sk_q8_bfrag(q8w[s], ob & 3, oc & 3, nok);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const f16x8s av = *(const f16x8s*)(sA + (16 * h + (lane & 15)) * SA + 32 * (s0 + s) + 8 * kq);
            acc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[h], 0, 0, 0);
        }
    }
    if (kg > 0) {
        float* r = sR + (((kg - 1) * WR + wr) * 64 + lane) * 8;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j) r[4 * h + j] = acc[h][j];
    }
    __syncthreads();
    if (kg == 0) {
#pragma unroll
        for (int gk = 1; gk < NWK; ++gk) {
            const float* r = sR + (((gk - 1) * WR + wr) * 64 + lane) * 8;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[h][j] += r[4 * h + j];
        }
    }
    // acc[h][j] of waves 0-3: row 16 h + 4 (lane / 16) + j, weight row column lane % 16
    if (DUAL) {
        if (kg == 0 && wr >= 2) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int j = 0; j < 4; ++j) sU[(16 * h + 4 * kq + j) * 33 + 16 * (wr & 1) + col] = acc[h][j];
        }
        __syncthreads();
        if (kg == 0 && wr < 2) {
            const int oc = n0 + 16 * wr + col;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r = 16 * h + 4 * kq + j, m = m0 + r;
                    if (m < mend && oc < P.N) {
                        const float gv = acc[h][j], uv = sU[r * 33 + 16 * wr + col];
                        P.out16[(size_t)m * P.N + oc] = f32_to_f16(gv / (1.0f + expf(-gv)) * uv);
                    }
                }
        }
    } else if (kg == 0 && comb) {
        // the ordered combine of tokens m, output nrow: every load of the lane first (the routed
        // outputs and the accumulated rows), then the stores, so the loads are not serialised
        // behind stores the compiler cannot tell apart from them
        float cyv[2][4][CKM], ov[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = m0 + 16 * h + 4 * kq + j;
                const bool ok = m < mend && nok;
#pragma unroll
                for (int k = 0; k < CKM; ++k)
                    cyv[h][j][k] = ok && k < P.cK ? P.cy[(size_t)cp[h][j][k] * P.N + nrow] : 0.f;
                ov[h][j] = ok && P.caccum ? P.cout[(size_t)m * P.N + nrow] : 0.f;
            }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = m0 + 16 * h + 4 * kq + j;
                if (m < mend && nok) {
                    float v = acc[h][j];
#pragma unroll
                    for (int k = 0; k < CKM; ++k)
                        if (k < P.cK) v += cwv[h][j][k] * cyv[h][j][k];
                    P.cout[(size_t)m * P.N + nrow] = P.caccum ? ov[h][j] + v : v;
                }
            }
    } else if (kg == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = m0 + 16 * h + 4 * kq + j;
                if (m < mend && nok) {
                    if (P.cout) {  // more than CKM experts per token
                        float v = acc[h][j];
                        for (int k = 0; k < P.cK; ++k) {
                            const int sl = m * P.cK + k;
                            v += P.cw[sl] * P.cy[(size_t)P.cpos[sl] * P.N + nrow];
                        }
                        float* o = P.cout + (size_t)m * P.N + nrow;
                        *o = P.caccum ? *o + v : v;
                    } else {
                        P.out[(size_t)m * P.N + nrow] = acc[h][j];
                    }
                }
            }
    }
}

// the skinny kernel for K = 256 or 512 (the caller checks K); grid (tiles, outputs / 32 or
// 16 WR). P1 (optional, ntiles1 blocks) runs in the same launch after P0's ntiles0; both take
// the same K. A plain product takes 64, 32 or 16 weight rows per block: the first that gives
// 256 blocks, or 16.
template <int KK, int WR, bool DUAL, int KIND>
static void skinny_go(dim3 grid, const GroupGemm& P0, const GroupGemm& Q1, int ntiles0) {
    hipLaunchKernelGGL((k_moe_skinny<DUAL, KK, WR, KIND>), grid, dim3(512), 0, stream(), P0, Q1, ntiles0);
}
template <bool DUAL, int KIND>
static void launch_skinny(const GroupGemm& P0, int ntiles0, const GroupGemm* P1 = nullptr, int ntiles1 = 0) {
    const int nw = std::max(P0.N, P1 ? P1->N : 0);
    const GroupGemm Q1 = P1 ? *P1 : GroupGemm{};
    const int nt = ntiles0 + ntiles1;
    if constexpr (DUAL) {
        const dim3 grid(nt, cdiv(nw, 32));
        if (P0.K == 256) skinny_go<256, 4, true, KIND>(grid, P0, Q1, ntiles0);
        else skinny_go<512, 4, true, KIND>(grid, P0, Q1, ntiles0);
    } else {
        int wr = 1;
        for (int c = 4; c >= 2; c >>= 1)
            if ((int64_t)nt * cdiv(nw, 16 * c) >= 256) { wr = c; break; }
        const dim3 grid(nt, cdiv(nw, 16 * wr));
        if (P0.K == 256) {
            if (wr == 4) skinny_go<256, 4, false, KIND>(grid, P0, Q1, ntiles0);
            else if (wr == 2) skinny_go<256, 2, false, KIND>(grid, P0, Q1, ntiles0);
            else skinny_go<256, 1, false, KIND>(grid, P0, Q1, ntiles0);
        } else {
            if (wr == 4) skinny_go<512, 4, false, KIND>(grid, P0, Q1, ntiles0);
            else if (wr == 2) skinny_go<512, 2, false, KIND>(grid, P0, Q1, ntiles0);
            else skinny_go<512, 1, false, KIND>(grid, P0, Q1, ntiles0);
        }
    }
}

// tile table of one group covering rows [0, N)
__global__ void k_single_group_tiles(int32_t* tiles, int32_t* offs, int N, int bm) {
    const int nt = (N + bm - 1) / bm;
    for (int i = threadIdx.x; i < nt; i += blockDim.x) {
        tiles[1 + 2 * i] = 0;
        tiles[2 + 2 * i] = i * bm;
    }
    if (threadIdx.x == 0) {
        tiles[0] = nt;
        offs[0] = 0;
        offs[1] = N;
    }
}

template <int KIND>
static int moe_kind(const float* x, const float* w_route, const int32_t* idx, const void* gates, const void* ups,
                    const void* downs, const void* sh_g, const void* sh_u, const void* sh_d, float* out, float* acc_dst,
                    int* added, int N, int d, int E, int ne, int K, int SH, const float* rlogits = nullptr,
                    const float* rbias = nullptr, float* rprobs = nullptr) {
    const int S = N * K;
    const bool has_sh = sh_g && sh_u && sh_d;
    const size_t rowb_d = KIND == 4 ? (size_t)d * 2 : row_bytes(KIND, d);
    const size_t rowb_E = KIND == 4 ? (size_t)E * 2 : row_bytes(KIND, E);
    const size_t rowb_SH = KIND == 4 ? (size_t)SH * 2 : row_bytes(KIND, SH);
    float* act = (float*)workspace(WS_MOE_ACT, (size_t)S * E * 4);
    float* yr = (float*)workspace(WS_MOE_OUT, (size_t)S * d * 4);
    float* shb = (float*)workspace(WS_MOE_SHARED, (size_t)N * ((size_t)SH + d) * 4);
    if (!act || !yr || !shb) return fail(GH_ENOMEM, "moe: workspace");
    float* sh_act = shb;
    float* sh_y = shb + (size_t)N * SH;

    if (N <= 8) {
        // decode: two grouped GEMV launches (gate+up+SwiGLU, down) + combine
        GemvJobs J{};
        J.x = x; J.idx = idx; J.S = S; J.N = has_sh ? N : 0; J.K = K; J.d = d;
        J.wa = (const uint8_t*)gates; J.wb = (const uint8_t*)ups; J.estride = (size_t)E * rowb_d;
        J.sa = (const uint8_t*)sh_g; J.sb = (const uint8_t*)sh_u;
        J.rows_r = E; J.rows_s = SH; J.kin_r = d; J.kin_s = d; J.rowb_r = rowb_d; J.rowb_s = rowb_d;
        J.out_r = act; J.out_s = sh_act;
        const int maxrows = has_sh ? (E > SH ? E : SH) : E;
        auto rows_per_block = [&](int kin) {
            int T = kin / 64, LPR = 64;
            while (LPR > 1 && LPR > T) LPR >>= 1;
            return 4 * (64 / LPR);
        };
        dim3 g1(cdiv(maxrows, rows_per_block(d)), S + J.N);
        if (rlogits) {  // the selection runs in the gate/up blocks, which write idx / w (/ probs)
            J.rlogits = rlogits; J.rbias = rbias; J.ne = ne; J.ridx = const_cast<int32_t*>(idx);
            J.rwout = const_cast<float*>(w_route); J.rprobs = rprobs;
            hipLaunchKernelGGL((k_moe_gemv<KIND, true, false, false, true>), g1, dim3(256), 0, stream(), J);
        } else {
            hipLaunchKernelGGL((k_moe_gemv<KIND, true>), g1, dim3(256), 0, stream(), J);
        }
        GH_LAUNCHED("k_moe_gemv(gate/up)");
        GemvJobs D{};
        D.x = act; D.idx = idx; D.S = S; D.N = J.N; D.K = K; D.d = d;
        D.wa = (const uint8_t*)downs; D.estride = (size_t)d * rowb_E; D.sa = (const uint8_t*)sh_d;
        D.rows_r = d; D.rows_s = d; D.kin_r = E; D.kin_s = SH; D.rowb_r = rowb_E; D.rowb_s = rowb_SH;
        D.in_s = sh_act;
        // down projections + ordered combine in one launch
        const int LPR = down_lpr(E, SH, has_sh);
        const int rpb = 4 * (64 / LPR);
        const size_t lds = ((has_sh ? (size_t)SH : 0) + (size_t)K * E) * 4;
        if (lds > 60 * 1024) {  // activations do not fit LDS: per-expert outputs + ordered combine
            D.out_r = yr; D.out_s = sh_y;
            const int rpb2 = rows_per_block(E) < rows_per_block(SH) ? rows_per_block(E) : rows_per_block(SH);
            hipLaunchKernelGGL((k_moe_gemv<KIND, false>), dim3(cdiv(d, rpb2), S + D.N), dim3(256), 0, stream(), D);
            GH_LAUNCHED("k_moe_gemv(down)");
            {
                float* cdst = out;
                int cacc = 0;
                combine_target(acc_dst, added, cdst, cacc);
                hipLaunchKernelGGL(k_moe_combine, dim3(N), dim3(256), 0, stream(), has_sh ? sh_y : nullptr, yr,
                                   nullptr, w_route, cdst, N, K, d, cacc);
            }
            GH_LAUNCHED("k_moe_combine");
            return GH_OK;
        }
        if (down_par_fits<KIND>(has_sh, K, E, SH)) {
            hipLaunchKernelGGL((k_moe_down_par<KIND>), dim3(cdiv(d, DP_RB), N), dim3(64 * (K + 1)), lds, stream(), D,
                               w_route, out, 0);
        } else {
            hipLaunchKernelGGL((k_moe_down_combine<KIND>), dim3(cdiv(d, rpb), N), dim3(256), lds, stream(), D, w_route,
                               out, LPR, 0);
        }
        GH_LAUNCHED("k_moe_down_combine");
        return GH_OK;
    }
    // prefill: permutation, grouped gate/up GEMM, grouped down GEMM, combine. Small groups
    // (a few dozen rows per expert) take the skinny 32-row tiles with the whole K in one pass.
    auto kfits = [](int k) { return k == 256 || k == 512; };
    const bool skinny = (KIND == 3 || KIND == 2) && (size_t)S <= (size_t)64 * ne && kfits(d) && kfits(E) && (!has_sh || kfits(SH));
    const int bm = skinny ? 32 : BM;
    int32_t* perm = (int32_t*)workspace(WS_MOE_XG, ((size_t)2 * S + ne + 1 + 1 + 2 * ((size_t)S / bm + ne + 1)) * 4);
    if (!perm) return fail(GH_ENOMEM, "moe: workspace");
    int32_t* grouped = perm;
    int32_t* pos = perm + S;
    int32_t* offsets = pos + S;
    int32_t* tiles = offsets + ne + 1;
    const int max_tiles = S / bm + ne + 1;
    int rc = permute(idx, S, ne, grouped, offsets, pos, tiles, bm);
    if (rc) return rc;
    if constexpr (KIND == 2 || KIND == 3 || KIND == 4) {
        // v2: fp16 activations converted once; gate/up write fp16 SwiGLU rows
        uint16_t* x16 = (uint16_t*)workspace(WS_MOE_X16, (size_t)N * d * 2);
        if (!x16) return fail(GH_ENOMEM, "moe: workspace");
        uint16_t* act16 = (uint16_t*)act;         // [S][E] fp16 in the fp32 buffer
        uint16_t* sh_act16 = (uint16_t*)sh_act;   // [N][SH] fp16
        if (!skinny) {  // the skinny gate/up converts its fp32 rows itself
            rc = launch_to_f16(x, x16, (int64_t)N * d);
            if (rc) return rc;
        }
        GroupGemm P{};
        P.A16 = skinny ? nullptr : x16; P.A = x; P.lda = d; P.gather = grouped; P.topk = K; P.tiles = tiles;
        P.offsets = offsets;
        P.W0 = (const uint8_t*)gates; P.W1 = (const uint8_t*)ups; P.gstride = (size_t)E * rowb_d; P.rowb = rowb_d;
        P.K = d; P.N = E; P.out16 = act16;
        GroupGemm Q{};
        Q.A16 = act16; Q.lda = E; Q.gather = nullptr; Q.topk = 1; Q.tiles = tiles; Q.offsets = offsets;
        Q.W0 = (const uint8_t*)downs; Q.gstride = (size_t)d * rowb_E; Q.rowb = rowb_E; Q.K = E; Q.N = d; Q.out = yr;
        if (skinny) {
            // gate/up of the routed experts and of the shared expert (one group of N rows, no tile
            // table) in one launch; the routed downs; the shared down with the ordered combine
            // (and the residual add) in its epilogue
            GroupGemm R{};
            R.A = x; R.lda = d; R.topk = 1; R.rows = N;
            R.W0 = (const uint8_t*)sh_g; R.W1 = (const uint8_t*)sh_u; R.rowb = rowb_d; R.K = d; R.N = SH;
            R.out16 = sh_act16;
            launch_skinny<true, KIND>(P, max_tiles, has_sh ? &R : nullptr, has_sh ? cdiv(N, 32) : 0);
            GH_LAUNCHED("k_moe_skinny(gate/up)");
            launch_skinny<false, KIND>(Q, max_tiles);
            GH_LAUNCHED("k_moe_skinny(down)");
            if (has_sh) {
                float* cdst = out;
                int cacc = 0;
                combine_target(acc_dst, added, cdst, cacc);
                GroupGemm U{};
                U.A16 = sh_act16; U.lda = SH; U.topk = 1; U.rows = N;
                U.W0 = (const uint8_t*)sh_d; U.rowb = rowb_SH; U.K = SH; U.N = d;
                U.cy = yr; U.cpos = pos; U.cw = w_route; U.cK = K; U.caccum = cacc; U.cout = cdst;
                launch_skinny<false, KIND>(U, cdiv(N, 32));
                GH_LAUNCHED("k_moe_skinny(shared down + combine)");
                return GH_OK;
            }
        } else {
            hipLaunchKernelGGL((k_moe_group_gemm2<KIND, true>), dim3(max_tiles, cdiv(E, 64)), dim3(256), 0, stream(), P);
            GH_LAUNCHED("k_moe_group_gemm2(gate/up)");
            hipLaunchKernelGGL((k_moe_group_gemm2<KIND, false>), dim3(max_tiles, cdiv(d, BN)), dim3(256), 0, stream(), Q);
            GH_LAUNCHED("k_moe_group_gemm2(down)");
        }
        if (has_sh) {
            int32_t* sh_tiles = (int32_t*)workspace(WS_MOE_H, ((size_t)2 * (N / bm + 2) + 1 + 2) * 4);
            if (!sh_tiles) return fail(GH_ENOMEM, "moe: workspace");
            int32_t* sh_off = sh_tiles + 2 * (N / bm + 2) + 1;
            const int nt = cdiv(N, bm);
            hipLaunchKernelGGL(k_single_group_tiles, dim3(1), dim3(64), 0, stream(), sh_tiles, sh_off, N, bm);
            GH_LAUNCHED("k_single_group_tiles");
            GroupGemm R{};
            R.A16 = x16; R.lda = d; R.gather = nullptr; R.topk = 1; R.tiles = sh_tiles; R.offsets = sh_off;
            R.W0 = (const uint8_t*)sh_g; R.W1 = (const uint8_t*)sh_u; R.gstride = 0; R.rowb = rowb_d;
            R.K = d; R.N = SH; R.out16 = sh_act16;
            hipLaunchKernelGGL((k_moe_group_gemm2<KIND, true>), dim3(nt, cdiv(SH, 64)), dim3(256), 0, stream(), R);
            GroupGemm U{};
            U.A16 = sh_act16; U.lda = SH; U.gather = nullptr; U.topk = 1; U.tiles = sh_tiles; U.offsets = sh_off;
            U.W0 = (const uint8_t*)sh_d; U.gstride = 0; U.rowb = rowb_SH; U.K = SH; U.N = d; U.out = sh_y;
            hipLaunchKernelGGL((k_moe_group_gemm2<KIND, false>), dim3(nt, cdiv(d, BN)), dim3(256), 0, stream(), U);
            GH_LAUNCHED("k_moe_group_gemm2(shared)");
        }
        {
            float* cdst = out;
            int cacc = 0;
            combine_target(acc_dst, added, cdst, cacc);
            hipLaunchKernelGGL(k_moe_combine, dim3(N), dim3(256), 0, stream(), has_sh ? sh_y : nullptr, yr, pos,
                               w_route, cdst, N, K, d, cacc);
        }
        GH_LAUNCHED("k_moe_combine");
        return GH_OK;
    }
    GroupGemm P{};
    P.A = x; P.lda = d; P.gather = grouped; P.topk = K; P.tiles = tiles; P.offsets = offsets;
    P.W0 = (const uint8_t*)gates; P.W1 = (const uint8_t*)ups; P.gstride = (size_t)E * rowb_d; P.rowb = rowb_d;
    P.K = d; P.N = E; P.out = act;
    hipLaunchKernelGGL((k_moe_group_gemm<KIND, true>), dim3(max_tiles, cdiv(E, 64)), dim3(256), 0, stream(), P);
    GH_LAUNCHED("k_moe_group_gemm(gate/up)");
    GroupGemm Q{};
    Q.A = act; Q.lda = E; Q.gather = nullptr; Q.topk = 1; Q.tiles = tiles; Q.offsets = offsets;
    Q.W0 = (const uint8_t*)downs; Q.gstride = (size_t)d * rowb_E; Q.rowb = rowb_E; Q.K = E; Q.N = d; Q.out = yr;
    hipLaunchKernelGGL((k_moe_group_gemm<KIND, false>), dim3(max_tiles, cdiv(d, BN)), dim3(256), 0, stream(), Q);
    GH_LAUNCHED("k_moe_group_gemm(down)");
    if (has_sh) {
        // the shared expert is one group over all N tokens
        int32_t* sh_tiles = (int32_t*)workspace(WS_MOE_H, ((size_t)2 * (N / BM + 2) + 1 + 2) * 4);
        if (!sh_tiles) return fail(GH_ENOMEM, "moe: workspace");
        int32_t* sh_off = sh_tiles + 2 * (N / BM + 2) + 1;
        const int nt = cdiv(N, BM);
        hipLaunchKernelGGL(k_single_group_tiles, dim3(1), dim3(64), 0, stream(), sh_tiles, sh_off, N, BM);
        GH_LAUNCHED("k_single_group_tiles");
        GroupGemm R{};
        R.A = x; R.lda = d; R.gather = nullptr; R.topk = 1; R.tiles = sh_tiles; R.offsets = sh_off;
        R.W0 = (const uint8_t*)sh_g; R.W1 = (const uint8_t*)sh_u; R.gstride = 0; R.rowb = rowb_d;
        R.K = d; R.N = SH; R.out = sh_act;
        hipLaunchKernelGGL((k_moe_group_gemm<KIND, true>), dim3(nt, cdiv(SH, 64)), dim3(256), 0, stream(), R);
        GroupGemm U{};
        U.A = sh_act; U.lda = SH; U.gather = nullptr; U.topk = 1; U.tiles = sh_tiles; U.offsets = sh_off;
        U.W0 = (const uint8_t*)sh_d; U.gstride = 0; U.rowb = rowb_SH; U.K = SH; U.N = d; U.out = sh_y;
        hipLaunchKernelGGL((k_moe_group_gemm<KIND, false>), dim3(nt, cdiv(d, BN)), dim3(256), 0, stream(), U);
        GH_LAUNCHED("k_moe_group_gemm(shared)");
    }
    {
        float* cdst = out;
        int cacc = 0;
        combine_target(acc_dst, added, cdst, cacc);
        hipLaunchKernelGGL(k_moe_combine, dim3(N), dim3(256), 0, stream(), has_sh ? sh_y : nullptr, yr, pos, w_route,
                           cdst, N, K, d, cacc);
    }
    GH_LAUNCHED("k_moe_combine");
    return GH_OK;
}

// Decode MoE FFN of N <= 8 tokens as three launches, fused with the block
// around it: xres += MoE(rmsnorm(xres) * nw). (1) norm + route, (2) grouped
// gate/up GEMV with SwiGLU, (3) grouped down GEMV + combine + residual.
template <int KIND>
static int moe_decode_fused_kind(float* xres, const float* nw, float eps, const float* rw, const float* bias,
                                 const void* gates, const void* ups, const void* downs, const void* sh_g,
                                 const void* sh_u, const void* sh_d, int N, int d, int E, int ne, int K, int SH) {
    const int S = N * K;
    const bool has_sh = sh_g && sh_u && sh_d;
    const size_t rowb_d = KIND == 4 ? (size_t)d * 2 : row_bytes(KIND, d);
    const size_t rowb_E = KIND == 4 ? (size_t)E * 2 : row_bytes(KIND, E);
    const size_t rowb_SH = KIND == 4 ? (size_t)SH * 2 : row_bytes(KIND, SH);
    char* r = (char*)workspace(WS_MOE_ROUTE, (size_t)S * 8);
    float* xn = (float*)workspace(WS_MOE_XG, (size_t)N * d * 4);
    float* act = (float*)workspace(WS_MOE_ACT, (size_t)N * (ne > K ? ne : K) * E * 4);
    float* sh_act = (float*)workspace(WS_MOE_SHARED, (size_t)N * ((size_t)SH + d) * 4);
    if (!r || !xn || !act || !sh_act) return fail(GH_ENOMEM, "moe: workspace");
    int32_t* idx = (int32_t*)r;
    float* w = (float*)(r + (size_t)S * 4);
    // a small router runs inside the gate/up kernel (one launch less); a large one on its own
    const int gw = route_window(d, ne, N);
    const size_t rlds = route_lds(d, ne, N);
    const bool fused_route = K <= 8 && gw >= d / 4 && rlds <= 32 * 1024 && (size_t)ne * d <= 16384;
    // small expert sets: every expert's gate/up is computed (at most a few MB of weights) so the
    // routing runs beside the GEMVs instead of in front of them
    const bool allexp = fused_route && has_sh && ne > K && (size_t)ne * E * d <= ((size_t)4 << 20);
    // a large router: its logits by k_route_chain, the selection inside the gate/up blocks
    const bool chain = !fused_route && ne <= 64 && d % 4 == 0 && d <= 4096;
    float* logits = nullptr;
    if (chain) {
        logits = (float*)workspace(WS_MOE_TERMS, (size_t)N * ne * 4);
        if (!logits) return fail(GH_ENOMEM, "moe: workspace");
        hipLaunchKernelGGL(k_route_chain, dim3(ne, N), dim3(64), 0, stream(), xres, rw, logits, d, ne, nw, eps, xn);
        GH_LAUNCHED("k_route_chain");
    } else if (!fused_route) {
        const int rc = launch_route(xres, rw, bias, nullptr, idx, w, N, d, ne, K, nw, eps, xn);
        if (rc) return rc;
    }
    GemvJobs J{};
    J.x = xn; J.idx = idx; J.S = S; J.N = has_sh ? N : 0; J.K = K; J.d = d;
    J.wa = (const uint8_t*)gates; J.wb = (const uint8_t*)ups; J.estride = (size_t)E * rowb_d;
    J.sa = (const uint8_t*)sh_g; J.sb = (const uint8_t*)sh_u;
    J.rows_r = E; J.rows_s = SH; J.kin_r = d; J.kin_s = d; J.rowb_r = rowb_d; J.rowb_s = rowb_d;
    J.out_r = act; J.out_s = sh_act;
    auto rows_per_block = [&](int kin) {
        int T = kin / 64, LPR = 64;
        while (LPR > 1 && LPR > T) LPR >>= 1;
        return 4 * (64 / LPR);
    };
    const int maxrows = has_sh ? (E > SH ? E : SH) : E;
    const dim3 g1(cdiv(maxrows, rows_per_block(d)), S + J.N);
    if (allexp) {
        J.rx = xres; J.rw = rw; J.rbias = bias; J.rnw = nw; J.reps = eps; J.ne = ne; J.gw = gw;
        J.ridx = idx; J.rwout = w;
        const dim3 ga(g1.x, N * ne + N + N);  // every expert, the shared experts, the routers
        hipLaunchKernelGGL((k_moe_gemv<KIND, true, false, true>), ga, dim3(256), rlds, stream(), J);
    } else if (fused_route) {
        J.rx = xres; J.rw = rw; J.rbias = bias; J.rnw = nw; J.reps = eps; J.ne = ne; J.gw = gw;
        J.ridx = idx; J.rwout = w;
        hipLaunchKernelGGL((k_moe_gemv<KIND, true, true>), g1, dim3(256), rlds, stream(), J);
    } else if (chain) {
        J.rlogits = logits; J.rbias = bias; J.ne = ne; J.ridx = idx; J.rwout = w;
        hipLaunchKernelGGL((k_moe_gemv<KIND, true, false, false, true>), g1, dim3(256), 0, stream(), J);
    } else {
        hipLaunchKernelGGL((k_moe_gemv<KIND, true>), g1, dim3(256), 0, stream(), J);
    }
    GH_LAUNCHED("k_moe_gemv(gate/up)");
    GemvJobs D{};
    D.gather_ne = allexp ? ne : 0;
    D.x = act; D.idx = idx; D.S = S; D.N = J.N; D.K = K; D.d = d;
    D.wa = (const uint8_t*)downs; D.estride = (size_t)d * rowb_E; D.sa = (const uint8_t*)sh_d;
    D.rows_r = d; D.rows_s = d; D.kin_r = E; D.kin_s = SH; D.rowb_r = rowb_E; D.rowb_s = rowb_SH;
    D.in_s = sh_act;
    const int LPR = down_lpr(E, SH, has_sh);
    const int rpb = 4 * (64 / LPR);
    const size_t lds = ((has_sh ? (size_t)SH : 0) + (size_t)K * E) * 4;
    if (down_par_fits<KIND>(has_sh, K, E, SH)) {
        hipLaunchKernelGGL((k_moe_down_par<KIND>), dim3(cdiv(d, DP_RB), N), dim3(64 * (K + 1)), lds, stream(), D, w,
                           xres, 1);
    } else {
        hipLaunchKernelGGL((k_moe_down_combine<KIND>), dim3(cdiv(d, rpb), N), dim3(256), lds, stream(), D, w, xres,
                           LPR, 1);
    }
    GH_LAUNCHED("k_moe_down_combine");
    return GH_OK;
}

int moe_decode_fused(float* xres, const float* nw, float eps, const float* rw, const float* bias, const void* gates,
                     const void* ups, const void* downs, const void* sh_g, const void* sh_u, const void* sh_d, int N,
                     int d, int E, int ne, int K, int SH, int qkind) {
    GH_REQUIRE(N >= 1 && N <= 8 && K >= 1 && K <= 8 && ne > 0 && ne <= 64, "moe decode: bad arguments");
    const int bv = qkind == 3 ? 256 : 64;
    GH_REQUIRE(d % bv == 0 && E % bv == 0 && SH % bv == 0, "moe decode: dims must be multiples of %d", bv);
    GH_REQUIRE((size_t)K * E + SH <= 15 * 1024, "moe decode: K*E + SH = %d activations exceed LDS", K * E + SH);
    switch (qkind) {
        case -1: return moe_decode_fused_kind<4>(xres, nw, eps, rw, bias, gates, ups, downs, sh_g, sh_u, sh_d, N, d, E, ne, K, SH);
        case 0: return moe_decode_fused_kind<0>(xres, nw, eps, rw, bias, gates, ups, downs, sh_g, sh_u, sh_d, N, d, E, ne, K, SH);
        case 1: return moe_decode_fused_kind<1>(xres, nw, eps, rw, bias, gates, ups, downs, sh_g, sh_u, sh_d, N, d, E, ne, K, SH);
        case 2: return moe_decode_fused_kind<2>(xres, nw, eps, rw, bias, gates, ups, downs, sh_g, sh_u, sh_d, N, d, E, ne, K, SH);
        default: return moe_decode_fused_kind<3>(xres, nw, eps, rw, bias, gates, ups, downs, sh_g, sh_u, sh_d, N, d, E, ne, K, SH);
    }
}

int moe_route(const float* x, const float* rw, const float* bias, float* probs, int32_t* idx, float* w, int N, int d,
              int ne, int K) {
    return launch_route(x, rw, bias, probs, idx, w, N, d, ne, K, nullptr, 0.f, nullptr);
}

}  // namespace gh

using namespace gh;

namespace gh {

// moe_forward_bias_half with an optional residual target: when acc_dst is given and the path
// ends in the ordered combine, the combined output is added into acc_dst (one addition, as the
// caller's add_inplace would do) and *added is set; otherwise `out` holds it.
int moe_forward_acc(const float* x, const float* router_w, const float* router_bias, const void* gates,
                    const void* ups, const void* downs, const void* sh_g, const void* sh_u, const void* sh_d,
                    float* out, float* acc_dst, int* added, float* probs_cache, int32_t* idx_cache, float* w_cache,
                    int64_t N, int d, int E, int ne, int K, int SH, int qkind, const float* nw, float eps,
                    float* xn) {
    if (added) *added = 0;
    if (N <= 0) return GH_OK;
    // core/moe_cpu.cpp:207-209
    GH_REQUIRE(K >= 1 && K <= 8, "moe_forward: K must be in [1,8]");
    GH_REQUIRE(ne > 0 && ne <= 64, "moe_forward: ne out of range");
    GH_REQUIRE(d > 0 && E > 0, "moe_forward: bad dims");
    GH_REQUIRE(x && router_w && gates && ups && downs && out, "moe_forward: null pointer");
    GH_REQUIRE(qkind >= -1 && qkind <= 3, "moe_forward: unknown qkind %d", qkind);
    const int bv = qkind == 3 ? 256 : 64;
    const bool has_sh = sh_g && sh_u && sh_d;
    GH_REQUIRE(d % bv == 0 && E % bv == 0 && (!has_sh || SH % bv == 0),
               "moe_forward: d=%d, E=%d, SH=%d must be multiples of %d", d, E, SH, bv);
    GH_REQUIRE(N <= 8192, "moe_forward: at most 8192 tokens per call");
    const int S = (int)N * K;
    int32_t* idx = idx_cache;
    float* w = w_cache;
    if (!idx || !w) {
        char* r = (char*)workspace(WS_MOE_ROUTE, (size_t)S * 8);
        if (!r) return fail(GH_ENOMEM, "moe: workspace");
        if (!idx) idx = (int32_t*)r;
        if (!w) w = (float*)(r + (size_t)S * 4);
    }
    // few tokens, a large router: logits by k_route_chain, the selection inside the gate/up blocks
    const bool chain = N <= 8 && (size_t)ne * d > 16384 && d % 4 == 0 && d <= 4096 && qkind >= 0;
    if (chain) {
        GH_REQUIRE(!nw || xn, "moe_forward: a normalised-row buffer is needed with the norm");
        float* lg = (float*)workspace(WS_MOE_TERMS, (size_t)N * ne * 4);
        if (!lg) return fail(GH_ENOMEM, "moe: workspace");
        hipLaunchKernelGGL(k_route_chain, dim3(ne, (unsigned)N), dim3(64), 0, stream(), x, router_w, lg, d, ne, nw, eps,
                           xn);
        GH_LAUNCHED("k_route_chain");
        const float* xi = nw ? xn : x;
        const int n = (int)N;
        switch (qkind) {
            case 0: return moe_kind<0>(xi, w, idx, gates, ups, downs, sh_g, sh_u, sh_d, out, acc_dst, added, n, d, E, ne, K, SH, lg, router_bias, probs_cache);
            case 1: return moe_kind<1>(xi, w, idx, gates, ups, downs, sh_g, sh_u, sh_d, out, acc_dst, added, n, d, E, ne, K, SH, lg, router_bias, probs_cache);
            case 2: return moe_kind<2>(xi, w, idx, gates, ups, downs, sh_g, sh_u, sh_d, out, acc_dst, added, n, d, E, ne, K, SH, lg, router_bias, probs_cache);
            default: return moe_kind<3>(xi, w, idx, gates, ups, downs, sh_g, sh_u, sh_d, out, acc_dst, added, n, d, E, ne, K, SH, lg, router_bias, probs_cache);
        }
    }
    int rc;
    if (nw) {
        // x is the raw residual row: the norm (ffn_norm) runs inside the router launch where that
        // path has it (k_route writes the normalised rows to xn), else as its own launch first
        GH_REQUIRE(xn, "moe_forward: a normalised-row buffer is needed with the norm");
        const bool fused = !(N > 8 && ne >= 16);  // the many-token logits path has no norm
        if (fused) {
            rc = launch_route(x, router_w, router_bias, probs_cache, idx, w, (int)N, d, ne, K, nw, eps, xn);
        } else {
            rc = gh_rmsnorm_forward(x, nw, xn, nullptr, N, d, eps);
            if (!rc) rc = moe_route(xn, router_w, router_bias, probs_cache, idx, w, (int)N, d, ne, K);
        }
        x = xn;
    } else {
        rc = moe_route(x, router_w, router_bias, probs_cache, idx, w, (int)N, d, ne, K);
    }
    if (rc) return rc;
    const int n = (int)N;
    switch (qkind) {
        case -1: return moe_kind<4>(x, w, idx, gates, ups, downs, sh_g, sh_u, sh_d, out, acc_dst, added, n, d, E, ne, K, SH);
        case 0: return moe_kind<0>(x, w, idx, gates, ups, downs, sh_g, sh_u, sh_d, out, acc_dst, added, n, d, E, ne, K, SH);
        case 1: return moe_kind<1>(x, w, idx, gates, ups, downs, sh_g, sh_u, sh_d, out, acc_dst, added, n, d, E, ne, K, SH);
        case 2: return moe_kind<2>(x, w, idx, gates, ups, downs, sh_g, sh_u, sh_d, out, acc_dst, added, n, d, E, ne, K, SH);
        default: return moe_kind<3>(x, w, idx, gates, ups, downs, sh_g, sh_u, sh_d, out, acc_dst, added, n, d, E, ne, K, SH);
    }
}

}  // namespace gh

extern "C" {

int gh_moe_route(const float* x, const float* rw, const float* bias, float* probs, int32_t* idx, float* w, int64_t N,
                 int d, int ne, int K) {
    GH_REQUIRE(K >= 1 && K <= 8, "moe_forward: K must be in [1,8]");
    GH_REQUIRE(ne > 0 && ne <= 64, "moe_forward: ne out of range");
    GH_REQUIRE(d > 0 && d % 4 == 0, "moe_forward: bad dims");
    GH_REQUIRE(x && rw && idx && w, "moe_route: null pointer");
    if (N <= 0) return GH_OK;
    return moe_route(x, rw, bias, probs, idx, w, (int)N, d, ne, K);
}

int gh_moe_permute(const int32_t* idx, int64_t N, int K, int ne, int32_t* grouped, int32_t* offsets) {
    GH_REQUIRE(idx && grouped && offsets && ne > 0 && ne <= 64 && K >= 1, "moe_permute: bad arguments");
    return permute(idx, (int)(N * K), ne, grouped, offsets, nullptr, nullptr, BM);
}

int gh_moe_forward_bias_half(const float* x, const float* router_w, const float* router_bias, const void* gates,
                             const void* ups, const void* downs, const void* sh_g, const void* sh_u,
                             const void* sh_d, float* out, float* probs_cache, int32_t* idx_cache, float* w_cache,
                             float* s_gate, float* s_up, float* s_act, int64_t N, int d, int E, int ne, int K, int SH,
                             int qkind) {
    (void)s_gate;
    (void)s_up;
    (void)s_act;
    return moe_forward_acc(x, router_w, router_bias, gates, ups, downs, sh_g, sh_u, sh_d, out, nullptr, nullptr,
                           probs_cache, idx_cache, w_cache, N, d, E, ne, K, SH, qkind, nullptr, 0.f, nullptr);
}

}  // extern "C"
