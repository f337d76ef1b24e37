// Router top-k of the MoE FFN (core/moe_cpu.cpp:218-256) as block-level
// device functions, shared by the MoE kernels (moe.hip) and the persistent
// decode kernel (decode_persistent.hip).
#pragma once
#include "gh_common.h"

namespace gh {

// =============================================================== router
// core/moe_cpu.cpp:218-256, one block per token, same arithmetic order:
// logit_e = dot_row: s += ((p0 + p1) + p2) + p3 over groups of 4, left to
// right, no fused multiply-add. The group terms are independent, so the
// block computes all of them in parallel into LDS and lane e then adds its
// terms in order -- the sequential sum stays exact while the weight loads
// are spread over the block (the first batch is requested together with the
// activations). softmax_row (core/math_cpu.cpp:546-558: sequential sum, exp
// rounded once from double = correctly rounded), selection on p + bias by K
// rounds of strict '>' argmax with the lowest index winning ties, weights
// from the unbiased p renormalised (uniform if their sum <= 1e-8).
// LDS: x [d] | terms [ne][gw + 1] for a window of gw groups (all groups
// when they fit; the lane sums run on across windows, still in order).
// Softmax + top-k of one token's logits sp[0..ne) (LDS, overwritten with
// the exponentials), run by the 64 lanes of one wave (see k_route).
__device__ __forceinline__ void route_finish(float* sp, const float* __restrict__ bias, int ne, int K, int t,
                             int32_t* __restrict__ idx, float* __restrict__ wout, float* __restrict__ probs,
                             int* sel_lds = nullptr, float* wsel_lds = nullptr) {
#pragma clang fp contract(off)
    // one wave per token (K <= 8, ne <= 64, at most 16 waves per block). The serial parts (the
    // sums in expert order) read their operands as LDS vectors, every lane running the same
    // chain (a readlane per operand stalls on the scalar-register hazard each step); the rank
    // of each candidate is counted by every lane over LDS vectors of all keys.
    __shared__ int rf_sel_all[16][8];
    __shared__ __attribute__((aligned(16))) float rf_p_all[16][64];
    __shared__ __attribute__((aligned(16))) uint32_t rf_k_all[16][64];
    const int wv_id = threadIdx.x >> 6;
    int* rf_sel = rf_sel_all[wv_id];
    float* rf_p = rf_p_all[wv_id];
    uint32_t* rf_k = rf_k_all[wv_id];
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    const int lane = threadIdx.x & 63;
    const float lg = lane < ne ? sp[lane] : -INFINITY;
    const float bl = (lane < ne && bias) ? bias[lane] : 0.0f;
    const float mx = wave_max(lg);  // order-free
    const float ev = lane < ne ? (float)exp((double)(lg - mx)) : 0.f;
    rf_p[lane] = ev;
    wave_sync();
    // sequential sum in expert order (the reference's rounding); the zeros past ne add nothing
    const int nq = (ne + 3) >> 2;  // wave-uniform
    float sum = 0.f;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        if (q < nq) {
            const float4 v = ((const float4*)rf_p)[q];
            sum = (((sum + v.x) + v.y) + v.z) + v.w;
        }
    }
    const float inv = (sum > 1e-12f) ? (1.0f / sum) : 0.0f;
    const float p = ev * inv;
    const float sel = lane < ne ? p + bl : -INFINITY;
    // K rounds of "largest value, lowest index among the rest" pick the candidates in the
    // order of this key: the value in an order-preserving unsigned form, ties by index.
    // Each candidate's rank (number of candidates before it) is its round.
    const bool cand = lane < ne && sel > -1e30f;
    const uint32_t u = __builtin_bit_cast(uint32_t, sel);
    const uint32_t key = cand ? ((u & 0x80000000u) ? ~u : (u | 0x80000000u)) : 0u;
    wave_sync();  // every lane has read rf_p
    rf_p[lane] = p;
    rf_k[lane] = key;
    wave_sync();
    int rank = 0;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        if (q >= nq) continue;
        const uint4 k4 = ((const uint4*)rf_k)[q];
        const int j = 4 * q;
        rank += (k4.x > key || (k4.x == key && j < lane)) ? 1 : 0;
        rank += (k4.y > key || (k4.y == key && j + 1 < lane)) ? 1 : 0;
        rank += (k4.z > key || (k4.z == key && j + 2 < lane)) ? 1 : 0;
        rank += (k4.w > key || (k4.w == key && j + 3 < lane)) ? 1 : 0;
    }
    const int ncand = __popcll(__ballot(cand));
    if (cand && rank < K) rf_sel[rank] = lane;
    wave_sync();
    // round k: expert rf_sel[k] (a round without candidates takes expert 0, as the reference)
    int selk[8];
    float wk[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        selk[k] = (k < K && k < ncand) ? rf_sel[k] : 0;
        wk[k] = k < K ? rf_p[selk[k]] : 0.f;
    }
    // weights from the unbiased probabilities, renormalised in round order
    float sw = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k)
        if (k < K) sw += wk[k];
    if (lane < K) {
        int mine = 0;
        float wv = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (k == lane) {
                mine = selk[k];
                wv = wk[k];
            }
        const float w = (sw > 1e-8f) ? wv * (1.0f / sw) : 1.0f / (float)K;
        if (idx) idx[(size_t)t * K + lane] = mine;
        if (wout) wout[(size_t)t * K + lane] = w;
        if (sel_lds) sel_lds[lane] = mine;
        if (wsel_lds) wsel_lds[lane] = w;
    }
    if (probs && lane < ne) probs[(size_t)t * ne + lane] = p;
}

constexpr int ROUTE_RB = 8;  // float4 weight loads per thread per batch
// Routing of token t by a block of 256 threads. With `nw` set, the token is
// first RMS-normalised (elementwise.hip k_rmsnorm arithmetic); the
// (normalised) row stays in sx [d] (LDS) and is also written to xn when
// given. term: LDS [ne][GW + 1]. sel_lds (LDS [K], optional) receives the
// selected experts; idx / wout / probs (global) may be null.
// Token row t of x into sx [d] (LDS), RMS-normalised when nw is given
// (elementwise.hip k_rmsnorm arithmetic: double sum of squares) and written
// to xn when given. A block of 256 threads; every caller gets bit-identical
// values (the same loads, sums and order).
__device__ __forceinline__ void route_norm(const float* __restrict__ x, int t, int d, const float* __restrict__ nw,
                                           float eps, float* __restrict__ xn, float* sx) {
    __shared__ double dred[4];
    const int tid = threadIdx.x, ngroups = d / 4;
    const float4* xt = (const float4*)(x + (size_t)t * d);
    double ss = 0.0;
    for (int g = tid; g < ngroups; g += 256) {
        const float4 v = xt[g];
        *(float4*)(sx + 4 * g) = v;
        ss += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
    }
    if (nw) {
        ss = wave_sum(ss);
        if ((tid & 63) == 0) dred[tid >> 6] = ss;
        __syncthreads();
        const double tot = dred[0] + dred[1] + dred[2] + dred[3];
        const double invd = 1.0 / sqrt(tot / (double)d + (double)eps);
        const float inv = isfinite(invd) ? (float)invd : 0.0f;
        for (int i = tid; i < d; i += 256) {
            const float v = sx[i] * inv * nw[i];
            sx[i] = v;
            if (xn) xn[(size_t)t * d + i] = v;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ void route_token(const float* __restrict__ x, const float* __restrict__ rw, const float* __restrict__ bias,
                            float* __restrict__ probs, int32_t* __restrict__ idx, float* __restrict__ wout, int d,
                            int ne, int K, const float* __restrict__ nw, float eps, float* __restrict__ xn, int GW,
                            int t, float* sx, float* term, int* sel_lds, float* wsel_lds = nullptr) {
#pragma clang fp contract(off)
    const int ngroups = d / 4, ts = GW + 1;
    __shared__ float sp[64];
    const int tid = threadIdx.x;
    const float4* rw4 = (const float4*)rw;
    auto widx = [&](int q, int g0, int gw) {  // pair q of a window -> float4 index in rw
        const int e = q / gw;
        return e * ngroups + g0 + (q - e * gw);
    };
    // first batch of router weights, requested with the activations
    float4 wreg[ROUTE_RB];
    {
        const int gw = min(GW, ngroups);
#pragma unroll
        for (int b = 0; b < ROUTE_RB; ++b) {
            const int q = tid + b * 256;
            if (q < ne * gw) wreg[b] = rw4[widx(q, 0, gw)];
        }
    }
    route_norm(x, t, d, nw, eps, xn, sx);
    float s = 0.0f;  // lane e < ne owns logit e
    for (int g0 = 0; g0 < ngroups; g0 += GW) {
        const int gw = min(GW, ngroups - g0), np = ne * gw;
        for (int q0 = 0; q0 < np; q0 += ROUTE_RB * 256) {
            if (g0 > 0 || q0 > 0) {
#pragma unroll
                for (int b = 0; b < ROUTE_RB; ++b) {
                    const int q = q0 + tid + b * 256;
                    if (q < np) wreg[b] = rw4[widx(q, g0, gw)];
                }
            }
#pragma unroll
            for (int b = 0; b < ROUTE_RB; ++b) {
                const int q = q0 + tid + b * 256;
                if (q < np) {
                    const int e = q / gw, gl = q - e * gw;
                    const int i = 4 * (g0 + gl);
                    const float4 w = wreg[b];
                    const float p0 = sx[i] * w.x, p1 = sx[i + 1] * w.y, p2 = sx[i + 2] * w.z, p3 = sx[i + 3] * w.w;
                    term[e * ts + gl] = ((p0 + p1) + p2) + p3;
                }
            }
        }
        __syncthreads();
        if (tid < ne) {
            // in order; the LDS reads are batched so only the adds are serial
            const float* tr = term + tid * ts;
            int g = 0;
            for (; g + 16 <= gw; g += 16) {
                float v[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) v[j] = tr[g + j];
#pragma unroll
                for (int j = 0; j < 16; ++j) s += v[j];
            }
            for (; g < gw; ++g) s += tr[g];
        }
        __syncthreads();
    }
    if (tid < ne) sp[tid] = s;
    __syncthreads();
    if (tid < 64) route_finish(sp, bias, ne, K, t, idx, wout, probs, sel_lds, wsel_lds);
    __syncthreads();  // sel_lds, sx visible to the block
}

}  // namespace gh
