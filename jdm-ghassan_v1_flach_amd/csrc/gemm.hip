// Prefill GEMM: y[M,N] = x[M,K] dequant(W)[N,K]^T for M > 8, with the
// weights dequantised straight into LDS as fp16 and multiplied on the
// matrix cores (v_mfma_f32_32x32x16_f16), fp32 accumulation. fp16 operands
// reproduce the reference's numerics: its CPU path rounds every dequantised
// weight to fp16 (core/ops.cpp:304-338) and its CUDA path converts x to fp16
// for an fp16 x fp16 -> fp32 GEMM (cuda/kernels.cu:600-633).
// Replaces the cuBLAS path of cuda/kernels.cu:190-441 / :583-633 (which
// first materialised an fp16 copy of the weight in HBM).
//
// Block tile 128 (tokens) x 128 (output rows) x 64 (K), 4 waves in a 2x2
// arrangement, each wave a 64x64 sub-tile = 2x2 MFMA 32x32 tiles. Per K
// step every thread converts 32 activations (fp32 -> fp16) and dequantises
// 32 weights of one row (its half of a 64-value task) into LDS; the next
// K step's global loads are issued before the MFMAs of the current one.
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "gemm_tile.h"
#include "lds_dma.h"

namespace gh {

int launch_add_to(float* y, const float* t, int64_t n);

template <int KIND>
__global__ void __launch_bounds__(256) k_gemm_q(const float* __restrict__ X, const uint8_t* __restrict__ W,
                                                float* __restrict__ Y, int M, int K, int N, size_t rowb) {
    __shared__ __attribute__((aligned(16))) uint16_t sA[BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t sB[BN * LDS_STRIDE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // XCD-aware tile order: consecutive block ids land on different XCDs
    // (round robin over 8), so give each XCD a contiguous run of N tiles that
    // share the same activation rows in its L2.
    const int tilesN = cdiv(N, BN), tilesM = cdiv(M, BM);
    const int nblk = tilesN * tilesM;
    int bid = blockIdx.x;
    if (nblk % 8 == 0) bid = (bid % 8) * (nblk / 8) + bid / 8;
    const int tm = bid % tilesM, tn = bid / tilesM;
    const int m0 = tm * BM, n0 = tn * BN;

    // loader roles: thread -> (row r = tid/2, half h = tid%2) for both tiles
    const int lr = tid >> 1, lh = tid & 1;
    const int am = m0 + lr, bn = n0 + lr;
    const float* xrow = X + (size_t)(am < M ? am : M - 1) * K;
    const uint8_t* wrow = W + (size_t)(bn < N ? bn : N - 1) * rowb;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int T = K / BK;

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
        // registers -> LDS (fp16)
        {
            float v[32];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v[4 * i] = xa[i].x; v[4 * i + 1] = xa[i].y; v[4 * i + 2] = xa[i].z; v[4 * i + 3] = xa[i].w;
            }
            if (am >= M) {
#pragma unroll
                for (int i = 0; i < 32; ++i) v[i] = 0.f;
            }
            store_f16x32(sA + lr * LDS_STRIDE + lh * 32, v);
            wl.decode(v);
            if (bn >= N) {
#pragma unroll
                for (int i = 0; i < 32; ++i) v[i] = 0.f;
            }
            store_f16x32(sB + lr * LDS_STRIDE + lh * 32, v);
        }
        __syncthreads();
        if (t + 1 < T) gload(t + 1);
        // 4 k-slices of 16
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
    // D layout: col = lane%32, row = 8*(e/4) + 4*(lane/32) + e%4
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn + j * 32 + (lane & 31);
            if (col >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row < M) Y[(size_t)row * N + col] = acc[i][j][e];
            }
        }
}

// ---------------------------------------------------------------- v2
// Activations converted to fp16 ONCE (k_to_f16) instead of once per N tile;
// the A tile then moves with 16-byte copies. LDS is double-buffered (one
// barrier per K step): the next step's activation pieces and weight bytes
// are requested right after the barrier and land in registers while the
// MFMAs of the current step run. Weight decode for Q4_K / Q8_0 builds fp16
// integer codes with one v_and_or_b32 per pair (code | 0x6400 = 1024 + q)
// and scales them with one v_fma_mix_f32 each.
__global__ void k_to_f16(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t n4) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
        const float4 v = ((const float4*)x)[i];
        f16x4v h;
        h[0] = (_Float16)v.x; h[1] = (_Float16)v.y; h[2] = (_Float16)v.z; h[3] = (_Float16)v.w;
        ((f16x4v*)y)[i] = h;
    }
}

// Range-safe fp16 activations for the MFMA GEMMs: row r is stored as x * 2^s_r with s_r chosen
// so that the row's largest magnitude lands in [2^14, 2^15) (fp16's largest finite value is
// 65504), and rinv[r] = 2^-s_r rescales that row of the product exactly. The relative rounding
// of every element is then fp16's 2^-11 whatever the row's range (a plain cast turns
// |x| > 65504 into inf and flushes |x| < 6e-8 to zero). Rows without a finite non-zero
// maximum keep s_r = 0. One block per row.
__device__ __forceinline__ int f16_row_shift(float amax) {
    if (!(amax > 0.0f) || !isfinite(amax)) return 0;
    int e = 0;
    (void)frexpf(amax, &e);  // amax = m 2^e, m in [0.5, 1)
    return min(max(15 - e, -120), 120);
}
__global__ void __launch_bounds__(256) k_to_f16_rows(const float* __restrict__ x, uint16_t* __restrict__ y,
                                                     float* __restrict__ rinv, int K) {
    const int r = blockIdx.x;
    const float4* xr = (const float4*)(x + (size_t)r * K);
    const int k4 = K / 4;
    float amax = 0.0f;
    for (int i = threadIdx.x; i < k4; i += 256) {
        const float4 v = xr[i];
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    __shared__ float red[4];
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    const int sh = f16_row_shift(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
    if (threadIdx.x == 0) rinv[r] = ldexpf(1.0f, -sh);
    f16x4v* yr = (f16x4v*)(y + (size_t)r * K);
    for (int i = threadIdx.x; i < k4; i += 256) {
        const float4 v = xr[i];
        f16x4v h;
        h[0] = (_Float16)ldexpf(v.x, sh); h[1] = (_Float16)ldexpf(v.y, sh);
        h[2] = (_Float16)ldexpf(v.z, sh); h[3] = (_Float16)ldexpf(v.w, sh);
        yr[i] = h;
    }
}

template <int KIND>
__global__ void __launch_bounds__(256, 2) k_gemm_q2(const uint16_t* __restrict__ X16, const float* __restrict__ rinv,
                                                   const uint8_t* __restrict__ W, float* __restrict__ Y, int M, int K,
                                                   int N, size_t rowb, int Ts) {
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * LDS_STRIDE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tilesN = cdiv(N, BN), tilesM = cdiv(M, BM);
    const int nblk = tilesN * tilesM;
    int bid = blockIdx.x;
    if (nblk % 8 == 0) bid = (bid % 8) * (nblk / 8) + bid / 8;  // XCD-aware: an XCD keeps a run of N tiles
    const int tm = bid % tilesM, tn = bid / tilesM;
    const int m0 = tm * BM, n0 = tn * BN;

    // A pieces: thread -> rows ar + 32i (i < 4), 8 halves at ac
    const int ar = tid >> 3, ac = (tid & 7) * 8;
    // B: thread -> (row lr = tid/2, half lh = tid%2)
    const int lr = tid >> 1, lh = tid & 1;
    const int bn = n0 + lr;
    const uint8_t* wrow = W + (size_t)(bn < N ? bn : N - 1) * rowb;
    const uint16_t* xrows[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int am = m0 + ar + 32 * i;
        xrows[i] = X16 + (size_t)(am < M ? am : M - 1) * K;
    }
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    // K steps [tb, te) of split blockIdx.y; splits write partial tiles at Y + split * M * N
    const int tb = blockIdx.y * Ts, te = min(K / BK, tb + Ts);
    Y += (size_t)blockIdx.y * M * N;
    uint32_t magic = 0x64006400u;
    asm volatile("" : "+v"(magic));

    gh_u32x4v xa[4];
    WLoad<KIND> wl;
#pragma unroll
    for (int i = 0; i < 4; ++i) xa[i] = *(const gh_u32x4v*)(xrows[i] + (size_t)tb * BK + ac);
    wl.load(wrow, tb, lh);
    int buf = 0;
    for (int t = tb; t < te; ++t, buf ^= 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            gh_u32x4v v = xa[i];
            if (m0 + ar + 32 * i >= M) v = gh_u32x4v{0u, 0u, 0u, 0u};
            *(gh_u32x4v*)(sA[buf] + (ar + 32 * i) * LDS_STRIDE + ac) = v;
        }
        {
            uint16_t* dst = sB[buf] + lr * LDS_STRIDE + lh * 32;
            if (bn < N) {
                decode16<KIND>(wl, dst, magic);
            } else {
                float z[32];
#pragma unroll
                for (int i = 0; i < 32; ++i) z[i] = 0.f;
                store_f16x32(dst, z);
            }
        }
        __syncthreads();
        if (t + 1 < te) {
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
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn + j * 32 + (lane & 31);
            if (col >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row < M) Y[(size_t)row * N + col] = acc[i][j][e] * rinv[row];
            }
        }
}

// y = sum of the S split partials, in split order (deterministic); with
// `accumulate` the sum is added to y (the residual add of the caller).
__global__ void k_splitk_sum(const float* __restrict__ part, float* __restrict__ y, int64_t n, int S, int accumulate) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float v = part[i];
        for (int s = 1; s < S; ++s) v += part[(size_t)s * n + i];
        y[i] = accumulate ? y[i] + v : v;
    }
}

// ---------------------------------------------------------------- v4
// Large tiles for large M, Q4_K / Q8_0 weights: a block of 4 waves computes
// 256 (tokens) x 256 (output rows), each wave 128x128 as 4x4
// v_mfma_f32_32x32x16_f16 tiles (accumulators in the accumulation registers,
// one wave per SIMD). Per K step of 64:
//  - the fp16 activation tile (256 rows x 128 B) moves global -> LDS by
//    direct transfers (global_load_lds_dwordx4, no register round trip);
//  - every thread dequantises 64 weights of one output row (loaded one step
//    ahead) into the other LDS buffer, a quarter after each k-substep's
//    MFMAs, so the decode overlaps the matrix cores;
//  - MFMA operands are read one k-substep ahead (scheduling barriers keep
//    the compiler from sinking the reads next to their use).
// LDS rows are 128 B with the 16-byte piece c of row r stored at
// c ^ ((r >> 1) & 7): the 16 rows one ds_read_b128 / ds_write_b128 phase
// touches then cover all 64 banks. A and B are double-buffered (128 KB), one
// barrier per step. gridDim.y = 2 splits K for grids that would not fill the
// chip; the two halves then add into a zeroed Y (two addends onto 0 give the
// same sum in either order, so the result stays deterministic).
constexpr int G4M = 256, G4N = 256;
constexpr size_t G4_LDS = 4 * 256 * 128;  // A[2], B[2]: 256 rows x 128 bytes

__device__ __forceinline__ void g4_dma(const void* base, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base),
                 "s"(__builtin_amdgcn_readfirstlane(lds_base))
                 : "memory");
}

struct G4Scale {
    float d1[2], m1[2];
};
template <int KIND>
struct G4Raw;
template <>
struct G4Raw<3> {  // Q4_K: super-block header + the 32 nibble bytes of pair t&3
    gh_u32x4v hd, a, b;
    __device__ __forceinline__ void load(const uint8_t* row, int t) {
        const uint8_t* sb = row + (size_t)(t >> 2) * 144;
        const int p = t & 3;
        hd = *(const gh_u32x4v*)sb;
        a = *(const gh_u32x4v*)(sb + 16 + 32 * p);
        b = *(const gh_u32x4v*)(sb + 32 + 32 * p);
    }
};
template <>
struct G4Raw<2> {  // Q8_0: two 34-byte blocks at t*68 (4-byte aligned)
    gh_u32x4v q[4];
    uint32_t last;
    __device__ __forceinline__ void load(const uint8_t* row, int t) {
        const uint8_t* p = row + (size_t)t * 68;
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = *(const gh_u32x4v*)(p + 16 * i);
        last = *(const uint32_t*)(p + 64);
    }
    __device__ __forceinline__ uint32_t w(int i) const { return i < 16 ? q[i >> 2][i & 3] : last; }
};

__device__ __forceinline__ uint32_t g4_pack(float lo, float hi) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 v;
    v[0] = (_Float16)lo;  // RNE, as fp32_to_fp16
    v[1] = (_Float16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ G4Scale g4_scales(const G4Raw<2>&, int) { return G4Scale{}; }
// Q4_K scales of the two sub-blocks (2p, 2p+1) of step t: y = q * (d*sc) - dmin*m
__device__ __forceinline__ G4Scale g4_scales(const G4Raw<3>& r, int t) {
    // scale bytes 0..7 in lo, 8..11 in hi; shifts instead of an indexed array (t is a runtime value)
    const uint64_t lo = (uint64_t)r.hd[1] | ((uint64_t)r.hd[2] << 32);
    const uint32_t hi = r.hd[3];
    const float d = f16_to_f32((uint16_t)(r.hd[0] & 0xFFFF)), dm = f16_to_f32((uint16_t)(r.hd[0] >> 16));
    const int p = t & 3;
    G4Scale s;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int j = 2 * p + h;
        int scv, mv;
        if (p < 2) {
            scv = (int)(lo >> (8 * j)) & 63;
            mv = (int)(lo >> (8 * j + 32)) & 63;
        } else {
            const int b4 = (int)(hi >> (8 * (j - 4))) & 0xFF;
            scv = (b4 & 0xF) | ((((int)(lo >> (8 * (j - 4))) >> 6) & 3) << 4);
            mv = (b4 >> 4) | ((((int)(lo >> (8 * j))) >> 6 & 3) << 4);
        }
        s.d1[h] = d * (float)scv;
        s.m1[h] = dm * (float)mv;
    }
    return s;
}

// values 16Q..16Q+15 of a row's step as 8 packed fp16 pairs
template <int Q>
__device__ __forceinline__ void g4_quarter(const G4Raw<3>& r, const G4Scale& s, uint32_t, uint32_t (&h)[8]) {
    constexpr int hi = Q >> 1;  // values 0..31: low nibbles (sub-block 2p), 32..63: high (2p+1)
    const gh_u32x4v& src = (Q & 1) ? r.b : r.a;
    const float d1 = s.d1[hi], nm = -s.m1[hi];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t w = (hi ? (src[i] >> 4) : src[i]) & 0x0F0F0F0Fu;
        const float q0 = (float)(w & 0xFF), q1 = (float)((w >> 8) & 0xFF);
        const float q2 = (float)((w >> 16) & 0xFF), q3 = (float)(w >> 24);
        // q * d1 is exact (4 + 17 bits), so one fma rounds like q*d1 - m1 in fp32
        h[2 * i] = g4_pack(fmaf(q0, d1, nm), fmaf(q1, d1, nm));
        h[2 * i + 1] = g4_pack(fmaf(q2, d1, nm), fmaf(q3, d1, nm));
    }
}
template <int Q>
__device__ __forceinline__ void g4_quarter(const G4Raw<2>& r, const G4Scale&, uint32_t magic, uint32_t (&h)[8]) {
    // block Q>>1; its quants 16(Q&1)..+15 start at byte 34(Q>>1) + 2 + 16(Q&1)
    constexpr int off = 34 * (Q >> 1) + 2 + 16 * (Q & 1);
    const uint32_t dbits = (Q >> 1) ? (r.w(8) >> 16) : (r.w(0) & 0xFFFF);
    const float d = f16_to_f32((uint16_t)dbits);
    const float nb = -1152.f * d;  // (1152 + q) d - 1152 d = q d exactly
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        constexpr int dw = off >> 2;
        uint32_t u;
        if constexpr ((off & 3) == 2) u = __builtin_amdgcn_alignbyte(r.w(dw + i + 1), r.w(dw + i), 2);
        else u = r.w(dw + i);
        u ^= 0x80808080u;
        const uint32_t c0 = gq_and_or(u, 0x00FF00FFu, magic);
        const uint32_t c1 = gq_and_or(u >> 8, 0x00FF00FFu, magic);
        h[2 * i] = g4_pack(fmaf(gq_lo(c0), d, nb), fmaf(gq_lo(c1), d, nb));
        h[2 * i + 1] = g4_pack(fmaf(gq_hi(c0), d, nb), fmaf(gq_hi(c1), d, nb));
    }
}
template <int KIND>
__device__ __forceinline__ void g4_quarter_rt(const G4Raw<KIND>& r, const G4Scale& s, uint32_t magic, int q,
                                              uint32_t (&h)[8]) {
    if (q == 0) g4_quarter<0>(r, s, magic, h);
    if (q == 1) g4_quarter<1>(r, s, magic, h);
    if (q == 2) g4_quarter<2>(r, s, magic, h);
    if (q == 3) g4_quarter<3>(r, s, magic, h);
}

// K steps [t_beg, t_beg + T) of block (tile, blockIdx.y); T even, >= 2
template <int KIND>
__global__ void __launch_bounds__(256, 1) k_gemm_q4(const uint16_t* __restrict__ X16, const float* __restrict__ rinv,
                                                   const uint8_t* __restrict__ W, float* __restrict__ Y, int M, int K,
                                                   int N, size_t rowb, int T) {
    extern __shared__ __attribute__((aligned(16))) uint8_t g4_smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tilesN = cdiv(N, G4N), tilesM = cdiv(M, G4M);
    const int nblk = tilesN * tilesM;
    int bid = blockIdx.x;
    // XCD-aware order: consecutive block ids land on different XCDs, so give
    // each XCD a contiguous run of tiles (all M tiles of a few N tiles)
    if (nblk % 8 == 0) bid = (bid % 8) * (nblk / 8) + bid / 8;
    const int tm = bid % tilesM, tn = bid / tilesM;
    const int m0 = tm * G4M, n0 = tn * G4N;
    const int t_beg = blockIdx.y * T;
    const uint32_t lds0 = lds_addr(g4_smem);

    // A: wave w moves rows 64w..64w+63 as 8 transfers of 8 rows (16 B per lane)
    uint32_t avoff[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r = 64 * wave + 8 * i + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        const int rr = m0 + r < M ? m0 + r : M - 1;  // rows past M: any valid row (outputs masked)
        avoff[i] = (uint32_t)(((size_t)rr * K + c * 8) * 2);
    }
    const uint32_t a_lds = __builtin_amdgcn_readfirstlane(lds0 + 64 * wave * 128);
    // B: thread -> output row tid of the tile
    const int bn = n0 + tid;
    const uint8_t* wrow = W + (size_t)(bn < N ? bn : N - 1) * rowb;
    const int bsw = (tid >> 1) & 7;
    uint8_t* bdst0 = g4_smem + 65536 + tid * 128;
    // MFMA operands: row = wm/wn + 32 i + lane%32, logical piece 2 ks + lane/32
    const int wm = (wave >> 1) * 128, wn = (wave & 1) * 128;
    const int fsw = (lane >> 1) & 7, fhi = lane >> 5;
    const int frow = (lane & 31) * 128;

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    uint32_t magic = 0x64006400u;
    asm volatile("" : "+v"(magic));

    auto dma_a = [&](int t, int buf) {
        const uint16_t* base = X16 + (size_t)(t_beg + t) * 64;
#pragma unroll
        for (int i = 0; i < 8; ++i) g4_dma(base, avoff[i], a_lds + buf * 32768 + i * 1024);
    };
    auto load_b = [&](G4Raw<KIND>& r, int t) { r.load(wrow, t_beg + t); };
    auto put_b = [&](int buf, int q, const uint32_t (&h)[8]) {
        uint8_t* d = bdst0 + buf * 32768;
        *(gh_u32x4v*)(d + (((2 * q) ^ bsw) * 16)) = gh_u32x4v{h[0], h[1], h[2], h[3]};
        *(gh_u32x4v*)(d + (((2 * q + 1) ^ bsw) * 16)) = gh_u32x4v{h[4], h[5], h[6], h[7]};
    };
    // one step: MFMAs on buffer cur, decode of rn (step tt+1) into the other;
    // `issue` requests later steps' data once the first operand reads are out
    auto compute = [&](int tt, int cur, const G4Raw<KIND>& rn, auto has_next_c, auto issue) {
        constexpr bool has_next = decltype(has_next_c)::value;
        const uint8_t* sA = g4_smem + cur * 32768 + wm * 128 + frow;
        const uint8_t* sB = g4_smem + 65536 + cur * 32768 + wn * 128 + frow;
        f16x8 a[2][4], b[2][4];
        auto frag = [&](int ks, f16x8 (&fa)[4], f16x8 (&fb)[4]) {
            const int co = (((2 * ks + fhi) ^ fsw) * 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                fa[i] = *(const f16x8*)(sA + i * 32 * 128 + co);
                fb[i] = *(const f16x8*)(sB + i * 32 * 128 + co);
            }
        };
        frag(0, a[0], b[0]);
        issue();
        __builtin_amdgcn_sched_barrier(0);
        [[maybe_unused]] G4Scale s;
        if constexpr (has_next) s = g4_scales(rn, t_beg + tt + 1);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if (ks + 1 < 4) frag(ks + 1, a[(ks + 1) & 1], b[(ks + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[ks & 1][i], b[ks & 1][j], acc[i][j], 0, 0, 0);
            if constexpr (has_next) {
                uint32_t h[8];
                g4_quarter_rt<KIND>(rn, s, magic, ks, h);
                put_b(cur ^ 1, ks, h);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto sync = [&]() {
        __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): A transfers, weight bytes, B stores
        __builtin_amdgcn_s_barrier();
    };
    using YES = std::integral_constant<bool, true>;
    using NO = std::integral_constant<bool, false>;
    auto nothing = [] {};

    G4Raw<KIND> r0, r1;
    dma_a(0, 0);
    load_b(r0, 0);
    load_b(r1, 1);
    {
        const G4Scale s0 = g4_scales(r0, t_beg);
        uint32_t h[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            g4_quarter_rt<KIND>(r0, s0, magic, q, h);
            put_b(0, q, h);
        }
    }
    sync();
    int tt = 0;
    // steady state: buffer tt&1 holds step tt; r1 (even tt) / r0 (odd tt) holds step tt+1
    for (; tt + 3 < T; tt += 2) {
        compute(tt, 0, r1, YES{}, [&] { dma_a(tt + 1, 1); load_b(r0, tt + 2); });
        sync();
        compute(tt + 1, 1, r0, YES{}, [&] { dma_a(tt + 2, 0); load_b(r1, tt + 3); });
        sync();
    }
    compute(tt, 0, r1, YES{}, [&] { dma_a(tt + 1, 1); });
    sync();
    compute(tt + 1, 1, r0, NO{}, nothing);

    const bool split = gridDim.y > 1;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = n0 + wn + j * 32 + (lane & 31);
            if (col >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row >= M) continue;
                const float v = acc[i][j][e] * rinv[row];
                if (split) atomicAdd(&Y[(size_t)row * N + col], v);
                else Y[(size_t)row * N + col] = v;
            }
        }
}

__global__ void k_zero_f32(float* __restrict__ y, int64_t n4) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x)
        ((float4*)y)[i] = float4{0.f, 0.f, 0.f, 0.f};
}

int launch_to_f16(const float* x, uint16_t* y, int64_t n) {
    const int64_t n4 = n / 4;
    hipLaunchKernelGGL(k_to_f16, dim3((unsigned)std::min<int64_t>(cdiv64(n4, 256), 8192)), dim3(256), 0, stream(), x,
                       y, n4);
    GH_LAUNCHED("k_to_f16");
    return GH_OK;
}

__global__ void k_add_to(float* __restrict__ y, const float* __restrict__ t, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] += t[i];
}

// ---------------------------------------------------------------- skinny
// Row prologues of the skinny GEMM (the row is normalised while it is staged, so the norm
// takes no launch of its own):
//  SK_RMSNORM:  x * inv * w with inv = 1 / sqrt(mean(x^2) + eps) in double, the sum of squares
//               in double (elementwise.hip k_rmsnorm, core/math_cpu.cpp rmsnorm);
//  SK_GATENORM: rows already gated (v = y * silu(z), applied by the SSD scan's stores), then
//               v * inv * w with inv = 1 / sqrtf(mean(v^2) + eps) in float (mamba.hip
//               k_gated_norm, the Mamba-2 gated RMSNorm before out_proj).
enum { SK_PLAIN = 0, SK_RMSNORM = 1, SK_GATENORM = 2 };
struct SkPro {
    const float* nw;  // norm weight (K values)
    float eps;
};
// Up to three products of the same rows in one launch (the attention q / k / v projections):
// output rows [off[s], off[s + 1]) of the grid belong to segment s (weights w[s], outputs y[s]
// of n[s] columns; y16[s], if set, takes an fp16 copy of them, the KV cache's copy). Each
// segment is a whole number of the launch's weight-row tiles. n = 0 segments: one product.
struct SkSeg {
    const uint8_t* w[3];
    float* y[3];
    uint16_t* y16[3];
    int off[4];
    int nseg;
};
template <int PRO>
__device__ __forceinline__ float sk_inv(double ss, int n, float eps) {
    if constexpr (PRO == SK_RMSNORM) {
        const double invd = 1.0 / sqrt(ss / (double)n + (double)eps);
        return isfinite(invd) ? (float)invd : 0.0f;
    } else {
        return 1.0f / sqrtf((float)(ss / (double)n) + eps);
    }
}

// Small M (prefill of a short prompt), Q4_K or Q8_0, K = 256, 512 or 1024: a block takes MT (16 or
// 32) rows of x (fp32, converted to fp16 while staged into LDS) and 16*WR weight rows over
// the WHOLE K: each lane requests every Q4_K byte of its MFMA B operands before the first
// multiply (one memory wait per block instead of one per K step, and no split-K partials in
// HBM), wave w owns weight rows 16(w%WR)..+15 over K range w/WR of NWK
// (v_mfma_f32_16x16x32_f16, activations as A in MT/16 16-row halves). The tile is chosen per
// shape so that a launch spreads over the CUs (a short prompt has few 32x64 tiles). Each
// output is written (or added, with `accumulate`) by exactly one lane.
template <int KK, int NWK, int WR, int MT, int PRO = SK_PLAIN, int KIND = 3>
__global__ void __launch_bounds__(64 * WR * NWK) k_gemm_skinny(const float* __restrict__ X, const uint8_t* __restrict__ W,
                                                               float* __restrict__ Y, int M, int N, size_t rowb,
                                                               int accumulate, SkPro pro, SkSeg seg) {
    // NWK wave groups split K: group kg takes k-steps kg*NS .. kg*NS + NS - 1; the groups'
    // sums meet in LDS and group 0 adds them in group order
    constexpr int SA = KK + 8, NS = KK / 32 / NWK, NT = 64 * WR * NWK, NW = WR * NWK, NH2 = MT / 16;
    static_assert(NS >= 1 && (8 % NS == 0 || NS % 8 == 0), "K steps of a group stay within whole super-blocks");
    __shared__ __attribute__((aligned(16))) _Float16 sA[MT * SA];
    __shared__ float sR[NWK > 1 ? (NWK - 1) * WR * 64 * 4 * NH2 : 1];
    const int m0 = blockIdx.x * MT, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave % WR, kg = wave / WR;
    const int col = lane & 15, kq = lane >> 4;
    int nrow = blockIdx.y * 16 * WR + 16 * wr + col;
    uint16_t* Y16 = nullptr;
    if (seg.nseg > 0) {  // the block's segment (block-uniform: segments are whole tiles)
        const int n0 = blockIdx.y * 16 * WR;
        const int sg = n0 >= seg.off[2] && seg.nseg > 2 ? 2 : n0 >= seg.off[1] && seg.nseg > 1 ? 1 : 0;
        W = seg.w[sg];
        Y = seg.y[sg];
        Y16 = seg.y16[sg];
        N = seg.off[sg + 1] - seg.off[sg];
        nrow -= seg.off[sg];
    }
    const bool nok = nrow < N;
    const uint8_t* wrow = W + (size_t)(nok ? nrow : 0) * rowb;
    const int s0 = kg * NS;
    // every weight byte of the lane, requested first: Q4_K, the headers of the super-blocks it
    // touches and 8 code bytes per k-step; Q8_0, per k-step (one 34-byte block) the dword holding
    // the block's scale and the three dwords holding codes 8 kq .. 8 kq + 7 (2-byte aligned)
    constexpr int NH = KIND == 3 ? (NS >= 8 ? NS / 8 : 1) : 1;
    uint4 hdr[NH];
    uint2 qb[KIND == 3 ? NS : 1];
    uint32_t q8w[KIND == 2 ? NS : 1][4];
    if constexpr (KIND == 3) {
#pragma unroll
        for (int b = 0; b < NH; ++b) hdr[b] = *(const uint4*)(wrow + (size_t)((s0 >> 3) + b) * 144);
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
    // MT rows x KK fp32 -> fp16 LDS (8 values per piece), each row scaled by 2^s_r as
    // k_to_f16_rows does (the row maxima first, one wave per row). With a row prologue the
    // staged values are the normalised rows.
    constexpr int RQ = KK / 8;
    __shared__ int sShift[MT];
    if constexpr (PRO != SK_PLAIN) {
        // one wave per row: the row's values stay in registers (4 per lane per float4), its norm,
        // maximum and fp16 copy are formed from them
        constexpr int U = KK / 256;  // float4 per lane
        for (int r = wave; r < MT; r += NW) {
            float4 v[U];
            double ss = 0.0;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                v[u] = m0 + r < M ? ((const float4*)(X + (size_t)(m0 + r) * KK))[lane + 64 * u]
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
                ss += (double)v[u].x * v[u].x + (double)v[u].y * v[u].y + (double)v[u].z * v[u].z +
                      (double)v[u].w * v[u].w;
            }
            ss = wave_sum(ss);
            const float inv = sk_inv<PRO>(ss, KK, pro.eps);
            float amax = 0.0f;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float4 w = ((const float4*)pro.nw)[lane + 64 * u];
                v[u].x = v[u].x * inv * w.x;
                v[u].y = v[u].y * inv * w.y;
                v[u].z = v[u].z * inv * w.z;
                v[u].w = v[u].w * inv * w.w;
                amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
            }
            for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
            const int sh = f16_row_shift(amax);
            if (lane == 0) sShift[r] = sh;
            typedef _Float16 sk_f16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int u = 0; u < U; ++u) {
                sk_f16x4 h;
                h[0] = (_Float16)ldexpf(v[u].x, sh); h[1] = (_Float16)ldexpf(v[u].y, sh);
                h[2] = (_Float16)ldexpf(v[u].z, sh); h[3] = (_Float16)ldexpf(v[u].w, sh);
                *(sk_f16x4*)(sA + r * SA + 4 * (lane + 64 * u)) = h;
            }
        }
        __syncthreads();
    } else {
        for (int r = wave; r < MT; r += NW) {
            float amax = 0.0f;
            if (m0 + r < M) {
                const float4* src = (const float4*)(X + (size_t)(m0 + r) * KK);
#pragma unroll
                for (int i = lane; i < KK / 4; i += 64) {
                    const float4 v = src[i];
                    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
                }
            }
            for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
            if (lane == 0) sShift[r] = f16_row_shift(amax);
        }
        __syncthreads();
        for (int e = tid; e < MT * RQ; e += NT) {
            const int r = e / RQ, c = e - r * RQ;
            float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
            if (m0 + r < M) {
                const float4* src = (const float4*)(X + (size_t)(m0 + r) * KK + 8 * c);
                a = src[0];
                b = src[1];
            }
            const int sh = sShift[r];
            sk_f16x8 h;
            h[0] = (_Float16)ldexpf(a.x, sh); h[1] = (_Float16)ldexpf(a.y, sh);
            h[2] = (_Float16)ldexpf(a.z, sh); h[3] = (_Float16)ldexpf(a.w, sh);
            h[4] = (_Float16)ldexpf(b.x, sh); h[5] = (_Float16)ldexpf(b.y, sh);
            h[6] = (_Float16)ldexpf(b.z, sh); h[7] = (_Float16)ldexpf(b.w, sh);
            *(sk_f16x8*)(sA + r * SA + 8 * c) = h;
        }
        __syncthreads();
    }
    typedef float f32x4k __attribute__((ext_vector_type(4)));
    f32x4k acc[NH2];
#pragma unroll
    for (int h = 0; h < NH2; ++h) acc[h] = f32x4k{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int sg = s0 + s;
        sk_f16x8 bv;
        if constexpr (KIND == 3) {
            bv = sk_q4k_bfrag(hdr[NS >= 8 ? s >> 3 : 0], qb[s], sg & 7, nok);
        } else {
            const int ob = 34 * sg, oc = ob + 2 + 8 * kq;
            bv = sk_q8_bfrag(q8w[s], ob & 3, oc & 3, nok);
        }
#pragma unroll
        for (int h = 0; h < NH2; ++h) {
            const sk_f16x8 av = *(const sk_f16x8*)(sA + (16 * h + col) * SA + 32 * sg + 8 * kq);
            acc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[h], 0, 0, 0);
        }
    }
    if constexpr (NWK > 1) {
        if (kg > 0) {
            float* r = sR + (((kg - 1) * WR + wr) * 64 + lane) * 4 * NH2;
#pragma unroll
            for (int h = 0; h < NH2; ++h)
#pragma unroll
                for (int j = 0; j < 4; ++j) r[4 * h + j] = acc[h][j];
        }
        __syncthreads();
        if (kg > 0) return;
#pragma unroll
        for (int g = 1; g < NWK; ++g) {
            const float* r = sR + (((g - 1) * WR + wr) * 64 + lane) * 4 * NH2;
#pragma unroll
            for (int h = 0; h < NH2; ++h)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[h][j] += r[4 * h + j];
        }
    }
    if (!nok) return;
    // with `accumulate`, every old value of the lane is loaded before the first store (the
    // compiler cannot tell the rows apart, and would otherwise wait for each load in turn)
    float old[NH2][4];
#pragma unroll
    for (int h = 0; h < NH2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = m0 + 16 * h + 4 * kq + j;
            old[h][j] = accumulate && m < M ? Y[(size_t)m * N + nrow] : 0.f;
        }
#pragma unroll
    for (int h = 0; h < NH2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = m0 + 16 * h + 4 * kq + j;
            if (m < M) {
                const float v = ldexpf(acc[h][j], -sShift[m - m0]);
                const float o = accumulate ? old[h][j] + v : v;
                Y[(size_t)m * N + nrow] = o;
                if (Y16) Y16[(size_t)m * N + nrow] = f32_to_f16(o);
            }
        }
}

template <int KK, int NWK, int WR, int MT, int KIND>
static void skinny_launch(const float* x, const uint8_t* w, float* y, int M, int N, size_t rowb, int accumulate,
                          int mode, const SkPro& pro, const SkSeg& seg) {
    const dim3 grid(cdiv(M, MT), cdiv(N, 16 * WR)), blk(64 * WR * NWK);
    if (mode == SK_RMSNORM)
        hipLaunchKernelGGL((k_gemm_skinny<KK, NWK, WR, MT, SK_RMSNORM, KIND>), grid, blk, 0, stream(), x, w, y, M, N, rowb,
                           accumulate, pro, seg);
    else if (mode == SK_GATENORM)
        hipLaunchKernelGGL((k_gemm_skinny<KK, NWK, WR, MT, SK_GATENORM, KIND>), grid, blk, 0, stream(), x, w, y, M, N, rowb,
                           accumulate, pro, seg);
    else
        hipLaunchKernelGGL((k_gemm_skinny<KK, NWK, WR, MT, SK_PLAIN, KIND>), grid, blk, 0, stream(), x, w, y, M, N, rowb,
                           accumulate, pro, seg);
}

// Whether the skinny path takes a product of linear_any / linear_acc: Q4_K, K 256 / 512 / 1024,
// 8 < M <= 256 rows (smaller M go to the GEMVs), 16-byte aligned x and W.
bool skinny_takes(const void* x, const void* w, int M, int K, int kind) {
    return (kind == 3 || kind == 2) && M > 8 && M <= 256 && (K == 256 || K == 512 || K == 1024) && !(((uintptr_t)x | (uintptr_t)w) & 15);
}

// Returns 1 if the skinny path took the product (Q4_K / Q8_0, K 256 / 512 / 1024, M <= 256). The
// 32x64 tile when it already gives a CU-filling grid; otherwise 16-row tiles over 64, 32 or
// 16 weight rows, the first of these that reaches 256 blocks (or the smallest), with the
// waves freed from weight rows splitting K instead. `mode` / `pro`: the row prologue.
static int gemm_skinny(const float* x, const void* w, float* y, int M, int K, int N, size_t rowb, int accumulate,
                       int* rc, int mode = SK_PLAIN, const SkPro& pro = SkPro{}, const SkSeg* seg = nullptr,
                       int kind = 3) {
    if ((kind != 3 && kind != 2) || M > 256 || (K != 256 && K != 512 && K != 1024) || (((uintptr_t)x | (uintptr_t)w) & 15)) return 0;
    const uint8_t* wb = (const uint8_t*)w;
    const int64_t b32 = (int64_t)cdiv(M, 32) * cdiv(N, 64), m16 = cdiv(M, 16);
    int cfg = 0;  // 0: 32x64, 1: 16x64, 2: 16x32, 3: 16x16
    if (b32 < 256) {
        cfg = 3;
        for (int c = 1; c <= 3; ++c)
            if (m16 * cdiv(N, 64 >> (c - 1)) >= 256) { cfg = c; break; }
    }
    SkSeg sg{};
    if (seg) {  // segments must be whole tiles of the chosen weight-row count
        const int rows = cfg <= 1 ? 64 : cfg == 2 ? 32 : 16;
        for (int i = 0; i < seg->nseg; ++i)
            if ((seg->off[i + 1] - seg->off[i]) % rows) return 0;
        sg = *seg;
    }
#define GH_SKINNY_K(KK, NWK0, KD)                                                                                \
    switch (cfg) {                                                                                               \
        case 0: skinny_launch<KK, NWK0, 4, 32, KD>(x, wb, y, M, N, rowb, accumulate, mode, pro, sg); break;      \
        case 1: skinny_launch<KK, NWK0, 4, 16, KD>(x, wb, y, M, N, rowb, accumulate, mode, pro, sg); break;      \
        case 2: skinny_launch<KK, 2 * NWK0, 2, 16, KD>(x, wb, y, M, N, rowb, accumulate, mode, pro, sg); break;  \
        default: skinny_launch<KK, 4 * NWK0, 1, 16, KD>(x, wb, y, M, N, rowb, accumulate, mode, pro, sg); break; \
    }
#define GH_SKINNY(KK, NWK0)                         \
    if (kind == 3) { GH_SKINNY_K(KK, NWK0, 3) }     \
    else { GH_SKINNY_K(KK, NWK0, 2) }
    if (K == 256) { GH_SKINNY(256, 2) }
    else if (K == 512) { GH_SKINNY(512, 2) }
    else { GH_SKINNY(1024, 4) }
#undef GH_SKINNY
#undef GH_SKINNY_K
    GH_LAUNCHED("k_gemm_skinny");
    *rc = GH_OK;
    return 1;
}

// Normalised-input product on the skinny path: y (+)= norm(x) W^T with the norm as the GEMM's
// row prologue (mode SK_RMSNORM or SK_GATENORM, x rows of K values). Returns GH_EUNSUPPORTED,
// launching nothing, where the skinny path does not take the shape (skinny_takes false) or the
// norm weights are not 16-byte aligned.
int linear_norm_skinny(const float* x, int mode, const float* nw, float eps, const void* w, float* y, int M, int K,
                       int N, int kind, int accumulate) {
    if (!skinny_takes(x, w, M, K, kind) || ((uintptr_t)nw & 15)) return GH_EUNSUPPORTED;
    SkPro pro{nw, eps};
    int rc = GH_OK;
    if (!gemm_skinny(x, w, y, M, K, N, row_bytes(kind, K), accumulate, &rc, mode, pro, nullptr, kind))
        return GH_EUNSUPPORTED;
    return rc;
}

// q / k / v (up to three weight matrices of the same K over the same rows) in one skinny launch,
// with the row prologue `mode` (SK_PLAIN / SK_RMSNORM) and optional fp16 copies of the outputs.
// GH_EUNSUPPORTED, launching nothing, where the skinny path does not take it.
int linear_multi_skinny(const float* x, int mode, const float* nw, float eps, int nseg, const void* const* w,
                        float* const* y, uint16_t* const* y16, const int* n, int M, int K, int kind) {
    if (nseg < 1 || nseg > 3 || (mode != SK_PLAIN && ((uintptr_t)nw & 15))) return GH_EUNSUPPORTED;
    SkSeg sg{};
    sg.nseg = nseg;
    sg.off[0] = 0;
    for (int i = 0; i < nseg; ++i) {
        if (!skinny_takes(x, w[i], M, K, kind) || n[i] <= 0) return GH_EUNSUPPORTED;
        sg.w[i] = (const uint8_t*)w[i];
        sg.y[i] = y[i];
        sg.y16[i] = y16 ? y16[i] : nullptr;
        sg.off[i + 1] = sg.off[i] + n[i];
    }
    SkPro pro{nw, eps};
    int rc = GH_OK;
    if (!gemm_skinny(x, w[0], y[0], M, K, sg.off[nseg], row_bytes(kind, K), 0, &rc, mode, pro, &sg, kind))
        return GH_EUNSUPPORTED;
    return rc;
}

// y = x W^T, or y += x W^T with `accumulate` (the split-K sum adds in place; the other paths
// write a temporary that one more launch adds)
template <int KIND>
static int gemm2_launch(const float* x, const void* w, float* y, int M, int K, int N, size_t rowb, int accumulate) {
    const size_t xbytes = ((size_t)M * K * 2 + 255) & ~(size_t)255;
    uint16_t* x16 = (uint16_t*)workspace(WS_GEMM_X, xbytes + (size_t)M * 4);
    if (!x16) return fail(GH_ENOMEM, "gemm: workspace");
    float* rinv = (float*)((uint8_t*)x16 + xbytes);
    hipLaunchKernelGGL(k_to_f16_rows, dim3((unsigned)M), dim3(256), 0, stream(), x, x16, rinv, K);
    GH_LAUNCHED("k_to_f16_rows");
    float* yout = y;  // where the product goes; with accumulate outside the split-K path: a temporary
    auto finish_acc = [&]() -> int {
        if (yout == y) return GH_OK;
        const int64_t n = (int64_t)M * N;
        hipLaunchKernelGGL(k_add_to, dim3((unsigned)std::min<int64_t>(cdiv64(n, 256), 2048)), dim3(256), 0, stream(), y,
                           yout, n);
        GH_LAUNCHED("k_add_to");
        return GH_OK;
    };
    {
        const int blocks = cdiv(M, BM) * cdiv(N, BN), T = K / BK;
        const bool will_split = 2 * blocks <= num_cus() && T >= 4;
        if (accumulate && !will_split) {
            yout = (float*)workspace(WS_GEMM_ACC, (size_t)M * N * 4);
            if (!yout) return fail(GH_ENOMEM, "gemm: workspace");
        }
    }
    if constexpr (KIND == 2 || KIND == 3) {
        const int tiles = cdiv(M, G4M) * cdiv(N, G4N), T = K / 64;
        // 256x256 tiles once they fill the chip (split K in two when that is needed to fill it)
        const int split = tiles >= num_cus() ? 1 : (2 * tiles >= num_cus() && T % 4 == 0) ? 2 : 0;
        if (K % 256 == 0 && split && (split == 1 || ((size_t)M * N % 4 == 0 && ((uintptr_t)yout & 15) == 0))) {
            static bool configured = false;
            if (!configured) {
                const hipError_t e = hipFuncSetAttribute((const void*)k_gemm_q4<KIND>,
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)G4_LDS);
                if (e != hipSuccess) return fail(GH_EHIP, "k_gemm_q4 LDS attribute: %s", hipGetErrorString(e));
                configured = true;
            }
            if (split > 1) {
                const int64_t n4 = (int64_t)M * N / 4;
                hipLaunchKernelGGL(k_zero_f32, dim3((unsigned)std::min<int64_t>(cdiv64(n4, 256), 4096)), dim3(256), 0,
                                   stream(), yout, n4);
            }
            hipLaunchKernelGGL(k_gemm_q4<KIND>, dim3(tiles, split), dim3(256), G4_LDS, stream(), x16, rinv,
                               (const uint8_t*)w, yout, M, K, N, rowb, T / split);
            GH_LAUNCHED("k_gemm_q4");
            return finish_acc();
        }
    }
    const int blocks = cdiv(M, BM) * cdiv(N, BN), T = K / BK;
    // few tiles (small M): split K so more blocks share the sequential K walk, partials summed in order
    int S = 1;
    if (2 * blocks <= num_cus() && T >= 4) {
        S = std::min(T / 2, std::max(1, num_cus() / blocks));
        S = cdiv(T, cdiv(T, S));
    }
    if (S > 1) {
        const int Ts = cdiv(T, S);
        float* part = (float*)workspace(WS_GEMM_PART, (size_t)S * M * N * 4);
        if (!part) return fail(GH_ENOMEM, "gemm: split-K workspace");
        hipLaunchKernelGGL(k_gemm_q2<KIND>, dim3(blocks, S), dim3(256), 0, stream(), x16, rinv, (const uint8_t*)w,
                           part, M, K, N, rowb, Ts);
        const int64_t n = (int64_t)M * N;
        hipLaunchKernelGGL(k_splitk_sum, dim3((unsigned)std::min<int64_t>(cdiv64(n, 256), 2048)), dim3(256), 0,
                           stream(), part, y, n, S, accumulate);
        GH_LAUNCHED("k_gemm_q2 (split K)");
        return GH_OK;
    }
    hipLaunchKernelGGL(k_gemm_q2<KIND>, dim3(blocks), dim3(256), 0, stream(), x16, rinv, (const uint8_t*)w, yout, M, K,
                       N, rowb, T);
    GH_LAUNCHED("k_gemm_q2");
    return finish_acc();
}

int gemm_lib(const float* x, const void* w, float* y, int M, int K, int N, int kind, int accumulate);  // gemm_lib.hip

int gemm_dispatch(const float* x, const void* w, float* y, int M, int K, int N, int kind, int accumulate) {
    {
        const int rc = gemm_lib(x, w, y, M, K, N, kind, accumulate);
        if (rc != GH_EUNSUPPORTED) return rc;
    }
    const int blocks = cdiv(M, BM) * cdiv(N, BN);
    size_t rowb = kind == 4 ? (size_t)K * 2 : kind == 5 ? (size_t)K * 4 : row_bytes(kind, K);
    const dim3 g(blocks), b(256);
    if ((kind == 2 || kind == 3 || kind == 4) && K % 4 == 0) {
        switch (kind) {
            case 2: {
                int rc = GH_OK;
                if (gemm_skinny(x, w, y, M, K, N, rowb, accumulate, &rc, SK_PLAIN, SkPro{}, nullptr, 2)) return rc;
                return gemm2_launch<2>(x, w, y, M, K, N, rowb, accumulate);
            }
            case 3: {
                int rc = GH_OK;
                if (gemm_skinny(x, w, y, M, K, N, rowb, accumulate, &rc)) return rc;
                return gemm2_launch<3>(x, w, y, M, K, N, rowb, accumulate);
            }
            default: return gemm2_launch<4>(x, w, y, M, K, N, rowb, accumulate);
        }
    }
    float* yo = y;
    if (accumulate) {
        yo = (float*)workspace(WS_GEMM_ACC, (size_t)M * N * 4);
        if (!yo) return fail(GH_ENOMEM, "gemm: workspace");
    }
    switch (kind) {
        case 0: hipLaunchKernelGGL(k_gemm_q<0>, g, b, 0, stream(), x, (const uint8_t*)w, yo, M, K, N, rowb); break;
        case 1: hipLaunchKernelGGL(k_gemm_q<1>, g, b, 0, stream(), x, (const uint8_t*)w, yo, M, K, N, rowb); break;
        case 2: hipLaunchKernelGGL(k_gemm_q<2>, g, b, 0, stream(), x, (const uint8_t*)w, yo, M, K, N, rowb); break;
        case 3: hipLaunchKernelGGL(k_gemm_q<3>, g, b, 0, stream(), x, (const uint8_t*)w, yo, M, K, N, rowb); break;
        case 4: hipLaunchKernelGGL(k_gemm_q<4>, g, b, 0, stream(), x, (const uint8_t*)w, yo, M, K, N, rowb); break;
        case 5: hipLaunchKernelGGL(k_gemm_q<5>, g, b, 0, stream(), x, (const uint8_t*)w, yo, M, K, N, rowb); break;
        default: return fail(GH_EINVAL, "gemm: bad kind %d", kind);
    }
    GH_LAUNCHED("k_gemm_q");
    return accumulate ? launch_add_to(y, yo, (int64_t)M * N) : GH_OK;
}

int launch_add_to(float* y, const float* t, int64_t n) {
    hipLaunchKernelGGL(k_add_to, dim3((unsigned)std::min<int64_t>(cdiv64(n, 256), 2048)), dim3(256), 0, stream(), y, t,
                       n);
    GH_LAUNCHED("k_add_to");
    return GH_OK;
}

}  // namespace gh
