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

#include "gemm_tile.h"

namespace gh {

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

template <int KIND>
__global__ void __launch_bounds__(256, 2) k_gemm_q2(const uint16_t* __restrict__ X16, const uint8_t* __restrict__ W,
                                                   float* __restrict__ Y, int M, int K, int N, size_t rowb) {
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
    const int T = K / BK;
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

// ---------------------------------------------------------------- v3
// Large tiles for large M: a block of 4 waves computes 256x256, each wave
// 128x128 as 4x4 v_mfma_f32_32x32x16_f16 tiles (accumulators in the
// accumulation registers, one wave per SIMD). Per K step of 64 a wave issues
// 64 MFMAs (2048 cycles at the issue rate) against 32 16-byte operand reads
// from LDS, so the matrix cores rather than LDS bound the step (the 128x128
// tile of v2 read one operand per MFMA). LDS double-buffered, one barrier per
// step, next step's pieces in registers while the MFMAs run.
constexpr int B3M = 256, B3N = 256;
template <int KIND>
__global__ void __launch_bounds__(256, 1) k_gemm_q3(const uint16_t* __restrict__ X16, const uint8_t* __restrict__ W,
                                                   float* __restrict__ Y, int M, int K, int N, size_t rowb) {
    extern __shared__ __attribute__((aligned(16))) uint16_t g3_smem[];
    uint16_t* sA0 = g3_smem;                        // [2][B3M * LDS_STRIDE]
    uint16_t* sB0 = g3_smem + 2 * B3M * LDS_STRIDE;  // [2][B3N * LDS_STRIDE]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tilesN = cdiv(N, B3N), tilesM = cdiv(M, B3M);
    const int nblk = tilesN * tilesM;
    int bid = blockIdx.x;
    if (nblk % 8 == 0) bid = (bid % 8) * (nblk / 8) + bid / 8;  // XCD-aware: an XCD keeps a run of N tiles
    const int tm = bid % tilesM, tn = bid / tilesM;
    const int m0 = tm * B3M, n0 = tn * B3N;
    // A pieces: thread -> rows ar + 32 i (i < 8), 8 halves at ac
    const int ar = tid >> 3, ac = (tid & 7) * 8;
    // B: thread -> row tid, both halves of the step's 64 values
    const int bn = n0 + tid;
    const uint8_t* wrow = W + (size_t)(bn < N ? bn : N - 1) * rowb;
    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    const int wm = (wave >> 1) * 128, wn = (wave & 1) * 128;
    const int T = K / BK;
    uint32_t magic = 0x64006400u;
    asm volatile("" : "+v"(magic));

    gh_u32x4v xa[8];
    WLoad<KIND> wl0, wl1;
    size_t xoff[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int am = m0 + ar + 32 * i;
        xoff[i] = (size_t)(am < M ? am : M - 1) * K + ac;
    }
    // the blocks of one M tile (and of one N tile) run together and would read the same lines in
    // lockstep: each block starts its K walk at its own step
    const int t0 = (tn * 5 + tm * 3) % T;
#pragma unroll
    for (int i = 0; i < 8; ++i) xa[i] = *(const gh_u32x4v*)(X16 + xoff[i] + (size_t)t0 * BK);
    wl0.load(wrow, t0, 0);
    wl1.load(wrow, t0, 1);
    int buf = 0;
    for (int tt = 0; tt < T; ++tt, buf ^= 1) {
        const int tnext = tt + 1 + t0 < T ? tt + 1 + t0 : tt + 1 + t0 - T;
        uint16_t* sA = sA0 + buf * B3M * LDS_STRIDE;
        uint16_t* sB = sB0 + buf * B3N * LDS_STRIDE;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            gh_u32x4v v = xa[i];
            if (m0 + ar + 32 * i >= M) v = gh_u32x4v{0u, 0u, 0u, 0u};
            *(gh_u32x4v*)(sA + (ar + 32 * i) * LDS_STRIDE + ac) = v;
        }
        {
            uint16_t* dst = sB + tid * LDS_STRIDE;
            if (bn < N) {
                decode16<KIND>(wl0, dst, magic);
                decode16<KIND>(wl1, dst + 32, magic);
            } else {
                float z[32];
#pragma unroll
                for (int i = 0; i < 32; ++i) z[i] = 0.f;
                store_f16x32(dst, z);
                store_f16x32(dst + 32, z);
            }
        }
        __syncthreads();
        if (tt + 1 < T) {
#pragma unroll
            for (int i = 0; i < 8; ++i) xa[i] = *(const gh_u32x4v*)(X16 + xoff[i] + (size_t)tnext * BK);
            wl0.load(wrow, tnext, 0);
            wl1.load(wrow, tnext, 1);
        }
        // operand fragments of k-substep ks + 1 are read while the MFMAs of ks run
        f16x8 a[2][4], b[2][4];
        auto frag = [&](int ks, f16x8 (&fa)[4], f16x8 (&fb)[4]) {
            const int kofs = ks * 16 + (lane >> 5) * 8;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                fa[i] = *(const f16x8*)(sA + (wm + i * 32 + (lane & 31)) * LDS_STRIDE + kofs);
                fb[i] = *(const f16x8*)(sB + (wn + i * 32 + (lane & 31)) * LDS_STRIDE + kofs);
            }
        };
        frag(0, a[0], b[0]);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            if (ks + 1 < BK / 16) frag(ks + 1, a[(ks + 1) & 1], b[(ks + 1) & 1]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[ks & 1][i], b[ks & 1][j], acc[i][j], 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = n0 + wn + j * 32 + (lane & 31);
            if (col >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row < M) Y[(size_t)row * N + col] = acc[i][j][e];
            }
        }
}
constexpr size_t G3_LDS = (size_t)2 * (B3M + B3N) * LDS_STRIDE * 2;

int launch_to_f16(const float* x, uint16_t* y, int64_t n) {
    const int64_t n4 = n / 4;
    hipLaunchKernelGGL(k_to_f16, dim3((unsigned)std::min<int64_t>(cdiv64(n4, 256), 8192)), dim3(256), 0, stream(), x,
                       y, n4);
    GH_LAUNCHED("k_to_f16");
    return GH_OK;
}

template <int KIND>
static int gemm2_launch(const float* x, const void* w, float* y, int M, int K, int N, size_t rowb) {
    uint16_t* x16 = (uint16_t*)workspace(WS_GEMM_X, (size_t)M * K * 2);
    if (!x16) return fail(GH_ENOMEM, "gemm: workspace");
    const int64_t n4 = (int64_t)M * K / 4;
    hipLaunchKernelGGL(k_to_f16, dim3((unsigned)std::min<int64_t>(cdiv64(n4, 256), 8192)), dim3(256), 0, stream(), x,
                       x16, n4);
    static const int v3 = [] {
        const char* e = getenv("GH_GEMM_V3");
        return e ? atoi(e) : 1;
    }();
    if (v3 && (int64_t)cdiv(M, B3M) * cdiv(N, B3N) >= num_cus()) {  // large tiles once they fill the chip
        static bool configured = false;
        if (!configured) {
            const hipError_t e = hipFuncSetAttribute((const void*)k_gemm_q3<KIND>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)G3_LDS);
            if (e != hipSuccess) return fail(GH_EHIP, "k_gemm_q3 LDS attribute: %s", hipGetErrorString(e));
            configured = true;
        }
        const int blocks = cdiv(M, B3M) * cdiv(N, B3N);
        hipLaunchKernelGGL(k_gemm_q3<KIND>, dim3(blocks), dim3(256), G3_LDS, stream(), x16, (const uint8_t*)w, y, M, K,
                           N, rowb);
        GH_LAUNCHED("k_gemm_q3");
        return GH_OK;
    }
    const int blocks = cdiv(M, BM) * cdiv(N, BN);
    hipLaunchKernelGGL(k_gemm_q2<KIND>, dim3(blocks), dim3(256), 0, stream(), x16, (const uint8_t*)w, y, M, K, N,
                       rowb);
    GH_LAUNCHED("k_gemm_q2");
    return GH_OK;
}

int gemm_dispatch(const float* x, const void* w, float* y, int M, int K, int N, int kind) {
    const int blocks = cdiv(M, BM) * cdiv(N, BN);
    size_t rowb = kind == 4 ? (size_t)K * 2 : kind == 5 ? (size_t)K * 4 : row_bytes(kind, K);
    const dim3 g(blocks), b(256);
    static const int v2 = [] {
        const char* e = getenv("GH_GEMM_V2");
        return e ? atoi(e) : 1;
    }();
    if (v2 && (kind == 2 || kind == 3 || kind == 4) && K % 4 == 0) {
        switch (kind) {
            case 2: return gemm2_launch<2>(x, w, y, M, K, N, rowb);
            case 3: return gemm2_launch<3>(x, w, y, M, K, N, rowb);
            default: return gemm2_launch<4>(x, w, y, M, K, N, rowb);
        }
    }
    switch (kind) {
        case 0: hipLaunchKernelGGL(k_gemm_q<0>, g, b, 0, stream(), x, (const uint8_t*)w, y, M, K, N, rowb); break;
        case 1: hipLaunchKernelGGL(k_gemm_q<1>, g, b, 0, stream(), x, (const uint8_t*)w, y, M, K, N, rowb); break;
        case 2: hipLaunchKernelGGL(k_gemm_q<2>, g, b, 0, stream(), x, (const uint8_t*)w, y, M, K, N, rowb); break;
        case 3: hipLaunchKernelGGL(k_gemm_q<3>, g, b, 0, stream(), x, (const uint8_t*)w, y, M, K, N, rowb); break;
        case 4: hipLaunchKernelGGL(k_gemm_q<4>, g, b, 0, stream(), x, (const uint8_t*)w, y, M, K, N, rowb); break;
        case 5: hipLaunchKernelGGL(k_gemm_q<5>, g, b, 0, stream(), x, (const uint8_t*)w, y, M, K, N, rowb); break;
        default: return fail(GH_EINVAL, "gemm: bad kind %d", kind);
    }
    GH_LAUNCHED("k_gemm_q");
    return GH_OK;
}

}  // namespace gh
