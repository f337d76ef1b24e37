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

int gemm_dispatch(const float* x, const void* w, float* y, int M, int K, int N, int kind) {
    const int blocks = cdiv(M, BM) * cdiv(N, BN);
    size_t rowb = kind == 4 ? (size_t)K * 2 : kind == 5 ? (size_t)K * 4 : row_bytes(kind, K);
    const dim3 g(blocks), b(256);
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
