// Prefill GEMM: y[M,N] = x[M,K] dequant(W)[N,K]^T for M > 8, with the
// weights dequantised straight into LDS as bf16 and multiplied on the
// matrix cores (v_mfma_f32_32x32x16_bf16), fp32 accumulation.
// Replaces the cuBLAS path of cuda/kernels.cu:190-441 / :583-633 (which
// first materialised an fp16 copy of the weight in HBM).
//
// Block tile 128 (tokens) x 128 (output rows) x 64 (K), 4 waves in a 2x2
// arrangement, each wave a 64x64 sub-tile = 2x2 MFMA 32x32 tiles. Per K
// step every thread converts 32 activations (fp32 -> bf16) and dequantises
// 32 weights of one row (its half of a 64-value task) into LDS; the next
// K step's global loads are issued before the MFMAs of the current one.
#include "gh_common.h"

namespace gh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

constexpr int BM = 128, BN = 128, BK = 64, LDS_STRIDE = BK + 8;  // in bf16 elements

__device__ __forceinline__ uint16_t bf16_bits(float f) { return f32_to_bf16(f); }

// 32 dequantised weights of row-task half `h` (values 32h..32h+31 of the
// 64-value task t) for each kind, from raw bytes.
template <int KIND>
struct WLoad;

template <>
struct WLoad<2> {  // Q8_0: block t*2+h, 34 bytes, 2-byte aligned
    uint32_t w[9];
    int shift;
    __device__ void load(const uint8_t* row, int t, int h) {
        const size_t off = (size_t)t * 68 + (size_t)h * 34;
        const uint32_t* p = (const uint32_t*)(row + (off & ~(size_t)3));
        shift = (int)(off & 3);  // 0 or 2
#pragma unroll
        for (int i = 0; i < 9; ++i) w[i] = p[i];
    }
    __device__ void decode(float* v) const {
        // byte b of the block is stream byte shift + b
        auto byte = [&](int b) {
            const int s = shift + b;
            return (int)__builtin_amdgcn_sbfe((int)w[s >> 2], 8 * (s & 3), 8);
        };
        const int s0 = shift;
        const uint32_t dbits = (s0 == 0) ? (w[0] & 0xFFFF) : (w[0] >> 16);
        const float d = f16_to_f32((uint16_t)dbits);
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = (float)byte(2 + i) * d;
    }
};
template <>
struct WLoad<0> {  // Q4_0: block t*2+h, 18 bytes
    uint32_t w[5];
    int shift;
    __device__ void load(const uint8_t* row, int t, int h) {
        const size_t off = (size_t)t * 36 + (size_t)h * 18;
        const uint32_t* p = (const uint32_t*)(row + (off & ~(size_t)3));
        shift = (int)(off & 3);
#pragma unroll
        for (int i = 0; i < 5; ++i) w[i] = p[i];
    }
    __device__ void decode(float* v) const {
        auto ub = [&](int b) { const int s = shift + b; return (w[s >> 2] >> (8 * (s & 3))) & 0xFF; };
        const float d = f16_to_f32((uint16_t)(ub(0) | (ub(1) << 8)));
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t b = ub(2 + j);
            v[j] = (float)((int)(b & 0xF) - 8) * d;
            v[j + 16] = (float)((int)(b >> 4) - 8) * d;
        }
    }
};
template <>
struct WLoad<1> {  // Q4_1: 20 bytes, 4-byte aligned
    uint32_t w[5];
    __device__ void load(const uint8_t* row, int t, int h) {
        const uint32_t* p = (const uint32_t*)(row + (size_t)t * 40 + (size_t)h * 20);
#pragma unroll
        for (int i = 0; i < 5; ++i) w[i] = p[i];
    }
    __device__ void decode(float* v) const {
        const float d = f16_to_f32((uint16_t)(w[0] & 0xFFFF)), mn = f16_to_f32((uint16_t)(w[0] >> 16));
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t b = (w[1 + (j >> 2)] >> (8 * (j & 3))) & 0xFF;
            v[j] = (float)(b & 0xF) * d + mn;
            v[j + 16] = (float)(b >> 4) * d + mn;
        }
    }
};
template <>
struct WLoad<3> {  // Q4_K: header + 32 nibble bytes of the pair; h picks low/high
    uint4 hd, a, b;
    int p, h;
    __device__ void load(const uint8_t* row, int t, int hh) {
        const uint8_t* sb = row + (size_t)(t >> 2) * 144;
        p = t & 3;
        h = hh;
        hd = *(const uint4*)sb;
        a = *(const uint4*)(sb + 16 + 32 * p);
        b = *(const uint4*)(sb + 32 + 32 * p);
    }
    __device__ void decode(float* v) const {
        const uint32_t sc4[3] = {hd.y, hd.z, hd.w};
        auto scb = [&](int i) { return (int)((sc4[i >> 2] >> (8 * (i & 3))) & 0xFF); };
        const int s = 2 * p + h;
        int scv, mv;
        if (s < 4) {
            scv = scb(s) & 63;
            mv = scb(s + 4) & 63;
        } else {
            scv = (scb(s + 4) & 0xF) | ((scb(s - 4) >> 6) << 4);
            mv = (scb(s + 4) >> 4) | ((scb(s) >> 6) << 4);
        }
        const float d1 = f16_to_f32((uint16_t)(hd.x & 0xFFFF)) * (float)scv;
        const float m1 = f16_to_f32((uint16_t)(hd.x >> 16)) * (float)mv;
        const uint32_t q[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            const float qq = (float)((q[l >> 2] >> (8 * (l & 3) + 4 * h)) & 0xF);
            v[l] = d1 * qq - m1;
        }
    }
};
template <>
struct WLoad<4> {  // fp16 weights: 64 bytes
    uint4 r[4];
    __device__ void load(const uint8_t* row, int t, int h) {
        const uint4* p = (const uint4*)(row + (size_t)t * 128 + (size_t)h * 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = p[i];
    }
    __device__ void decode(float* v) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t u[4] = {r[i].x, r[i].y, r[i].z, r[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[8 * i + 2 * j] = f16_to_f32((uint16_t)(u[j] & 0xFFFF));
                v[8 * i + 2 * j + 1] = f16_to_f32((uint16_t)(u[j] >> 16));
            }
        }
    }
};
template <>
struct WLoad<5> {  // fp32 weights: 128 bytes
    float4 r[8];
    __device__ void load(const uint8_t* row, int t, int h) {
        const float4* p = (const float4*)(row + (size_t)t * 256 + (size_t)h * 128);
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = p[i];
    }
    __device__ void decode(float* v) const {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[4 * i] = r[i].x; v[4 * i + 1] = r[i].y; v[4 * i + 2] = r[i].z; v[4 * i + 3] = r[i].w;
        }
    }
};

__device__ __forceinline__ void store_bf16x32(uint16_t* dst, const float* v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        u16x8 o;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = bf16_bits(v[8 * i + j]);
        *(u16x8*)(dst + 8 * i) = o;
    }
}

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
        // registers -> LDS (bf16)
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
            store_bf16x32(sA + lr * LDS_STRIDE + lh * 32, v);
            wl.decode(v);
            if (bn >= N) {
#pragma unroll
                for (int i = 0; i < 32; ++i) v[i] = 0.f;
            }
            store_bf16x32(sB + lr * LDS_STRIDE + lh * 32, v);
        }
        __syncthreads();
        if (t + 1 < T) gload(t + 1);
        // 4 k-slices of 16
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int kofs = ks * 16 + (lane >> 5) * 8;
            bf16x8 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                a[i] = *(const bf16x8*)(sA + (wm + i * 32 + (lane & 31)) * LDS_STRIDE + kofs);
                b[i] = *(const bf16x8*)(sB + (wn + i * 32 + (lane & 31)) * LDS_STRIDE + kofs);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
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
