// Single-token GEMV (M = 1) for Q4_K and Q8_0 weights -- the decode hot path.
//
// Budget: at 8 TB/s a Q4_K weight arrives every ~0.07 ns chip-wide, which
// leaves ~2.7 VALU lane-ops per weight. The kernel therefore spends about
// 1.9: integer codes become fp16 values with ONE v_and_or_b32 per pair
// (code | 0x6400 is the fp16 number 1024 + code; signed Q8_0 bytes are
// first flipped to 128 + q), and each weight costs one v_fma_mix_f32
// (fp16 code x fp32 activation, exact product, fp32 accumulate). The
// constant bias is removed once per sub-block with the activation sum:
//   sum x*(d1*q - m1) = d1*(sum x*(1024+q) - 1024*sum x) - m1*sum x.
//
// Work layout: a block is 4 waves; the K range of a row is split over WK
// waves (64 lanes x 64 values each, WK = 1, 2 or 4), so every lane owns ONE
// fixed 64-value task: its activations are loaded and summed once, before
// the persistent loop over row groups starts. The next group's packed bytes
// are prefetched while the current group is multiplied. Partial sums are
// reduced across lanes with shuffles and across the WK waves through LDS,
// in a fixed order (deterministic).
#include <stdlib.h>

#include "gemv_tasks.h"

namespace gh {

__device__ __forceinline__ float lo16(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFFu)); }
__device__ __forceinline__ float hi16(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }

// (a & m) | c in one v_and_or_b32 (VOP3 on gfx9 takes no literal, so the
// two constants are passed in registers; left to itself the compiler emits
// an and + an or with literals).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
    uint32_t r;
    asm volatile("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(c));
    return r;
}

// sum of x[i] * (1024 + nibble) over the 64 values of a Q4_K task, as two
// sub-block sums: low nibbles (sub-block 2p) and high nibbles (2p+1).
__device__ __forceinline__ void q4k_mix(const uint32_t* qs, const float* x, float& s0, float& s1, uint32_t magic) {
    constexpr uint32_t M4 = 0x000F000Fu;
    s0 = 0.f;
    s1 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t w = qs[i];
        // bytes b0..b3 = positions l = 4i..4i+3
        const uint32_t a = and_or(w, M4, magic);          // low nibbles of b0, b2
        const uint32_t b = and_or(w >> 8, M4, magic);     // low nibbles of b1, b3
        const uint32_t c = and_or(w >> 4, M4, magic);     // high nibbles of b0, b2
        const uint32_t d = and_or(w >> 12, M4, magic);    // high nibbles of b1, b3
        const float* xl = x + 4 * i;
        const float* xh = x + 32 + 4 * i;
        s0 = fmaf(lo16(a), xl[0], s0);
        s0 = fmaf(hi16(a), xl[2], s0);
        s0 = fmaf(lo16(b), xl[1], s0);
        s0 = fmaf(hi16(b), xl[3], s0);
        s1 = fmaf(lo16(c), xh[0], s1);
        s1 = fmaf(hi16(c), xh[2], s1);
        s1 = fmaf(lo16(d), xh[1], s1);
        s1 = fmaf(hi16(d), xh[3], s1);
    }
}

// Sum over the 64 lanes with DPP row operations (no LDS crossbar): within
// rows of 16 by xor-1/2 quad permutes and row mirrors, then across rows.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));  // quad [1,0,3,2]
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));  // quad [2,3,0,1]
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true)); // row_half_mirror
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true)); // row_mirror
    // every lane of a row now holds the row sum; combine the 4 rows
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

template <int KIND>
__device__ __forceinline__ float task_dot1(const uint32_t* w, const float* x, const float* xs, int p,
                                           uint32_t magic) {
    if constexpr (KIND == 3) {
        float s0, s1;
        q4k_mix(w + 4, x, s0, s1, magic);
        auto scb = [&](int i) { return (int)((w[1 + (i >> 2)] >> (8 * (i & 3))) & 0xFF); };
        auto scale_min = [&](int s, int& sc, int& m) {
            if (s < 4) {
                sc = scb(s) & 63;
                m = scb(s + 4) & 63;
            } else {
                sc = (scb(s + 4) & 0xF) | ((scb(s - 4) >> 6) << 4);
                m = (scb(s + 4) >> 4) | ((scb(s) >> 6) << 4);
            }
        };
        int sc0, m0, sc1, m1;
        scale_min(2 * p, sc0, m0);
        scale_min(2 * p + 1, sc1, m1);
        const float d = lo16(w[0]), dmin = hi16(w[0]);
        const float q0 = fmaf(-1024.f, xs[0], s0), q1 = fmaf(-1024.f, xs[1], s1);
        return d * ((float)sc0 * q0 + (float)sc1 * q1) - dmin * ((float)m0 * xs[0] + (float)m1 * xs[1]);
    } else {
        // Q8_0: two 34-byte blocks in 17 dwords. Block 0 quants are stream
        // bytes 2..33, block 1 quants bytes 36..67; byte b of the stream is
        // byte b%4 of dword b/4. Flipping the sign bit gives u = q + 128, and
        // (u | 0x6400) as fp16 is 1024 + u = 1152 + q.
        constexpr uint32_t M8 = 0x00FF00FFu;
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 17; ++j) {
            const uint32_t u = w[j] ^ 0x80808080u;
            const uint32_t a = and_or(u, M8, magic);       // bytes 4j, 4j+2
            const uint32_t b = and_or(u >> 8, M8, magic);  // bytes 4j+1, 4j+3
            const int bb[4] = {4 * j, 4 * j + 1, 4 * j + 2, 4 * j + 3};
            const float v[4] = {lo16(a), lo16(b), hi16(a), hi16(b)};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int by = bb[e];
                if (by >= 2 && by < 34) s0 = fmaf(v[e], x[by - 2], s0);
                else if (by >= 36) s1 = fmaf(v[e], x[32 + by - 36], s1);
            }
        }
        const float d0 = lo16(w[0]), d1 = hi16(w[8]);
        return d0 * fmaf(-1152.f, xs[0], s0) + d1 * fmaf(-1152.f, xs[1], s1);
    }
}

template <int KIND, int R>
__global__ void __launch_bounds__(256) k_gemv1(const float* __restrict__ x, const uint8_t* __restrict__ W,
                                               float* __restrict__ y, int K, int N, size_t rowb, int WK, int iters) {
    __shared__ float red[2][4][R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int T = K / 64;
    const int kw = wave % WK, gslot = wave / WK;
    const int GPB = 4 / WK;  // row groups per block per iteration
    const int t = kw * 64 + lane;
    const bool valid = t < T && gslot < GPB;
    const int tt = t < T ? t : T - 1;
    // this lane's activations, loaded and summed once. The block stages x
    // in LDS first (one L2 read of x per block instead of one per wave).
    extern __shared__ float sx[];
    for (int i = threadIdx.x * 4; i < K; i += 256 * 4) *(float4*)(sx + i) = *(const float4*)(x + i);
    __syncthreads();
    float xv[64], xs[2];
    {
        const float4* xp = (const float4*)(sx + (size_t)tt * 64);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 v = xp[i];
            xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
        }
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            a += xv[i];
            b += xv[32 + i];
        }
        xs[0] = a;
        xs[1] = b;
    }
    const float vmask = valid ? 1.0f : 0.0f;
    // the fp16 magic kept in a register (read by v_and_or_b32)
    uint32_t magic = 0x64006400u;
    asm volatile("" : "+v"(magic));
    const int ngroups = (N + R - 1) / R;
    const int gstride = gridDim.x * GPB;
    int grp = blockIdx.x * GPB + (gslot < GPB ? gslot : 0);
    auto load_group = [&](int g, uint32_t (*w)[Task<KIND>::DW]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int n = g * R + r;
            n = n < N ? n : N - 1;
            load_task<KIND>(W + (size_t)n * rowb, tt, w[r]);
        }
    };
    uint32_t wc[R][Task<KIND>::DW], wn[R][Task<KIND>::DW];
    load_group(grp < ngroups ? grp : ngroups - 1, wc);
    for (int it = 0; it < iters; ++it) {
        const int ng = grp + gstride;
        if (it + 1 < iters) load_group(ng < ngroups ? ng : ngroups - 1, wn);
        float part[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = task_dot1<KIND>(wc[r], xv, xs, tt & 3, magic) * vmask;
            part[r] = wave_sum_dpp(v);
        }
        if (WK == 1) {
            if (lane < R && grp < ngroups && gslot < GPB) {
                const int n = grp * R + lane;
                float v = part[0];
#pragma unroll
                for (int r = 1; r < R; ++r)
                    if (lane == r) v = part[r];
                if (n < N) y[n] = v;
            }
        } else {
            const int buf = it & 1;
            if (lane == 0 && gslot < GPB)
#pragma unroll
                for (int r = 0; r < R; ++r) red[buf][wave][r] = part[r];
            __syncthreads();
            if (kw == 0 && lane < R && grp < ngroups && gslot < GPB) {
                float v = 0.f;
                for (int k = 0; k < WK; ++k) v += red[buf][gslot * WK + k][lane];
                const int n = grp * R + lane;
                if (n < N) y[n] = v;
            }
        }
        grp = ng;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < Task<KIND>::DW; ++i) wc[r][i] = wn[r][i];
    }
}

// waves per CU of the persistent grid and rows per lane
constexpr int GEMV1_WPC = 8;
constexpr int GEMV1_R = 2;

template <int R>
static void launch1(const float* x, const void* w, float* y, int K, int N, int kind, int WK) {
    const int GPB = 4 / WK;
    const int ngroups = cdiv(N, R);
    const int max_blocks = GEMV1_WPC * num_cus() / 4;
    int blocks = cdiv(ngroups, GPB);
    if (blocks > max_blocks) blocks = max_blocks;
    const int iters = cdiv(ngroups, blocks * GPB);
    const size_t rowb = row_bytes(kind, K);
    if (kind == 3)
        hipLaunchKernelGGL((k_gemv1<3, R>), dim3(blocks), dim3(256), (size_t)K * 4, stream(), x, (const uint8_t*)w, y, K, N, rowb,
                           WK, iters);
    else
        hipLaunchKernelGGL((k_gemv1<2, R>), dim3(blocks), dim3(256), (size_t)K * 4, stream(), x, (const uint8_t*)w, y, K, N, rowb,
                           WK, iters);
}

// returns 1 if handled
int gemv1_dispatch(const float* x, const void* w, float* y, int K, int N, int kind, int* rc) {
    if (kind != 2 && kind != 3) return 0;
    const int T = K / 64;
    if (T > 256) return 0;
    const int WK = T <= 64 ? 1 : T <= 128 ? 2 : 4;
    const int r = GEMV1_R;
    if (r == 1) launch1<1>(x, w, y, K, N, kind, WK);
    else if (r == 4) launch1<4>(x, w, y, K, N, kind, WK);
    else launch1<2>(x, w, y, K, N, kind, WK);
    hipError_t e = hipGetLastError();
    *rc = e == hipSuccess ? GH_OK : fail(GH_EHIP, "launch of k_gemv1 failed: %s", hipGetErrorString(e));
    return 1;
}

}  // namespace gh
