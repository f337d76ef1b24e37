// Per-kind decode of one 64-value "task" of a packed weight row and its dot
// with 64 activations (shared by the dense GEMV and the grouped MoE GEMV).
#pragma once
#include "gh_common.h"

namespace gh {

// ----------------------------------------------------------------- GEMV
// internal kinds beyond the packed ones
constexpr int KF16 = 4, KF32 = 5;

template <int KIND>
struct Task;  // bytes per 64-value task and the dot of one task

__device__ __forceinline__ float i8f(uint32_t w, int b) {  // signed byte b of w
    return (float)(int)__builtin_amdgcn_sbfe((int)w, 8 * b, 8);
}
__device__ __forceinline__ float u4f(uint32_t w, int n) {  // nibble n of w
    return (float)__builtin_amdgcn_ubfe(w, 4 * n, 4);
}

// Q8_0: two 34-byte blocks. dwords: [d0|q0 q1][q2..q5]...; block 1 starts at byte 34.
template <>
struct Task<2> {
    static constexpr int DW = 17;
    __device__ static float dot(const uint32_t* w, const float* x) {
        auto byte = [&](int b) { return i8f(w[b >> 2], b & 3); };
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) s0 = fmaf(x[i], byte(2 + i), s0);
#pragma unroll
        for (int i = 0; i < 32; ++i) s1 = fmaf(x[32 + i], byte(36 + i), s1);
        const float d0 = f16_to_f32((uint16_t)(w[0] & 0xFFFF));
        const float d1 = f16_to_f32((uint16_t)(w[8] >> 16));
        return fmaf(d0, s0, d1 * s1);
    }
};
// Q4_0: two 18-byte blocks; low nibble = value j, high nibble = j+16.
template <>
struct Task<0> {
    static constexpr int DW = 9;
    __device__ static float dot(const uint32_t* w, const float* x) {
        auto nib = [&](int byte, int hi) {
            return (float)__builtin_amdgcn_ubfe(w[byte >> 2], 8 * (byte & 3) + 4 * hi, 4);
        };
        float s0 = 0.f, s1 = 0.f, x0 = 0.f, x1 = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            s0 = fmaf(x[j], nib(2 + j, 0), s0);
            s0 = fmaf(x[j + 16], nib(2 + j, 1), s0);
            s1 = fmaf(x[32 + j], nib(20 + j, 0), s1);
            s1 = fmaf(x[48 + j], nib(20 + j, 1), s1);
        }
#pragma unroll
        for (int j = 0; j < 32; ++j) { x0 += x[j]; x1 += x[32 + j]; }
        const float d0 = f16_to_f32((uint16_t)(w[0] & 0xFFFF));
        const float d1 = f16_to_f32((uint16_t)(w[4] >> 16));
        // sum x*(q-8)*d = d*(sum x*q - 8*sum x)
        return d0 * fmaf(-8.f, x0, s0) + d1 * fmaf(-8.f, x1, s1);
    }
};
// Q4_1: two 20-byte blocks, value = q*d + m.
template <>
struct Task<1> {
    static constexpr int DW = 10;
    __device__ static float dot(const uint32_t* w, const float* x) {
        auto nib = [&](int byte, int hi) {
            return (float)__builtin_amdgcn_ubfe(w[byte >> 2], 8 * (byte & 3) + 4 * hi, 4);
        };
        float s0 = 0.f, s1 = 0.f, x0 = 0.f, x1 = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            s0 = fmaf(x[j], nib(4 + j, 0), s0);
            s0 = fmaf(x[j + 16], nib(4 + j, 1), s0);
            s1 = fmaf(x[32 + j], nib(24 + j, 0), s1);
            s1 = fmaf(x[48 + j], nib(24 + j, 1), s1);
        }
#pragma unroll
        for (int j = 0; j < 32; ++j) { x0 += x[j]; x1 += x[32 + j]; }
        const float d0 = f16_to_f32((uint16_t)(w[0] & 0xFFFF)), m0 = f16_to_f32((uint16_t)(w[0] >> 16));
        const float d1 = f16_to_f32((uint16_t)(w[5] & 0xFFFF)), m1 = f16_to_f32((uint16_t)(w[5] >> 16));
        return fmaf(d0, s0, m0 * x0) + fmaf(d1, s1, m1 * x1);
    }
};
// Q4_K: w[0..3] = block header (d, dmin, scales[12]); w[4..11] = 32 bytes of
// nibbles holding sub-blocks 2p (low) and 2p+1 (high); p is passed in.
template <>
struct Task<3> {
    static constexpr int DW = 12;
    __device__ static float dot(const uint32_t* w, const float* x, int p) {
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
        float s0 = 0.f, s1 = 0.f, x0 = 0.f, x1 = 0.f;
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            const uint32_t dw = w[4 + (l >> 2)];
            s0 = fmaf(x[l], (float)__builtin_amdgcn_ubfe(dw, 8 * (l & 3), 4), s0);
            s1 = fmaf(x[32 + l], (float)__builtin_amdgcn_ubfe(dw, 8 * (l & 3) + 4, 4), s1);
            x0 += x[l];
            x1 += x[32 + l];
        }
        const float d = f16_to_f32((uint16_t)(w[0] & 0xFFFF)), dmin = f16_to_f32((uint16_t)(w[0] >> 16));
        int sc0, m0, sc1, m1;
        scale_min(2 * p, sc0, m0);
        scale_min(2 * p + 1, sc1, m1);
        // sum x*(d*sc*q - dmin*m) = d*sc*sum(x q) - dmin*m*sum(x)
        return d * ((float)sc0 * s0 + (float)sc1 * s1) - dmin * ((float)m0 * x0 + (float)m1 * x1);
    }
};
template <>
struct Task<KF16> {
    static constexpr int DW = 32;
    __device__ static float dot(const uint32_t* w, const float* x) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            s = fmaf(x[2 * i], f16_to_f32((uint16_t)(w[i] & 0xFFFF)), s);
            s = fmaf(x[2 * i + 1], f16_to_f32((uint16_t)(w[i] >> 16)), s);
        }
        return s;
    }
};
template <>
struct Task<KF32> {
    static constexpr int DW = 64;
    __device__ static float dot(const uint32_t* w, const float* x) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 64; ++i) s = fmaf(x[i], __builtin_bit_cast(float, w[i]), s);
        return s;
    }
};

template <int KIND>
__device__ __forceinline__ void load_task(const uint8_t* row, int t, uint32_t* w) {
    if constexpr (KIND == 3) {
        const uint8_t* sb = row + (size_t)(t >> 2) * 144;
        const uint4 h = *(const uint4*)sb;
        const uint4 a = *(const uint4*)(sb + 16 + 32 * (t & 3));
        const uint4 b = *(const uint4*)(sb + 32 + 32 * (t & 3));
        w[0] = h.x; w[1] = h.y; w[2] = h.z; w[3] = h.w;
        w[4] = a.x; w[5] = a.y; w[6] = a.z; w[7] = a.w;
        w[8] = b.x; w[9] = b.y; w[10] = b.z; w[11] = b.w;
    } else if constexpr (KIND == KF16 || KIND == KF32) {
        const uint4* s = (const uint4*)(row + (size_t)t * Task<KIND>::DW * 4);
#pragma unroll
        for (int i = 0; i < Task<KIND>::DW / 4; ++i) {
            const uint4 v = s[i];
            w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
        }
    } else {
        const uint32_t* s = (const uint32_t*)(row + (size_t)t * Task<KIND>::DW * 4);
#pragma unroll
        for (int i = 0; i < Task<KIND>::DW; ++i) w[i] = __builtin_nontemporal_load(s + i);
    }
}

template <int KIND>
__device__ __forceinline__ float task_dot(const uint32_t* w, const float* x, int t) {
    if constexpr (KIND == 3) return Task<3>::dot(w, x, t & 3);
    else return Task<KIND>::dot(w, x);
}


}  // namespace gh
