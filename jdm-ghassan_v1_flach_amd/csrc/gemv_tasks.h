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

// Unsigned byte b of a dword as float: compiles to v_cvt_f32_ubyte{b}.
__device__ __forceinline__ float ub(uint32_t w, int b) { return (float)((w >> (8 * b)) & 0xFFu); }

// The dot of one task: w = raw dwords, x = 64 activations, xs = sums of
// x[0..31] and x[32..63] (computed once per task and reused by every row).
// Integer codes are turned into floats straight from bytes (low nibbles by
// masking 0x0F0F0F0F, high nibbles by shifting first, signed Q8_0 bytes by
// flipping the sign bit: q = u - 128), so a weight costs about one convert
// and one FMA.

// Q8_0: two 34-byte blocks; block 0 quants are stream bytes 2..33, block 1
// quants 36..67, scales at bytes 0-1 and 34-35.
template <>
struct Task<2> {
    static constexpr int DW = 17;
    __device__ static float dot(const uint32_t* w, const float* x, const float* xs) {
        uint32_t u[17];
#pragma unroll
        for (int i = 0; i < 17; ++i) u[i] = w[i] ^ 0x80808080u;
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const int b0 = 2 + i, b1 = 36 + i;
            s0 = fmaf(x[i], ub(u[b0 >> 2], b0 & 3), s0);
            s1 = fmaf(x[32 + i], ub(u[b1 >> 2], b1 & 3), s1);
        }
        const float d0 = f16_to_f32((uint16_t)(w[0] & 0xFFFF));
        const float d1 = f16_to_f32((uint16_t)(w[8] >> 16));
        return d0 * fmaf(-128.f, xs[0], s0) + d1 * fmaf(-128.f, xs[1], s1);
    }
};
// Q4_0: two 18-byte blocks; low nibble = value j, high nibble = j+16,
// value = (q - 8) * d.
template <>
struct Task<0> {
    static constexpr int DW = 9;
    __device__ static float dot(const uint32_t* w, const float* x, const float* xs) {
        // block 0 nibble bytes are stream bytes 2..17, block 1 bytes 20..35
        auto byte = [&](int b) { return (w[b >> 2] >> (8 * (b & 3))) & 0xFFu; };
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t b0 = byte(2 + j), b1 = byte(20 + j);
            s0 = fmaf(x[j], (float)(b0 & 0xF), s0);
            s0 = fmaf(x[j + 16], (float)(b0 >> 4), s0);
            s1 = fmaf(x[32 + j], (float)(b1 & 0xF), s1);
            s1 = fmaf(x[48 + j], (float)(b1 >> 4), s1);
        }
        const float d0 = f16_to_f32((uint16_t)(w[0] & 0xFFFF));
        const float d1 = f16_to_f32((uint16_t)(w[4] >> 16));
        return d0 * fmaf(-8.f, xs[0], s0) + d1 * fmaf(-8.f, xs[1], s1);
    }
};
// Q4_1: two 20-byte blocks (4-byte aligned), value = q*d + m.
template <>
struct Task<1> {
    static constexpr int DW = 10;
    __device__ static float dot(const uint32_t* w, const float* x, const float* xs) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo0 = w[1 + i] & 0x0F0F0F0Fu, hi0 = (w[1 + i] >> 4) & 0x0F0F0F0Fu;
            const uint32_t lo1 = w[6 + i] & 0x0F0F0F0Fu, hi1 = (w[6 + i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int j = 4 * i + b;
                s0 = fmaf(x[j], ub(lo0, b), s0);
                s0 = fmaf(x[j + 16], ub(hi0, b), s0);
                s1 = fmaf(x[32 + j], ub(lo1, b), s1);
                s1 = fmaf(x[48 + j], ub(hi1, b), s1);
            }
        }
        const float d0 = f16_to_f32((uint16_t)(w[0] & 0xFFFF)), m0 = f16_to_f32((uint16_t)(w[0] >> 16));
        const float d1 = f16_to_f32((uint16_t)(w[5] & 0xFFFF)), m1 = f16_to_f32((uint16_t)(w[5] >> 16));
        return fmaf(d0, s0, m0 * xs[0]) + fmaf(d1, s1, m1 * xs[1]);
    }
};
// Q4_K: w[0..3] = block header (d, dmin, scales[12]); w[4..11] = the 32
// nibble bytes holding sub-blocks 2p (low nibbles) and 2p+1 (high nibbles).
template <>
struct Task<3> {
    static constexpr int DW = 12;
    __device__ static float dot(const uint32_t* w, const float* x, const float* xs, int p) {
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
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lo = w[4 + i] & 0x0F0F0F0Fu, hi = (w[4 + i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                s0 = fmaf(x[4 * i + b], ub(lo, b), s0);
                s1 = fmaf(x[32 + 4 * i + b], ub(hi, b), s1);
            }
        }
        const float d = f16_to_f32((uint16_t)(w[0] & 0xFFFF)), dmin = f16_to_f32((uint16_t)(w[0] >> 16));
        int sc0, m0, sc1, m1;
        scale_min(2 * p, sc0, m0);
        scale_min(2 * p + 1, sc1, m1);
        // sum x*(d*sc*q - dmin*m) = d*sc*sum(x q) - dmin*m*sum(x)
        return d * ((float)sc0 * s0 + (float)sc1 * s1) - dmin * ((float)m0 * xs[0] + (float)m1 * xs[1]);
    }
};
template <>
struct Task<KF16> {
    static constexpr int DW = 32;
    __device__ static float dot(const uint32_t* w, const float* x, const float* xs) {
        (void)xs;
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
    __device__ static float dot(const uint32_t* w, const float* x, const float* xs) {
        (void)xs;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 64; ++i) s = fmaf(x[i], __builtin_bit_cast(float, w[i]), s);
        return s;
    }
};

// sums of the two 32-value halves of a task's activations (only the
// affine codecs need them)
template <int KIND>
__device__ __forceinline__ void task_xsum(const float* x, float* xs) {
    if constexpr (KIND == KF16 || KIND == KF32) {
        xs[0] = xs[1] = 0.f;
    } else {
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            a += x[i];
            b += x[32 + i];
        }
        xs[0] = a;
        xs[1] = b;
    }
}

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
__device__ __forceinline__ float task_dot(const uint32_t* w, const float* x, const float* xs, int t) {
    if constexpr (KIND == 3) return Task<3>::dot(w, x, xs, t & 3);
    else return Task<KIND>::dot(w, x, xs);
}


}  // namespace gh
