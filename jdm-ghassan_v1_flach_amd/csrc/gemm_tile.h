// Weight-tile loaders of the MFMA GEMMs: raw bytes of 32 values of one row
// (half of a 64-value task) and their dequantisation to fp32, per kind.
#pragma once
#include "gh_common.h"

namespace gh {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4v __attribute__((ext_vector_type(4)));
typedef uint32_t gh_u32x4v __attribute__((ext_vector_type(4)));

inline int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }

constexpr int BM = 128, BN = 128, BK = 64, LDS_STRIDE = BK + 8;  // in fp16 elements


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

__device__ __forceinline__ void store_f16x32(uint16_t* dst, const float* v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f16x8 o;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = (_Float16)v[8 * i + j];  // RNE, as fp32_to_fp16
        *(f16x8*)(dst + 8 * i) = o;
    }
}


}  // namespace gh
