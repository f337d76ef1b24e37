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


// ---- fp16 weight decode of the MFMA GEMMs (32 values of a row-task half
// into LDS): fp16 integer codes by one v_and_or_b32 per pair (code | 0x6400
// is the fp16 number 1024 + code), scaled by one v_fma_mix_f32 each.
__device__ __forceinline__ uint32_t gq_and_or(uint32_t a, uint32_t m, uint32_t c) {
    uint32_t r;
    asm volatile("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(c));
    return r;
}
__device__ __forceinline__ float gq_lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFF)); }
__device__ __forceinline__ float gq_hi(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }

// 32 weights of a row-task half as fp16 into dst (LDS)
template <int KIND>
__device__ __forceinline__ void decode16(const WLoad<KIND>& wl, uint16_t* dst, uint32_t magic) {
    float v[32];
    if constexpr (KIND == 3) {
        const uint32_t sc4[3] = {wl.hd.y, wl.hd.z, wl.hd.w};
        auto scb = [&](int i) { return (int)((sc4[i >> 2] >> (8 * (i & 3))) & 0xFF); };
        const int s = 2 * wl.p + wl.h;
        int scv, mv;
        if (s < 4) {
            scv = scb(s) & 63;
            mv = scb(s + 4) & 63;
        } else {
            scv = (scb(s + 4) & 0xF) | ((scb(s - 4) >> 6) << 4);
            mv = (scb(s + 4) >> 4) | ((scb(s) >> 6) << 4);
        }
        const float d1 = f16_to_f32((uint16_t)(wl.hd.x & 0xFFFF)) * (float)scv;
        const float m1 = f16_to_f32((uint16_t)(wl.hd.x >> 16)) * (float)mv;
        const float nb = -fmaf(1024.f, d1, m1);  // (1024 + q) * d1 + nb = q * d1 - m1
        const uint32_t q[8] = {wl.a.x, wl.a.y, wl.a.z, wl.a.w, wl.b.x, wl.b.y, wl.b.z, wl.b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t w = q[i] >> (4 * wl.h);
            const uint32_t c0 = gq_and_or(w, 0x000F000Fu, magic);       // values 4i, 4i+2
            const uint32_t c1 = gq_and_or(w >> 8, 0x000F000Fu, magic);  // values 4i+1, 4i+3
            v[4 * i] = fmaf(gq_lo(c0), d1, nb);
            v[4 * i + 1] = fmaf(gq_lo(c1), d1, nb);
            v[4 * i + 2] = fmaf(gq_hi(c0), d1, nb);
            v[4 * i + 3] = fmaf(gq_hi(c1), d1, nb);
        }
    } else if constexpr (KIND == 2) {
        // block bytes: d at shift+0..1, quants at shift+2..33 (shift 0 or 2)
        const int sh = wl.shift;
        const uint32_t dbits = (sh == 0) ? (wl.w[0] & 0xFFFF) : (wl.w[0] >> 16);
        const float d = f16_to_f32((uint16_t)dbits);
        const float nb = -1152.f * d;  // (1152 + q) * d + nb = q * d
        // quant j = stream byte sh + 2 + j; with sh == 2 quants start at dword 1
        const int w0 = sh == 0 ? 0 : 1;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // 4 quants 4i..4i+3 from the (possibly 2-byte shifted) stream
            const uint32_t lo = wl.w[w0 + i], hi = wl.w[w0 + i + 1];
            const uint32_t u = (sh == 0 ? __builtin_amdgcn_alignbyte(hi, lo, 2) : lo) ^ 0x80808080u;
            const uint32_t c0 = gq_and_or(u, 0x00FF00FFu, magic);
            const uint32_t c1 = gq_and_or(u >> 8, 0x00FF00FFu, magic);
            v[4 * i] = fmaf(gq_lo(c0), d, nb);
            v[4 * i + 1] = fmaf(gq_lo(c1), d, nb);
            v[4 * i + 2] = fmaf(gq_hi(c0), d, nb);
            v[4 * i + 3] = fmaf(gq_hi(c1), d, nb);
        }
    } else {
        wl.decode(v);
    }
    store_f16x32(dst, v);
}


// Skinny-GEMM B operand: 8 weights (values 8 kq .. 8 kq + 7 of sub-block `sub`) of a Q4_K
// row as fp16, from the super-block header hd and the 8 nibble bytes q (low nibbles for an
// even sub-block, high for an odd one): d sc q - dmin m in fp32, rounded to fp16 (zero when
// !ok). Lane layout of v_mfma_f32_16x16x32_f16's B operand.
typedef _Float16 sk_f16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ sk_f16x8 sk_q4k_bfrag(uint4 hd, uint2 q, int sub, bool ok) {
    const uint32_t sc4[3] = {hd.y, hd.z, hd.w};
    auto scb = [&](int i) { return (int)((sc4[i >> 2] >> (8 * (i & 3))) & 0xFF); };
    int scv, mv;
    if (sub < 4) {
        scv = scb(sub) & 63;
        mv = scb(sub + 4) & 63;
    } else {
        scv = (scb(sub + 4) & 0xF) | ((scb(sub - 4) >> 6) << 4);
        mv = (scb(sub + 4) >> 4) | ((scb(sub) >> 6) << 4);
    }
    const float d1 = f16_to_f32((uint16_t)(hd.x & 0xFFFF)) * (float)scv;
    const float m1 = f16_to_f32((uint16_t)(hd.x >> 16)) * (float)mv;
    const int sh = 4 * (sub & 1);
    const uint32_t q2[2] = {q.x, q.y};
    sk_f16x8 bv;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float qq = (float)((q2[i >> 2] >> (8 * (i & 3) + sh)) & 0xF);
        bv[i] = (_Float16)(ok ? d1 * qq - m1 : 0.f);
    }
    return bv;
}
// byte offset, within a Q4_K row, of the 8 nibble bytes of k-step s (32 values) for lane group kq
__device__ __forceinline__ size_t sk_q4k_qofs(int s, int kq) {
    return (size_t)(s >> 3) * 144 + 16 + 32 * ((s & 7) >> 1) + 8 * kq;
}

// Q8_0 B operand of the skinny GEMMs: codes 8 kq .. 8 kq + 7 of a 34-byte block as fp16 q d,
// rounded once (the reference's quant_materialize weight). w[0]: the dword holding the scale
// at byte offset so; w[1..3]: the dwords holding the codes from byte offset co. A code becomes
// the exact fp16 integer 1024 + (q + 128) (0x6400 | byte), minus 1152, times the scale.
__device__ __forceinline__ sk_f16x8 sk_q8_bfrag(const uint32_t* w, int so, int co, bool ok) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const uint32_t c0 = __builtin_amdgcn_alignbyte(w[2], w[1], co), c1 = __builtin_amdgcn_alignbyte(w[3], w[2], co);
    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)((w[0] >> (8 * so)) & 0xFFFF));
    const h2 d2 = {d, d}, off = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t u[2] = {c0 ^ 0x80808080u, c1 ^ 0x80808080u};
    sk_f16x8 bv;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const h2 lo = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u[i], 0x04010400u)) - off;
        const h2 hi = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u[i], 0x04030402u)) - off;
        const h2 a = lo * d2, b = hi * d2;
        bv[4 * i] = ok ? a[0] : (_Float16)0.f;
        bv[4 * i + 1] = ok ? a[1] : (_Float16)0.f;
        bv[4 * i + 2] = ok ? b[0] : (_Float16)0.f;
        bv[4 * i + 3] = ok ? b[1] : (_Float16)0.f;
    }
    return bv;
}

// fp32 -> fp16 copy of n values (n a multiple of 4), on the backend stream
int launch_to_f16(const float* x, uint16_t* y, int64_t n);

}  // namespace gh
