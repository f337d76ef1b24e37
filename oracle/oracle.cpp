// CPU oracle for the quantized Granite-hybrid forward path.
//
// TEST INFRASTRUCTURE ONLY. This file restates, in code of its own, the
// reference engine's CPU path (core/*_cpu.cpp, the CPU branches of
// core/ops.cpp, Generator's host decode path) so that tests can check the
// HIP backend against it. Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load it, and only as the checker.
//
// Build: oracle/Makefile -> oracle/liboracle.so (gcc, -O3 -fopenmp,
// -ffp-contract=off so that no multiply-add is fused behind our back; the
// reference's own x86-64 build has no FMA outside its explicit AVX2 kernels).
//
// Parity status, per function (how each is pinned is in tests/):
//   fp16/bf16 conversions ...... pinned: golden vectors from the compiled
//                                reference + closed-form spot values.
//   Rng normal/uniform/below ... pinned: golden streams from core/rng.h.
//   Q8_0 / Q4_0 / Q4_1 codec ... pinned: golden blocks from
//                                quantization/quantize.cpp + round-trip bound.
//   Q4_K codec ................. NOT in the reference: pinned by hand-built
//                                blocks (closed form) and an error bound only.
//   linear_forward_q4 (0/1/2) .. pinned: golden outputs of ops::linear_forward_q4.
//   linear_forward_q4 (Q4_K) ... pinned through the dequant closed form + the
//                                same serial dot as kinds 0-2.
//   rmsnorm/swiglu/softmax/argmax/embedding ... pinned: golden outputs.
//   topk_select, apply_rep_penalties ........... pinned: golden outputs of
//                                the compiled ops:: CPU functions + numpy
//                                lexsort / per-token counting in tests.
//   attention_forward_ex, attention_decode_ring_fp16 ... pinned: golden.
//   paged bf16 decode .......... pinned: equals the ring kernel on widened
//                                values (test) -- an extension.
//   mamba2_forward (sequential) . pinned: golden ops::mamba2_forward_half.
//   mamba2 step ................ pinned: end-to-end golden greedy ids of the
//                                compiled reference Generator + the
//                                invariant "T steps == sequential scan".
//   moe route / forward ........ pinned: golden ops::moe_forward_bias_half.
//   moe permutation ............ own definition (stable counting sort);
//                                pinned against std::stable_sort in tests.
//   granite generate ........... pinned: golden greedy ids + margins from the
//                                compiled reference Generator.
#include "oracle.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <limits>
#include <map>
#include <string>
#include <vector>

typedef uint8_t u8;
typedef uint16_t u16;
typedef uint32_t u32;
typedef uint64_t u64;
typedef int32_t i32;
typedef int64_t i64;

namespace {

// ---------------------------------------------------------------- formats
// core/dtype.h:61-87 (RNE fp32 -> fp16, NaN keeps a quiet payload bit)
u16 f32_to_f16(float f) {
    u32 x;
    std::memcpy(&x, &f, 4);
    const u32 sign = (x >> 16) & 0x8000u;
    const u32 ebits = (x >> 23) & 0xFFu;
    u32 mant = x & 0x7FFFFFu;
    if (ebits == 0xFFu) return (u16)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    const i32 e = (i32)ebits - 127 + 15;
    if (e >= 31) return (u16)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (u16)sign;
        mant |= 0x800000u;
        const u32 sh = (u32)(14 - e);
        u32 q = mant >> sh;
        const u32 rem = mant & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (u16)(sign | q);
    }
    u16 h = (u16)(sign | ((u32)e << 10) | (mant >> 13));
    const u32 low = mant & 0x1FFFu;
    if (low > 0x1000u || (low == 0x1000u && (h & 1u))) ++h;
    return h;
}

// core/dtype.h:89-111
float f16_to_f32(u16 h) {
    const u32 sign = (u32)(h & 0x8000u) << 16;
    u32 e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, out;
    if (e == 0) {
        if (m == 0) out = sign;
        else {
            int shift = -1;
            do { m <<= 1; ++shift; } while (!(m & 0x400u));
            out = sign | ((u32)(127 - 15 - shift) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 0x1F) out = sign | 0x7F800000u | (m << 13);
    else out = sign | ((e + 112u) << 23) | (m << 13);
    float f;
    std::memcpy(&f, &out, 4);
    return f;
}

// core/dtype.h:113-126
u16 f32_to_bf16(float f) {
    u32 x;
    std::memcpy(&x, &f, 4);
    if (((x >> 23) & 0xFF) == 0xFF) return (u16)(x >> 16);
    return (u16)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}
float bf16_to_f32(u16 b) {
    u32 x = (u32)b << 16;
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

inline u16 rd16(const u8* p) { u16 v; std::memcpy(&v, p, 2); return v; }

// ------------------------------------------------------------------- rng
// core/rng.h:8-92: splitmix-seeded xoshiro256**, Marsaglia polar normal.
struct Xoshiro {
    u64 s[4];
    bool has_spare = false;
    float spare = 0.f;
    explicit Xoshiro(u64 seed) {
        for (int i = 0; i < 4; ++i) {
            seed += 0x9E3779B97F4A7C15ULL;
            u64 z = seed;
            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
            z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
            s[i] = z ^ (z >> 31);
        }
    }
    static u64 rotl(u64 v, int k) { return (v << k) | (v >> (64 - k)); }
    u64 next() {
        const u64 r = rotl(s[1] * 5, 7) * 9, t = s[1] << 17;
        s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3];
        s[2] ^= t; s[3] = rotl(s[3], 45);
        return r;
    }
    float uni() { return (float)((next() >> 40) * (1.0 / 16777216.0)); }
    u64 below(u64 n) {
        const u64 t = (0u - n) % n;
        u64 v;
        do { v = next(); } while (v < t);
        return v % n;
    }
    float normal(float mean, float sd) {
        if (has_spare) { has_spare = false; return mean + sd * spare; }
        float u, v, q;
        do {
            u = uni() * 2.0f - 1.0f;
            v = uni() * 2.0f - 1.0f;
            q = u * u + v * v;
        } while (q >= 1.0f || q == 0.0f);
        const float m = std::sqrt(-2.0f * std::log(q) / q);
        spare = v * m;
        has_spare = true;
        return mean + sd * (u * m);
    }
};

// ------------------------------------------------------------- dot kernels
// core/simd_cpu.h:30-51 (AVX2 path, taken for n >= 32 on an AVX2+FMA host):
// four 8-lane FMA accumulators over 32-wide strides, lane-wise combine
// (s0+s1)+(s2+s3), fold the two 128-bit halves, then movehl + shuffle, then
// a scalar tail. core/simd_cpu.h:84-99 is the scalar 4-way path for n < 32.
// (std::fma is compiled to the FMA3 instruction here, as in the reference's
// AVX2 kernel; the result is exactly rounded either way.)
__attribute__((target("avx2,fma"))) float dot_f32(const float* a, const float* b, int n) {
    if (n >= 32) {
        float acc[4][8] = {};
        const int n32 = n & ~31;
        for (int i = 0; i < n32; i += 32)
            for (int r = 0; r < 4; ++r)
                for (int l = 0; l < 8; ++l)
                    acc[r][l] = std::fma(a[i + 8 * r + l], b[i + 8 * r + l], acc[r][l]);
        float s[8];
        for (int l = 0; l < 8; ++l) s[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
        float h[4];
        for (int l = 0; l < 4; ++l) h[l] = s[l] + s[l + 4];
        const float h0 = h[0] + h[2], h1 = h[1] + h[3];
        float out = h0 + h1;
        for (int i = n32; i < n; ++i) out += a[i] * b[i];
        return out;
    }
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    int i = 0;
    for (; i + 4 <= n; i += 4) {
        s0 += a[i] * b[i];
        s1 += a[i + 1] * b[i + 1];
        s2 += a[i + 2] * b[i + 2];
        s3 += a[i + 3] * b[i + 3];
    }
    float s = s0 + s1 + s2 + s3;
    for (; i < n; ++i) s += a[i] * b[i];
    return s;
}

// core/simd_cpu.h:53-75 and :101-117 (y += a*x)
__attribute__((target("avx2,fma"))) void axpy_f32(float* y, const float* x, float a, int n) {
    int i = 0;
    if (n >= 32) {
        const int n32 = n & ~31;
        for (; i < n32; ++i) y[i] = std::fma(a, x[i], y[i]);
        for (; i < n; ++i) y[i] += a * x[i];
        return;
    }
    for (; i < n; ++i) y[i] += a * x[i];
}

// core/moe_cpu.cpp:76-83: the router dot, 4 products grouped left to right.
float dot_row(const float* a, const float* b, int n) {
    float s = 0.0f;
    int i = 0;
    for (; i + 4 <= n; i += 4)
        s += a[i] * b[i] + a[i + 1] * b[i + 1] + a[i + 2] * b[i + 2] + a[i + 3] * b[i + 3];
    for (; i < n; ++i) s += a[i] * b[i];
    return s;
}

// -------------------------------------------------------------- codecs
int block_values(int kind) { return kind == 3 ? 256 : 32; }
int block_bytes(int kind) {
    switch (kind) { case 0: return 18; case 1: return 20; case 2: return 34; case 3: return 144; }
    return -1;
}

// quantization/quantize.cpp:58-112
void quant_q8_0_block(const float* x, int cnt, u8* blk) {
    bool bad = false;
    float amax = 0.0f;
    for (int i = 0; i < cnt; ++i) {
        if (!std::isfinite(x[i])) { bad = true; break; }
        amax = std::max(amax, std::fabs(x[i]));
    }
    std::memset(blk, 0, 34);
    if (bad) return;  // fp16(0) scale, zero quants
    const float scale = amax / 127.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    const u16 hs = f32_to_f16(scale);
    std::memcpy(blk, &hs, 2);
    for (int i = 0; i < cnt; ++i) {
        int q = (int)std::lround(x[i] * inv);
        q = std::min(127, std::max(-127, q));
        blk[2 + i] = (u8)(int8_t)q;
    }
}

// quantization/quantize.cpp:114-133 (block 32 values x f16 scale)
float deq_one(int kind, const u8* blk, int j) {
    switch (kind) {
        case 0: {  // core/ops.cpp:312-317
            const float sc = f16_to_f32(rd16(blk));
            const u8 b = blk[2 + (j & 15)];
            const int q = (j < 16) ? (b & 0x0F) : (b >> 4);
            return (float)(q - 8) * sc;
        }
        case 1: {  // core/ops.cpp:318-324
            const float sc = f16_to_f32(rd16(blk)), mn = f16_to_f32(rd16(blk + 2));
            const u8 b = blk[4 + (j & 15)];
            const int q = (j < 16) ? (b & 0x0F) : (b >> 4);
            return (float)q * sc + mn;
        }
        case 2:  // core/ops.cpp:325-328
            return (float)((const int8_t*)(blk + 2))[j] * f16_to_f32(rd16(blk));
        case 3: {
            // Q4_K, GGML block_q4_K layout (NOT in the reference):
            //   f16 d | f16 dmin | u8 scales[12] | u8 qs[128]
            // sub-block s (32 values) has a 6-bit scale sc_s and min m_s;
            // value = (d*sc_s)*q - (dmin*m_s), q a nibble. Bytes 32i..32i+31
            // of qs hold sub-block 2i (low nibbles) and 2i+1 (high nibbles).
            const float d = f16_to_f32(rd16(blk)), dmin = f16_to_f32(rd16(blk + 2));
            const u8* sc = blk + 4;
            const u8* qs = blk + 16;
            const int s = j >> 5, l = j & 31;
            int scv, mv;
            if (s < 4) { scv = sc[s] & 63; mv = sc[s + 4] & 63; }
            else {
                scv = (sc[s + 4] & 0xF) | ((sc[s - 4] >> 6) << 4);
                mv = (sc[s + 4] >> 4) | ((sc[s] >> 6) << 4);
            }
            const u8 byte = qs[32 * (s >> 1) + l];
            const int q = (s & 1) ? (byte >> 4) : (byte & 0xF);
            const float d1 = d * (float)scv, m1 = dmin * (float)mv;
            return d1 * (float)q - m1;
        }
    }
    return 0.f;
}

// Q4_K quantizer (our own; the reference has none). Per sub-block s:
// lo = min(0, min x), hi = max x, scale_s = (hi-lo)/15, min_s = -lo. The
// super-block d = max scale/63 and dmin = max min/63 are stored as fp16;
// the 6-bit sc_s / m_s and the nibbles are rounded against the fp16-rounded
// d and dmin (lround, clamped). A block holding a non-finite value is zero.
void quant_q4_k_block(const float* x, u8* blk) {
    std::memset(blk, 0, 144);
    for (int i = 0; i < 256; ++i) if (!std::isfinite(x[i])) return;
    float scl[8], mn[8], maxs = 0.f, maxm = 0.f;
    for (int s = 0; s < 8; ++s) {
        float lo = 0.f, hi = x[32 * s];
        for (int l = 0; l < 32; ++l) { lo = std::min(lo, x[32 * s + l]); hi = std::max(hi, x[32 * s + l]); }
        scl[s] = (hi - lo) / 15.0f;
        mn[s] = -lo;
        maxs = std::max(maxs, scl[s]);
        maxm = std::max(maxm, mn[s]);
    }
    const u16 hd = f32_to_f16(maxs / 63.0f), hm = f32_to_f16(maxm / 63.0f);
    std::memcpy(blk, &hd, 2);
    std::memcpy(blk + 2, &hm, 2);
    const float d = f16_to_f32(hd), dmin = f16_to_f32(hm);
    int sc[8], m[8];
    for (int s = 0; s < 8; ++s) {
        sc[s] = d > 0.f ? std::min(63, std::max(0, (int)std::lround(scl[s] / d))) : 0;
        m[s] = dmin > 0.f ? std::min(63, std::max(0, (int)std::lround(mn[s] / dmin))) : 0;
    }
    u8* S = blk + 4;
    for (int s = 0; s < 4; ++s) {
        S[s] = (u8)(sc[s] | ((sc[s + 4] >> 4) << 6));
        S[s + 4] = (u8)(m[s] | ((m[s + 4] >> 4) << 6));
        S[s + 8] = (u8)((sc[s + 4] & 0xF) | ((m[s + 4] & 0xF) << 4));
    }
    u8* qs = blk + 16;
    for (int s = 0; s < 8; ++s) {
        const float d1 = d * (float)sc[s], m1 = dmin * (float)m[s];
        for (int l = 0; l < 32; ++l) {
            int q = 0;
            if (d1 > 0.f) q = std::min(15, std::max(0, (int)std::lround((x[32 * s + l] + m1) / d1)));
            qs[32 * (s >> 1) + l] |= (u8)((s & 1) ? (q << 4) : q);
        }
    }
}

// quantization/quantize.cpp:135-156 (Q4_0) and :183-220 (Q4_1), full blocks
void quant_q4_0_block(const float* x, u8* blk) {
    bool bad = false;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        if (!std::isfinite(x[i])) { bad = true; break; }
        amax = std::max(amax, std::fabs(x[i]));
    }
    std::memset(blk, 0, 18);
    if (bad) { std::memset(blk + 2, 0x88, 16); return; }
    const float scale = amax / 8.0f, inv = scale > 0.f ? 1.0f / scale : 0.f;
    const u16 hs = f32_to_f16(scale);
    std::memcpy(blk, &hs, 2);
    for (int j = 0; j < 16; ++j) {
        const int q0 = std::min(7, std::max(-8, (int)std::lround(x[j] * inv))) + 8;
        const int q1 = std::min(7, std::max(-8, (int)std::lround(x[j + 16] * inv))) + 8;
        blk[2 + j] = (u8)((q1 << 4) | q0);
    }
}
void quant_q4_1_block(const float* x, u8* blk) {
    std::memset(blk, 0, 20);
    for (int i = 0; i < 32; ++i) if (!std::isfinite(x[i])) return;
    float mn = x[0], mx = x[0];
    for (int i = 1; i < 32; ++i) { mn = std::min(mn, x[i]); mx = std::max(mx, x[i]); }
    const float scale = (mx - mn) / 15.0f, inv = scale > 0.f ? 1.0f / scale : 0.f;
    const u16 hs = f32_to_f16(scale), hm = f32_to_f16(mn);
    std::memcpy(blk, &hs, 2);
    std::memcpy(blk + 2, &hm, 2);
    for (int i = 0; i < 16; ++i) {
        const int q0 = std::min(15, std::max(0, (int)std::lround((x[i] - mn) * inv)));
        const int q1 = std::min(15, std::max(0, (int)std::lround((x[i + 16] - mn) * inv)));
        blk[4 + i] = (u8)((q1 << 4) | q0);
    }
}

// core/ops.cpp:304-337 generalised to Q4_K: dequantise value i to fp16.
void materialize(int kind, const void* packed, u16* dst, i64 n) {
    const u8* p = (const u8*)packed;
    const int bv = block_values(kind), bb = block_bytes(kind);
    for (i64 i = 0; i < n; ++i)
        dst[i] = f32_to_f16(deq_one(kind, p + (i / bv) * bb, (int)(i % bv)));
}

// core/ops.cpp:360-401: per output row n, dequantise the row to fp16, then a
// serial fp32 dot for every m.
void linear_q(const float* x, const void* w, float* y, int M, int K, int N, int kind) {
    const u8* p = (const u8*)w;
    const int bv = block_values(kind), bb = block_bytes(kind);
    const size_t row_bytes = (size_t)(K / bv) * bb;
    std::vector<float> row((size_t)K);
    for (int n = 0; n < N; ++n) {
        const u8* wr = p + (size_t)n * row_bytes;
        for (int k = 0; k < K; ++k) row[(size_t)k] = f16_to_f32(f32_to_f16(deq_one(kind, wr + (size_t)(k / bv) * bb, k % bv)));
        for (int m = 0; m < M; ++m) {
            const float* xa = x + (size_t)m * K;
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) acc += xa[k] * row[(size_t)k];
            y[(size_t)m * N + n] = acc;
        }
    }
}

// core/math_cpu.cpp:121-134
void linear_fp16(const float* x, const u16* w, float* y, int M, int K, int N) {
#pragma omp parallel for if (M * N > 256) schedule(static)
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float s = 0.0f;
            const u16* r = w + (size_t)n * K;
            const float* xr = x + (size_t)m * K;
            for (int k = 0; k < K; ++k) s += xr[k] * f16_to_f32(r[k]);
            y[(size_t)m * N + n] = s;
        }
}

// core/math_cpu.cpp:20-119: y = x W^T, each output one dot_f32 (beta = 0, so
// C = 0 + 1*dot).
void linear_f32(const float* x, const float* w, float* y, int M, int K, int N) {
#pragma omp parallel for if (N > 64) schedule(static)
    for (int n = 0; n < N; ++n)
        for (int m = 0; m < M; ++m) y[(size_t)m * N + n] = dot_f32(x + (size_t)m * K, w + (size_t)n * K, K);
}

// core/math_cpu.cpp:299-316
void rmsnorm(const float* x, const float* w, float* out, float* rrms, i64 rows, int dim, float eps) {
    for (i64 r = 0; r < rows; ++r) {
        const float* xr = x + r * dim;
        double ss = 0.0;
        for (int i = 0; i < dim; ++i) ss += (double)xr[i] * xr[i];
        const double invd = 1.0 / std::sqrt(ss / (double)dim + (double)eps);
        const float inv = std::isfinite(invd) ? (float)invd : 0.0f;
        if (rrms) rrms[r] = inv;
        float* o = out + r * dim;
        for (int i = 0; i < dim; ++i) o[i] = xr[i] * inv * w[i];
    }
}

inline float silu(float v) { return v / (1.0f + std::exp(-v)); }

// core/math_cpu.cpp:546-558
void softmax_row(float* x, int n) {
    if (n <= 0 || !x) return;
    float mx = x[0];
    for (int i = 1; i < n; ++i) mx = std::max(mx, x[i]);
    float sum = 0.f;
    for (int i = 0; i < n; ++i) { x[i] = std::exp(x[i] - mx); sum += x[i]; }
    const float inv = (sum > 1e-12f) ? (1.0f / sum) : 0.0f;
    for (int i = 0; i < n; ++i) x[i] *= inv;
}

// core/math_cpu.cpp:710-723
// core/math_cpu.cpp:695-707: the K largest logits, larger value first, lower
// index first among equal values (here: a full sort by that key, then the
// first K, which is the same set and order for any input without NaN).
void topk_select(const float* l, int V, int K, float* vals, i32* ids) {
    std::vector<int> order((size_t)V);
    for (int i = 0; i < V; ++i) order[(size_t)i] = i;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return l[a] > l[b]; });
    for (int k = 0; k < K; ++k) {
        ids[k] = order[(size_t)k];
        vals[k] = l[order[(size_t)k]];
    }
}

// core/math_cpu.cpp:725-752: every distinct in-range token of the history, seen
// n times, gets the repetition transform once (divide positive logits by rep,
// multiply the others), then minus freq * n, then minus pres. Counting here is
// a dense per-token table rather than a sort.
void apply_rep_penalties(float* l, int V, const i32* hist, int n, float rep, float freq, float pres) {
    if (n <= 0 || V <= 0) return;
    const bool use_rep = rep > 0.0f && rep != 1.0f, use_freq = freq != 0.0f, use_pres = pres != 0.0f;
    if (!use_rep && !use_freq && !use_pres) return;
    std::vector<int> cnt((size_t)V, 0);
    for (int i = 0; i < n; ++i)
        if (hist[i] >= 0 && hist[i] < V) ++cnt[(size_t)hist[i]];
    for (int t = 0; t < V; ++t) {
        const int c = cnt[(size_t)t];
        if (!c) continue;
        float v = l[t];
        if (use_rep) v = v > 0.0f ? v / rep : v * rep;
        if (use_freq) v -= freq * (float)c;
        if (use_pres) v -= pres;
        l[t] = v;
    }
}

i32 argmax(const float* l, int V) {
    int best = -1;
    float bv = -std::numeric_limits<float>::infinity();
    for (int i = 0; i < V; ++i)
        if (std::isfinite(l[i]) && (best < 0 || l[i] > bv)) { bv = l[i]; best = i; }
    if (best < 0) {
        best = 0;
        for (int i = 1; i < V; ++i) if (l[i] > l[best]) best = i;
    }
    return best;
}

// core/attn_cpu.cpp:151-156
size_t ring_slot(int j, int pinned, int ring_start, int cap) {
    if (j < pinned) return (size_t)j;
    const int c = cap > 0 ? cap : 1;
    return (size_t)pinned + (size_t)((ring_start + (j - pinned)) % c);
}

// core/attn_cpu.cpp:207-254, with a caller-chosen widening of the cache value.
template <typename Widen>
void decode_ring(const float* q, const u16* kc, const u16* vc, float* out, int H, int KV, int hd,
                 int ring_start, int pinned, int cur_len, int cache_max, float scale, int window,
                 Widen widen) {
    const int cap = cache_max - pinned, group = H / KV;
    std::vector<float> s((size_t)std::max(cur_len, 1));
    for (int h = 0; h < H; ++h) {
        const int kvh = h / group;
        const float* qh = q + (size_t)h * hd;
        const int j0 = (window > 0 && cur_len > window) ? cur_len - window : 0;
        float mx = -3.4e38f;
        for (int j = j0; j < cur_len; ++j) {
            const u16* kh = kc + (ring_slot(j, pinned, ring_start, cap) * KV + kvh) * hd;
            float d = 0.0f;
            for (int c = 0; c < hd; ++c) d += qh[c] * widen(kh[c]);
            d *= scale;
            s[(size_t)j] = d;
            mx = std::max(mx, d);
        }
        float sum = 0.f;
        for (int j = j0; j < cur_len; ++j) { s[(size_t)j] = std::exp(s[(size_t)j] - mx); sum += s[(size_t)j]; }
        const float inv = sum > 0.f ? 1.0f / sum : 0.0f;
        float* o = out + (size_t)h * hd;
        std::memset(o, 0, sizeof(float) * hd);
        for (int j = j0; j < cur_len; ++j) {
            const u16* vh = vc + (ring_slot(j, pinned, ring_start, cap) * KV + kvh) * hd;
            const float w = s[(size_t)j] * inv;
            for (int c = 0; c < hd; ++c) o[c] += w * widen(vh[c]);
        }
    }
}

// core/attn_cpu.cpp:29-94 (no segment mask, probs not kept)
void attn_prefill(const float* q, const float* k, const float* v, float* out, int B, int T, int H,
                  int KV, int hd, float scale, int window) {
    const int group = H / KV;
    const size_t qs = (size_t)T * H * hd, kvs = (size_t)T * KV * hd;
#pragma omp parallel
    {
        std::vector<float> s((size_t)T);
#pragma omp for schedule(static)
        for (int bh = 0; bh < B * H; ++bh) {
            const int b = bh / H, h = bh % H, kvh = h / group;
            for (int t = 0; t < T; ++t) {
                const float* qh = q + b * qs + ((size_t)t * H + h) * hd;
                const int j0 = (window > 0) ? std::max(t - window + 1, 0) : 0;
                const int len = t + 1 - j0;
                float mx = -3.4e38f;
                for (int j = j0; j <= t; ++j) {
                    const float d = dot_f32(qh, k + b * kvs + ((size_t)j * KV + kvh) * hd, hd) * scale;
                    s[(size_t)(j - j0)] = d;
                    mx = std::max(mx, d);
                }
                float sum = 0.f;
                for (int j = 0; j < len; ++j) {
                    float val = s[(size_t)j];
                    val = val < -3.0e38f ? 0.0f : std::exp(val - mx);
                    s[(size_t)j] = val;
                    sum += val;
                }
                const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
                float* o = out + b * qs + ((size_t)t * H + h) * hd;
                std::memset(o, 0, sizeof(float) * hd);
                for (int j = 0; j < len; ++j)
                    axpy_f32(o, v + b * kvs + ((size_t)(j + j0) * KV + kvh) * hd, s[(size_t)j] * inv, hd);
            }
        }
    }
}

// core/moe_cpu.cpp:85-100: K rounds of strict '>' argmax, lowest index wins.
void topk_pick(const float* p, int ne, int K, i32* idx, float* w) {
    for (int k = 0; k < K; ++k) {
        int best = -1;
        float bv = -1e30f;
        for (int e = 0; e < ne; ++e) {
            bool taken = false;
            for (int j = 0; j < k; ++j) if (idx[j] == e) { taken = true; break; }
            if (!taken && p[e] > bv) { bv = p[e]; best = e; }
        }
        if (best < 0) best = 0;
        idx[k] = best;
        w[k] = p[best];
    }
}

// core/moe_cpu.cpp:218-256 for one token: router dot_row, softmax, select on
// p + bias, weights from the unbiased p, renormalised (uniform if tiny).
void route_one(const float* xt, const float* rw, const float* bias, int d, int ne, int K,
               float* probs, i32* idx, float* w) {
    for (int e = 0; e < ne; ++e) probs[e] = dot_row(xt, rw + (size_t)e * d, d);
    softmax_row(probs, ne);
    std::vector<float> sel((size_t)ne);
    for (int e = 0; e < ne; ++e) sel[(size_t)e] = probs[e] + (bias ? bias[e] : 0.0f);
    float tsel[8];
    topk_pick(sel.data(), ne, K, idx, tsel);
    float sum = 0.f;
    for (int k = 0; k < K; ++k) { w[k] = probs[idx[k]]; sum += w[k]; }
    if (sum > 1e-8f) {
        const float inv = 1.0f / sum;
        for (int k = 0; k < K; ++k) w[k] *= inv;
    } else {
        for (int k = 0; k < K; ++k) w[k] = 1.0f / (float)K;
    }
}

// core/moe_cpu.cpp:198-288 on fp32 weights (the _half path widens fp16 to
// fp32 first, core/moe_cpu.cpp:290-316). gates/ups [ne*E, d], downs [ne*d, E].
void moe_fwd_f32(const float* x, const float* rw, const float* bias, const float* g, const float* u,
                 const float* dn, const float* sg, const float* su, const float* sd, float* out,
                 i32* idx_out, float* w_out, i64 N, int d, int E, int ne, int K, int SH) {
#pragma omp parallel if (N > 4)
    {
        std::vector<float> probs((size_t)ne), a((size_t)std::max(E, SH)), b((size_t)std::max(E, SH)),
            c((size_t)std::max(E, SH)), tmp((size_t)d);
#pragma omp for schedule(static)
        for (i64 t = 0; t < N; ++t) {
            const float* xt = x + t * d;
            float* ot = out + t * d;
            i32 idx[8];
            float w[8];
            route_one(xt, rw, bias, d, ne, K, probs.data(), idx, w);
            if (idx_out) std::memcpy(idx_out + t * K, idx, sizeof(i32) * K);
            if (w_out) std::memcpy(w_out + t * K, w, sizeof(float) * K);
            if (sg && su && sd) {
                linear_f32(xt, sg, a.data(), 1, d, SH);
                linear_f32(xt, su, b.data(), 1, d, SH);
                for (int i = 0; i < SH; ++i) c[(size_t)i] = silu(a[(size_t)i]) * b[(size_t)i];
                linear_f32(c.data(), sd, ot, 1, SH, d);
            } else {
                std::fill(ot, ot + d, 0.0f);
            }
            for (int k = 0; k < K; ++k) {
                const int e = idx[k];
                linear_f32(xt, g + (size_t)e * E * d, a.data(), 1, d, E);
                linear_f32(xt, u + (size_t)e * E * d, b.data(), 1, d, E);
                for (int i = 0; i < E; ++i) c[(size_t)i] = silu(a[(size_t)i]) * b[(size_t)i];
                linear_f32(c.data(), dn + (size_t)e * d * E, tmp.data(), 1, E, d);
                for (int j = 0; j < d; ++j) ot[j] += w[k] * tmp[(size_t)j];
            }
        }
    }
}

std::vector<float> widen_q(const void* w, int qkind, i64 n) {
    // core/ops.cpp:950-958 then core/moe_cpu.cpp:300-305: packed -> fp16 -> fp32
    std::vector<u16> h((size_t)n);
    if (qkind >= 0) materialize(qkind, w, h.data(), n);
    else std::memcpy(h.data(), w, (size_t)n * 2);
    std::vector<float> f((size_t)n);
    for (i64 i = 0; i < n; ++i) f[(size_t)i] = f16_to_f32(h[(size_t)i]);
    return f;
}

// Generator::decode_mamba_layer host branch, inference/generator.cpp:510-616
// (in_proj / out_proj through ops::linear_forward_q4 on the CPU).
void mamba_step(const float* x, const void* w_in, const float* conv_w, const float* conv_b,
                const float* dt_bias, const float* a_log, const float* D, const float* norm_w,
                const void* w_out, float* conv_state, float* ssm, float* out, int d, int d_inner,
                int conv_dim, int n_heads, int d_head, int d_state, int conv_k, float eps,
                int qkind) {
    const int proj = d_inner + conv_dim + n_heads;
    const int win = conv_k > 1 ? conv_k - 1 : 1;
    std::vector<float> pr((size_t)proj), bco((size_t)conv_dim), y((size_t)d_inner), nrm((size_t)d_inner);
    if (qkind >= 0) linear_q(x, w_in, pr.data(), 1, d, proj, qkind);
    else linear_fp16(x, (const u16*)w_in, pr.data(), 1, d, proj);
    const float* gate = pr.data();
    const float* bc = gate + d_inner;
    const float* dtr = bc + conv_dim;
    for (int ch = 0; ch < conv_dim; ++ch) {
        float acc = conv_b ? conv_b[ch] : 0.0f;
        const float* wc = conv_w + (size_t)ch * conv_k;
        for (int j = 0; j < conv_k; ++j)
            acc += wc[j] * ((j == conv_k - 1) ? bc[ch] : conv_state[(size_t)ch * win + j]);
        bco[(size_t)ch] = acc / (1.0f + std::exp(-acc));
    }
    for (int ch = 0; ch < conv_dim; ++ch) {
        for (int j = 0; j + 1 < win; ++j) conv_state[(size_t)ch * win + j] = conv_state[(size_t)ch * win + j + 1];
        conv_state[(size_t)ch * win + (win - 1)] = bc[ch];
    }
    const float* xs = bco.data();
    const float* Bm = xs + d_inner;
    const float* Cm = Bm + d_state;  // n_groups == 1
    for (int h = 0; h < n_heads; ++h) {
        const float a = -std::exp(a_log[h]);
        const float dtb = dtr[h] + dt_bias[h];
        const float dt = (dtb > 20.0f) ? dtb : std::log1p(std::exp(dtb));
        const float dA = std::exp(a * dt);
        for (int p = 0; p < d_head; ++p) {
            const int i = h * d_head + p;
            const float xv = xs[i];
            float* srow = ssm + (size_t)i * d_state;
            float acc = 0.0f;
            for (int j = 0; j < d_state; ++j) {
                srow[j] = dA * srow[j] + (Bm[j] * dt) * xv;
                acc += Cm[j] * srow[j];
            }
            y[(size_t)i] = acc + D[h] * xv;
        }
    }
    double var = 0.0;
    for (int i = 0; i < d_inner; ++i) {
        const float g = gate[i] / (1.0f + std::exp(-gate[i]));
        nrm[(size_t)i] = y[(size_t)i] * g;
        var += (double)nrm[(size_t)i] * (double)nrm[(size_t)i];
    }
    var /= (double)d_inner;
    const float inv = 1.0f / std::sqrt((float)var + eps);
    for (int i = 0; i < d_inner; ++i) nrm[(size_t)i] = nrm[(size_t)i] * inv * norm_w[i];
    if (qkind >= 0) linear_q(nrm.data(), w_out, out, 1, d_inner, d, qkind);
    else linear_fp16(nrm.data(), (const u16*)w_out, out, 1, d_inner, d);
}

}  // namespace

// ======================================================================= C ABI
extern "C" {

void orc_f32_to_f16(const float* s, uint16_t* d, int64_t n) { for (i64 i = 0; i < n; ++i) d[i] = f32_to_f16(s[i]); }
void orc_f16_to_f32(const uint16_t* s, float* d, int64_t n) { for (i64 i = 0; i < n; ++i) d[i] = f16_to_f32(s[i]); }
void orc_f32_to_bf16(const float* s, uint16_t* d, int64_t n) { for (i64 i = 0; i < n; ++i) d[i] = f32_to_bf16(s[i]); }
void orc_bf16_to_f32(const uint16_t* s, float* d, int64_t n) { for (i64 i = 0; i < n; ++i) d[i] = bf16_to_f32(s[i]); }

void orc_rng_normal(uint64_t seed, float mean, float sd, float* out, int64_t n) {
    Xoshiro r(seed);
    for (i64 i = 0; i < n; ++i) out[i] = r.normal(mean, sd);
}
void orc_rng_uniform(uint64_t seed, float lo, float hi, float* out, int64_t n) {
    Xoshiro r(seed);
    for (i64 i = 0; i < n; ++i) out[i] = lo + (hi - lo) * r.uni();
}
void orc_rng_below(uint64_t seed, uint64_t bound, int32_t* out, int64_t n) {
    Xoshiro r(seed);
    for (i64 i = 0; i < n; ++i) out[i] = (i32)r.below(bound);
}
// core/rng.h:94-101
uint64_t orc_fnv1a64(const void* data, int64_t n) {
    const u8* p = (const u8*)data;
    u64 h = 1469598103934665603ULL;
    for (i64 i = 0; i < n; ++i) { h ^= p[i]; h *= 1099511628211ULL; }
    return h;
}

int64_t orc_quant_row_bytes(int kind, int64_t k) {
    if (kind < 0 || kind > 3 || k % block_values(kind)) return -1;
    return k / block_values(kind) * block_bytes(kind);
}

int orc_quantize(int kind, const float* src, void* dst, int64_t n) {
    u8* o = (u8*)dst;
    if (kind == 2) {  // Q8_0 keeps the reference's partial-block tail
        const i64 full = n / 32;
        for (i64 b = 0; b < full; ++b) quant_q8_0_block(src + b * 32, 32, o + b * 34);
        if (n % 32) quant_q8_0_block(src + full * 32, (int)(n % 32), o + full * 34);
        return 0;
    }
    if (kind < 0 || kind > 3 || n % block_values(kind)) return -1;
    const int bv = block_values(kind), bb = block_bytes(kind);
    for (i64 b = 0; b < n / bv; ++b) {
        if (kind == 0) quant_q4_0_block(src + b * bv, o + b * bb);
        else if (kind == 1) quant_q4_1_block(src + b * bv, o + b * bb);
        else quant_q4_k_block(src + b * bv, o + b * bb);
    }
    return 0;
}

int orc_dequantize(int kind, const void* src, float* dst, int64_t n) {
    if (kind < 0 || kind > 3) return -1;
    const u8* p = (const u8*)src;
    const int bv = block_values(kind), bb = block_bytes(kind);
    for (i64 i = 0; i < n; ++i) dst[i] = deq_one(kind, p + (i / bv) * bb, (int)(i % bv));
    return 0;
}

int orc_quant_materialize(int kind, const void* packed, uint16_t* dst, int64_t n) {
    if (kind < 0 || kind > 3) return -1;
    materialize(kind, packed, dst, n);
    return 0;
}

int orc_linear_forward_q4(const float* x, const void* w, float* y, int M, int K, int N, int kind) {
    if (kind < 0 || kind > 3 || K % block_values(kind)) return -1;
    if (M <= 0 || N <= 0) return 0;
    linear_q(x, w, y, M, K, N, kind);
    return 0;
}
void orc_linear_forward_fp16(const float* x, const uint16_t* w, float* y, int M, int K, int N) { linear_fp16(x, w, y, M, K, N); }
void orc_linear_forward_f32(const float* x, const float* w, float* y, int M, int K, int N) { linear_f32(x, w, y, M, K, N); }
float orc_dot_f32(const float* a, const float* b, int n) { return dot_f32(a, b, n); }

void orc_rmsnorm_forward(const float* x, const float* w, float* out, float* rrms, int64_t rows, int dim, float eps) {
    rmsnorm(x, w, out, rrms, rows, dim, eps);
}
// core/math_cpu.cpp:522-529
void orc_swiglu_forward(const float* g, const float* u, float* out, int64_t n) {
    for (i64 i = 0; i < n; ++i) out[i] = silu(g[i]) * u[i];
}
void orc_softmax_row(float* x, int n) { softmax_row(x, n); }
int32_t orc_argmax_token(const float* l, int V) { return argmax(l, V); }
int orc_topk_select(const float* l, int V, int K, float* vals, int32_t* ids) {
    if (V <= 0 || K < 1 || K > V) return 1;
    topk_select(l, V, K, vals, ids);
    return 0;
}
void orc_apply_rep_penalties(float* l, int V, const int32_t* hist, int n, float rep, float freq, float pres) {
    apply_rep_penalties(l, V, hist, n, rep, freq, pres);
}
// core/math_cpu.cpp:227-241
void orc_embedding_forward_half(const int32_t* ids, const uint16_t* table, float* out, int64_t ntok, int dim, int vocab) {
    for (i64 t = 0; t < ntok; ++t) {
        float* o = out + t * dim;
        const i32 id = ids[t];
        if (id < 0 || id >= vocab) { std::memset(o, 0, sizeof(float) * dim); continue; }
        for (int i = 0; i < dim; ++i) o[i] = f16_to_f32(table[(size_t)id * dim + i]);
    }
}

void orc_attention_forward_ex(const float* q, const float* k, const float* v, float* out, int B, int T, int H, int KV,
                              int hd, float scale, int window) {
    attn_prefill(q, k, v, out, B, T, H, KV, hd, scale, window);
}

int orc_attention_decode_ring_fp16(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int H, int KV,
                                   int hd, int ring_start, int pinned, int cur_len, int cache_max, float scale,
                                   int window) {
    // core/attn_cpu.cpp:211-222 argument checks
    if (H <= 0 || KV <= 0 || hd <= 0 || H % KV) return -1;
    if (cur_len < 0 || cache_max < 0 || cur_len > cache_max) return -1;
    if (pinned < 0 || pinned > cur_len) return -1;
    const int cap = cache_max - pinned;
    if (cur_len > pinned && (cap <= 0 || ring_start < 0 || ring_start >= cap)) return -1;
    decode_ring(q, kc, vc, out, H, KV, hd, ring_start, pinned, cur_len, cache_max, scale, window,
                [](u16 h) { return f16_to_f32(h); });
    return 0;
}

int orc_attention_decode_paged_bf16(const float* q, const uint16_t* kp, const uint16_t* vp, const int32_t* pt,
                                    const int32_t* lens, int n_seqs, int max_pages, int page_size, float* out,
                                    int H, int KV, int hd, float scale) {
    if (H <= 0 || KV <= 0 || hd <= 0 || H % KV || page_size <= 0) return -1;
    for (int b = 0; b < n_seqs; ++b) {
        const int L = lens[b];
        if (L < 0 || L > max_pages * page_size) return -1;
        // gather the logical sequence into a contiguous cache, then the ring
        // kernel with no pinned prefix and ring_start 0 (slot j = j)
        std::vector<u16> kc((size_t)std::max(L, 1) * KV * hd), vc(kc.size());
        for (int j = 0; j < L; ++j) {
            const size_t src = ((size_t)pt[(size_t)b * max_pages + j / page_size] * page_size + j % page_size) * KV * hd;
            std::memcpy(&kc[(size_t)j * KV * hd], kp + src, sizeof(u16) * KV * hd);
            std::memcpy(&vc[(size_t)j * KV * hd], vp + src, sizeof(u16) * KV * hd);
        }
        decode_ring(q + (size_t)b * H * hd, kc.data(), vc.data(), out + (size_t)b * H * hd, H, KV, hd, 0, 0, L,
                    std::max(L, 1), scale, 0, [](u16 h) { return bf16_to_f32(h); });
    }
    return 0;
}

// core/mamba_cpu.cpp:120-170 restricted to its arithmetic: xs [T, H*P],
// Bm/Cm [T, N] (one group), dt [T, H] (already softplus'ed), A [H] (= -exp(A_log)).
void orc_ssd_scan_sequential(const float* xs, const float* Bm, const float* Cm, const float* dt, const float* A,
                             const float* D, float* state, float* y, int T, int H, int P, int N) {
#pragma omp parallel for schedule(static)
    for (int row = 0; row < H * P; ++row) {
        const int h = row / P;
        float* s = state + (size_t)row * N;
        for (int t = 0; t < T; ++t) {
            const float dtv = dt[(size_t)t * H + h];
            const float dA = std::exp(A[h] * dtv);
            const float xv = xs[(size_t)t * H * P + row];
            float acc = 0.f;
            for (int j = 0; j < N; ++j) {
                s[j] = dA * s[j] + (dtv * Bm[(size_t)t * N + j]) * xv;
                acc += Cm[(size_t)t * N + j] * s[j];
            }
            y[(size_t)t * H * P + row] = acc + D[h] * xv;
        }
    }
}

// core/ops.cpp:597-633 (CPU: materialise to fp16) + core/mamba_cpu.cpp:48-198
int orc_mamba2_forward_q(const float* x, const void* w_in, const float* conv_w, const float* conv_b,
                         const float* dt_bias, const float* a_log, const float* D, const float* norm_w,
                         const void* w_out, float* state, float* out, int B, int T, int d, int d_inner,
                         int conv_dim, int n_heads, int d_head, int d_state, int k, float eps, int qkind) {
    if (B <= 0 || T <= 0) return 0;
    const int proj = d_inner + conv_dim + n_heads, N = B * T;
    if ((conv_dim - d_inner) != 2 * d_state) return -1;  // n_groups == 1 only
    std::vector<u16> wi((size_t)proj * d), wo((size_t)d * d_inner);
    if (qkind >= 0) {
        materialize(qkind, w_in, wi.data(), (i64)proj * d);
        materialize(qkind, w_out, wo.data(), (i64)d * d_inner);
    } else {
        std::memcpy(wi.data(), w_in, wi.size() * 2);
        std::memcpy(wo.data(), w_out, wo.size() * 2);
    }
    std::vector<float> pr((size_t)N * proj), bc((size_t)N * conv_dim), y((size_t)N * d_inner);
    linear_fp16(x, wi.data(), pr.data(), N, d, proj);
    const int wl = (k > 1) ? k - 1 : 1;
    for (int c = 0; c < conv_dim; ++c) {
        std::vector<float> win((size_t)wl);
        const float* wc = conv_w + (size_t)c * k;
        const float bcv = conv_b ? conv_b[c] : 0.f;
        for (int b = 0; b < B; ++b) {
            std::fill(win.begin(), win.end(), 0.f);
            for (int t = 0; t < T; ++t) {
                const float raw = pr[((size_t)b * T + t) * proj + d_inner + c];
                float acc = bcv;
                for (int j = 0; j < k; ++j) acc += wc[j] * ((j == k - 1) ? raw : win[(size_t)j]);
                bc[((size_t)b * T + t) * conv_dim + c] = acc / (1.0f + std::exp(-acc));
                for (int j = 0; j + 1 < wl; ++j) win[(size_t)j] = win[(size_t)j + 1];
                win[(size_t)wl - 1] = raw;
            }
        }
    }
    const int inner = n_heads * d_head;
#pragma omp parallel for schedule(static)
    for (int row = 0; row < B * inner; ++row) {
        const int b = row / inner, rem = row - b * inner, h = rem / d_head, i = rem - h * d_head;
        const float a = -std::exp(a_log[h]);
        float* s = state + (size_t)row * d_state;
        for (int t = 0; t < T; ++t) {
            const float* p = pr.data() + ((size_t)b * T + t) * proj;
            const float* br = bc.data() + ((size_t)b * T + t) * conv_dim;
            const float dti = p[proj - n_heads + h] + dt_bias[h];
            const float dtv = (dti > 20.0f) ? dti : std::log1p(std::exp(dti));
            const float dA = std::exp(a * dtv);
            const float xv = br[h * d_head + i];
            float acc = 0.f;
            for (int j = 0; j < d_state; ++j) {
                s[j] = dA * s[j] + (dtv * br[d_inner + j]) * xv;
                acc += br[d_inner + d_state + j] * s[j];
            }
            y[((size_t)b * T + t) * d_inner + h * d_head + i] = acc + D[h] * xv;
        }
    }
    for (int n = 0; n < N; ++n) {
        float* yr = y.data() + (size_t)n * d_inner;
        const float* gr = pr.data() + (size_t)n * proj;
        double var = 0.0;
        for (int c = 0; c < d_inner; ++c) {
            const float v = yr[c] * (gr[c] / (1.0f + std::exp(-gr[c])));
            yr[c] = v;
            var += (double)v * v;
        }
        var /= (double)d_inner;
        const float inv = 1.0f / std::sqrt((float)var + eps);
        for (int c = 0; c < d_inner; ++c) yr[c] = yr[c] * inv * norm_w[c];
    }
    linear_fp16(y.data(), wo.data(), out, N, d_inner, d);
    return 0;
}

int orc_mamba2_step_q(const float* x, const void* w_in, const float* conv_w, const float* conv_b,
                      const float* dt_bias, const float* a_log, const float* D, const float* norm_w,
                      const void* w_out, float* conv_state, float* ssm_state, float* out, int d, int d_inner,
                      int conv_dim, int n_heads, int d_head, int d_state, int k, float eps, int qkind) {
    if ((conv_dim - d_inner) != 2 * d_state) return -1;
    mamba_step(x, w_in, conv_w, conv_b, dt_bias, a_log, D, norm_w, w_out, conv_state, ssm_state, out, d,
               d_inner, conv_dim, n_heads, d_head, d_state, k, eps, qkind);
    return 0;
}

int orc_moe_route(const float* x, const float* rw, const float* bias, float* probs, int32_t* idx, float* w,
                  int64_t N, int d, int ne, int K) {
    if (K < 1 || K > 8 || ne <= 0 || ne > 64) return -1;  // core/moe_cpu.cpp:207-209
    for (i64 t = 0; t < N; ++t)
        route_one(x + t * d, rw, bias, d, ne, K, probs + t * ne, idx + t * K, w + t * K);
    return 0;
}

// Token permutation (own definition; the reference's CUDA grouping,
// cuda/moe.cu:623-651, orders slots by atomics). Stable sort of the N*K slot
// ids s = t*K + k by expert idx[s]; offsets[e] = first position of expert e.
void orc_moe_permute(const int32_t* idx, int64_t N, int K, int ne, int32_t* grouped, int32_t* offsets) {
    const i64 S = N * K;
    std::vector<i32> order((size_t)S);
    for (i64 s = 0; s < S; ++s) order[(size_t)s] = (i32)s;
    std::stable_sort(order.begin(), order.end(), [&](i32 a, i32 b) { return idx[a] < idx[b]; });
    for (i64 s = 0; s < S; ++s) grouped[s] = order[(size_t)s];
    for (int e = 0; e <= ne; ++e) offsets[e] = 0;
    for (i64 s = 0; s < S; ++s) offsets[idx[s] + 1]++;
    for (int e = 0; e < ne; ++e) offsets[e + 1] += offsets[e];
}

int orc_moe_forward_q(const float* x, const float* rw, const float* bias, const void* gates, const void* ups,
                      const void* downs, const void* sh_g, const void* sh_u, const void* sh_d, float* out,
                      int32_t* idx_out, float* w_out, int64_t N, int d, int E, int ne, int K, int SH, int qkind) {
    if (K < 1 || K > 8 || ne <= 0 || ne > 64 || d <= 0 || E <= 0) return -1;
    if (N <= 0) return 0;
    const std::vector<float> g = widen_q(gates, qkind, (i64)ne * E * d), u = widen_q(ups, qkind, (i64)ne * E * d),
                             dn = widen_q(downs, qkind, (i64)ne * d * E);
    std::vector<float> sg, su, sd;
    if (sh_g && sh_u && sh_d) {
        sg = widen_q(sh_g, qkind, (i64)SH * d);
        su = widen_q(sh_u, qkind, (i64)SH * d);
        sd = widen_q(sh_d, qkind, (i64)d * SH);
    }
    const bool sh = !sg.empty();
    moe_fwd_f32(x, rw, bias, g.data(), u.data(), dn.data(), sh ? sg.data() : nullptr, sh ? su.data() : nullptr,
                sh ? sd.data() : nullptr, out, idx_out, w_out, N, d, E, ne, K, SH);
    return 0;
}

// Synthetic Granite weights (our own recipe, shared with the product's
// host-side initialiser): every parameter has its own Rng stream seeded
// with seed ^ fnv1a64(name). Norm weights, conv bias, D and dt_bias are 1,
// A_log[h] = log(h+1) (the reference's init, model/model.cpp:1586-1603),
// the aux-free router bias 0 (model/model.cpp:179-191); everything else is
// N(0, 0.02).
void orc_synth_param_f32(const char* name, uint64_t seed, float* out, int64_t n) {
    const std::string s(name);
    auto ends = [&](const char* suf) {
        const size_t l = std::strlen(suf);
        return s.size() >= l && s.compare(s.size() - l, l, suf) == 0;
    };
    if (ends("norm") || ends("norm.weight") || ends("conv1d.bias") || ends("mamba.D") || ends("dt_bias")) {
        for (i64 i = 0; i < n; ++i) out[i] = 1.0f;
        return;
    }
    if (ends("A_log")) {
        for (i64 i = 0; i < n; ++i) out[i] = std::log((float)(i + 1));
        return;
    }
    if (ends("moe_bias")) {
        for (i64 i = 0; i < n; ++i) out[i] = 0.0f;
        return;
    }
    orc_rng_normal(seed ^ orc_fnv1a64(name, (i64)s.size()), 0.0f, 0.02f, out, n);
}

// The tiny-model generator: Generator::prefill (inference/generator.cpp:627-915,
// Mamba layers token by token through the host decode path) followed by
// greedy decode steps (:221-443), CPU dispatch, fused-Q4 on. cfg ints:
//  [0]V [1]d [2]L [3]H [4]KV [5]hd [6]E [7]ne [8]K [9]SH [10]d_inner
//  [11]m_heads [12]m_dhead [13]m_dstate [14]conv_k [15]qkind [16..16+L) layer types
// fcfg: [0] eps [1] attention scale. Parameter names follow model/model.cpp:1087-1160.
// Writes n_new greedy ids and, per id, the top-2 logit margin it was chosen with.
int orc_granite_generate(const int32_t* cfg, const float* fcfg, const char** names, const void** ptrs, int nparams,
                         const int32_t* prompt, int P, int n_new, int max_ctx, int32_t* out_ids,
                         float* out_margins) {
    return orc_granite_generate_timed(cfg, fcfg, names, ptrs, nparams, prompt, P, n_new, max_ctx, out_ids,
                                      out_margins, nullptr);
}

// As above; seconds (optional): [0] prefill wall time, [1] decode wall time.
int orc_granite_generate_timed(const int32_t* cfg, const float* fcfg, const char** names, const void** ptrs,
                               int nparams, const int32_t* prompt, int P, int n_new, int max_ctx, int32_t* out_ids,
                               float* out_margins, double* seconds) {
    return orc_granite_generate_ex(cfg, 16 + cfg[2], fcfg, 2, names, ptrs, nparams, prompt, P, n_new, max_ctx,
                                   nullptr, out_ids, out_margins, nullptr, seconds);
}

// The general form. Optional Granite fields (defaults when past ncfg / nfcfg):
// cfg[16+L] tie_embeddings (1; 0 = the "lm_head" fp16 parameter is the output
// projection, model/model.h:465), cfg[17+L] moe_aux_free (0; 1 = per-layer
// "layers.N.moe_bias" fp32 router bias, Model::moe_bias_ptr), fcfg[2]
// embedding_multiplier, fcfg[3] residual_multiplier, fcfg[4] logits_scaling
// (1; inference/generator.cpp:248-249, 266-267, 440-441 and :705, 762, 907).
// forced (optional, n_new ids): step s feeds forced[s] instead of the greedy
// id (teacher forcing; out_ids still records the greedy id of each step).
// out_logits (optional, n_new x V): the logits each id was picked from.
int orc_granite_generate_ex(const int32_t* cfg, int ncfg, const float* fcfg, int nfcfg, const char** names,
                            const void** ptrs, int nparams, const int32_t* prompt, int P, int n_new, int max_ctx,
                            const int32_t* forced, int32_t* out_ids, float* out_margins, float* out_logits,
                            double* seconds) {
    using clk = std::chrono::steady_clock;
    const auto t_start = clk::now();
    const int V = cfg[0], d = cfg[1], L = cfg[2], H = cfg[3], KV = cfg[4], hd = cfg[5], E = cfg[6], ne = cfg[7],
              K = cfg[8], SH = cfg[9], di = cfg[10], mh = cfg[11], mdh = cfg[12], mds = cfg[13], ck = cfg[14],
              qk = cfg[15];
    const int* lt = cfg + 16;
    const float eps = fcfg[0], scale = fcfg[1];
    if (ncfg < 16 + L) return -1;
    const bool tied = ncfg > 16 + L ? cfg[16 + L] != 0 : true;
    const bool aux_free = ncfg > 17 + L ? cfg[17 + L] != 0 : false;
    const float emb_mult = nfcfg > 2 ? fcfg[2] : 1.0f, res_mult = nfcfg > 3 ? fcfg[3] : 1.0f,
                logits_scaling = nfcfg > 4 ? fcfg[4] : 1.0f;
    const int conv_dim = di + 2 * mds, qd = H * hd, kvd = KV * hd, win = ck > 1 ? ck - 1 : 1;
    if (P < 1 || P > 1024 || P + n_new > max_ctx) return -1;
    std::map<std::string, const void*> pm;
    for (int i = 0; i < nparams; ++i) pm[names[i]] = ptrs[i];
    auto W = [&](const std::string& n) -> const void* {
        auto it = pm.find(n);
        return it == pm.end() ? nullptr : it->second;
    };
    auto F = [&](const std::string& n) { return (const float*)W(n); };
    for (int l = 0; l < L; ++l) {
        const std::string pre = "layers." + std::to_string(l) + ".";
        if (!W(pre + "attn_norm") || !W(pre + "moe_gate")) return -2;
        if (lt[l] == 0 && !W(pre + "mamba.in_proj")) return -2;
        if (lt[l] != 0 && !W(pre + "wq")) return -2;
    }
    const u16* emb = (const u16*)W("tok_embeddings");
    const u16* head = tied ? emb : (const u16*)W("lm_head");
    if (!emb || !head || !W("final_norm")) return -2;
    auto scale_emb = [&](float* x, size_t n) {  // ops::scale_inplace: a[i] *= s
        if (emb_mult != 1.0f)
            for (size_t i = 0; i < n; ++i) x[i] *= emb_mult;
    };
    auto add_branch = [&](float* x, float* br, size_t n) {
        if (res_mult != 1.0f)
            for (size_t i = 0; i < n; ++i) br[i] *= res_mult;
        for (size_t i = 0; i < n; ++i) x[i] += br[i];
    };

    // state: per-mamba-layer conv + ssm, per-attention-layer fp16 K/V cache
    std::map<int, std::vector<float>> conv, ssm;
    std::map<int, std::vector<u16>> kc, vc;
    for (int l = 0; l < L; ++l) {
        if (lt[l] == 0) {
            conv[l].assign((size_t)conv_dim * win, 0.f);
            ssm[l].assign((size_t)mh * mdh * mds, 0.f);
        } else {
            kc[l].assign((size_t)max_ctx * kvd, 0);
            vc[l].assign((size_t)max_ctx * kvd, 0);
        }
    }
    const int pinned_cfg = std::max(0, std::min(8, max_ctx - 1));  // generator.cpp:94
    int len = 0;

    auto moe = [&](int l, const float* xb, float* outp, int n) {
        const std::string pre = "layers." + std::to_string(l) + ".";
        orc_moe_forward_q(xb, F(pre + "moe_router"), aux_free ? F(pre + "moe_bias") : nullptr, W(pre + "moe_gate"),
                          W(pre + "moe_up"),
                          W(pre + "moe_down"), W(pre + "moe_sh_gate"), W(pre + "moe_sh_up"), W(pre + "moe_sh_down"),
                          outp, nullptr, nullptr, n, d, E, ne, K, SH, qk);
    };
    auto mstep = [&](int l, const float* xin, float* outp) {
        const std::string mp = "layers." + std::to_string(l) + ".mamba.";
        mamba_step(xin, W(mp + "in_proj"), F(mp + "conv1d.weight"), F(mp + "conv1d.bias"), F(mp + "dt_bias"),
                   F(mp + "A_log"), F(mp + "D"), F(mp + "norm.weight"), W(mp + "out_proj"), conv[l].data(),
                   ssm[l].data(), outp, d, di, conv_dim, mh, mdh, mds, ck, eps, qk);
    };
    auto lin = [&](const std::string& n, const float* xx, float* yy, int M, int Kd, int Nd) {
        linear_q(xx, W(n), yy, M, Kd, Nd, qk);
    };
    std::vector<float> logits((size_t)V);
    auto finish = [&](const float* xrow) {
        std::vector<float> h((size_t)d);
        rmsnorm(xrow, F("final_norm"), h.data(), nullptr, 1, d, eps);
        linear_fp16(h.data(), head, logits.data(), 1, d, V);  // lm_head, fp16
        if (logits_scaling != 1.0f) {
            const float inv = 1.0f / logits_scaling;
            for (int i = 0; i < V; ++i) logits[(size_t)i] *= inv;
        }
    };

    // ---- prefill (generator.cpp:627-915)
    {
        std::vector<float> x((size_t)P * d), xb((size_t)P * d), pr((size_t)P * d), q((size_t)P * qd),
            k((size_t)P * kvd), v((size_t)P * kvd), att((size_t)P * qd);
        orc_embedding_forward_half(prompt, emb, x.data(), P, d, V);
        scale_emb(x.data(), x.size());
        for (int l = 0; l < L; ++l) {
            const std::string pre = "layers." + std::to_string(l) + ".";
            rmsnorm(x.data(), F(pre + "attn_norm"), xb.data(), nullptr, P, d, eps);
            if (lt[l] == 0) {
                for (int t = 0; t < P; ++t) mstep(l, xb.data() + (size_t)t * d, pr.data() + (size_t)t * d);
            } else {
                lin(pre + "wq", xb.data(), q.data(), P, d, qd);
                lin(pre + "wk", xb.data(), k.data(), P, d, kvd);
                lin(pre + "wv", xb.data(), v.data(), P, d, kvd);
                for (size_t i = 0; i < (size_t)P * kvd; ++i) {
                    kc[l][i] = f32_to_f16(k[i]);
                    vc[l][i] = f32_to_f16(v[i]);
                }
                attn_prefill(q.data(), k.data(), v.data(), att.data(), 1, P, H, KV, hd, scale, 0);
                lin(pre + "wo", att.data(), pr.data(), P, qd, d);
            }
            add_branch(x.data(), pr.data(), x.size());
            rmsnorm(x.data(), F(pre + "ffn_norm"), xb.data(), nullptr, P, d, eps);
            moe(l, xb.data(), pr.data(), P);
            add_branch(x.data(), pr.data(), x.size());
        }
        len = P;
        finish(x.data() + (size_t)(P - 1) * d);
    }
    const auto t_prefill = clk::now();
    // ---- greedy decode (generator.cpp:985-1098 greedy + :221-443)
    std::vector<float> x((size_t)d), xb((size_t)d), pr((size_t)d), q((size_t)qd), k((size_t)kvd), v((size_t)kvd),
        att((size_t)qd);
    for (int step = 0; step < n_new; ++step) {
        const i32 next = argmax(logits.data(), V);
        float best = -std::numeric_limits<float>::infinity(), second = best;
        for (int i = 0; i < V; ++i) {
            if (!std::isfinite(logits[(size_t)i])) continue;
            if (logits[(size_t)i] > best) { second = best; best = logits[(size_t)i]; }
            else if (logits[(size_t)i] > second) second = logits[(size_t)i];
        }
        out_ids[step] = next;
        out_margins[step] = best - second;
        if (out_logits) std::memcpy(out_logits + (size_t)step * V, logits.data(), sizeof(float) * (size_t)V);
        if (step == n_new - 1) break;
        const i32 fed = forced ? forced[step] : next;
        orc_embedding_forward_half(&fed, emb, x.data(), 1, d, V);
        scale_emb(x.data(), x.size());
        const int slot = len;  // ring never wraps: P + n_new <= max_ctx
        ++len;
        for (int l = 0; l < L; ++l) {
            const std::string pre = "layers." + std::to_string(l) + ".";
            rmsnorm(x.data(), F(pre + "attn_norm"), xb.data(), nullptr, 1, d, eps);
            if (lt[l] == 0) {
                mstep(l, xb.data(), pr.data());
            } else {
                lin(pre + "wq", xb.data(), q.data(), 1, d, qd);
                lin(pre + "wk", xb.data(), k.data(), 1, d, kvd);
                lin(pre + "wv", xb.data(), v.data(), 1, d, kvd);
                for (int i = 0; i < kvd; ++i) {
                    kc[l][(size_t)slot * kvd + i] = f32_to_f16(k[(size_t)i]);
                    vc[l][(size_t)slot * kvd + i] = f32_to_f16(v[(size_t)i]);
                }
                const int pinned = std::min(pinned_cfg, len);
                decode_ring(q.data(), kc[l].data(), vc[l].data(), att.data(), H, KV, hd, 0, pinned, len, max_ctx,
                            scale, 0, [](u16 h) { return f16_to_f32(h); });
                lin(pre + "wo", att.data(), pr.data(), 1, qd, d);
            }
            add_branch(x.data(), pr.data(), (size_t)d);
            rmsnorm(x.data(), F(pre + "ffn_norm"), xb.data(), nullptr, 1, d, eps);
            moe(l, xb.data(), pr.data(), 1);
            add_branch(x.data(), pr.data(), (size_t)d);
        }
        finish(x.data());
    }
    if (seconds) {
        seconds[0] = std::chrono::duration<double>(t_prefill - t_start).count();
        seconds[1] = std::chrono::duration<double>(clk::now() - t_prefill).count();
    }
    return 0;
}

}  // extern "C"
