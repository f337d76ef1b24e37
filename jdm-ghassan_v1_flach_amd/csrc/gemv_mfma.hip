// Small-M GEMV (M = 1..8 tokens) for Q4_K and Q8_0 weights on the matrix
// cores: y[t][n] = sum_k x[t][k] * w[n][k], the decode hot path of
// linear_forward_q4 (core/ops.cpp:360-408).
//
// Why MFMA for a memory-bound op: the VALU budget at 8 TB/s is under three
// lane-ops per Q4_K weight, and a scalar dot spends most of it turning
// nibbles into numbers. Here a weight costs ~0.6 lane-ops: integer codes are
// masked straight into fp16 *subnormals* (bits 0x000q are the number
// q * 2^-24, exact) and v_mfma_f32_16x16x32_f16 multiplies them exactly,
// accumulating in fp32. Per-sub-block scales are applied afterwards.
//
// Block-diagonal trick. In D[m][n] = sum_k A[m][k] B[k][n] (16x16x32), lane
// l holds B[8g..8g+7][n] and D[4g..4g+3][n] with n = l%16, g = l/16. The
// weights are B (16 rows of W = 16 columns n); lane (n, g) loads ITS OWN 8
// codes per MFMA. The activations are A, and A row m is non-zero only in
// k-slot g = m/4. So D[4g+e][n] is the dot of lane (n,g)'s own 8 codes with
// activation vector e: every lane ends up with the partial sums of exactly
// the codes it loaded, for 4 activation vectors e at once. e runs over
// (token, hi/lo part): x = hi + lo with hi = fp16(x), lo = fp16(x - hi),
// which keeps ~22 bits of each activation, so the result is as accurate as
// an fp32-activation dot (the reference's CPU path, core/ops.cpp:304-338,
// multiplies fp16-rounded weights with fp32 activations).
//
// Code types (u = a dword of 4 packed bytes; each 16-bit half must stay
// below 0x0400, the subnormal range, so only bits 0..9 may hold a code):
//   Q4_K  c0 = u & 0x000F000F        low nibbles of bytes 0,2    (value q)
//         c1 = (u>>8) & 0x000F000F   low nibbles of bytes 1,3    (q)
//         c2 = u & 0x00F000F0        high nibbles of bytes 0,2   (16 q)
//         c3 = (u>>8) & 0x00F000F0   high nibbles of bytes 1,3   (16 q)
//   Q8_0  v_perm_b32 spreads bytes (flipped: q + 128) into 16-bit halves.
// Codes of one sub-block (Q4_K) or one block (Q8_0) share an MFMA
// accumulation chain with a single power-of-two scale, removed exactly
// afterwards. The
// activations in LDS are laid out in the order the codes come out of the
// dwords (the dot is invariant under a common permutation of k).
//
// Work: a tile is 16 rows; the K range of a tile is split over the WB waves
// of a block (SBW super-blocks of 256 values each); the per-wave partials
// are summed through LDS in a fixed order (deterministic). A block walks
// over `tpb` consecutive tiles; a wave issues all its loads of a tile at
// once (the first tile's before the activations are staged, the next
// tile's as soon as the current one's bytes are consumed).
#include <stdlib.h>

#include "gemv_fuse.h"
#include "lds_dma.h"

namespace gh {

typedef _Float16 gm_half8 __attribute__((ext_vector_type(8)));
typedef float gm_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t gm_u4 __attribute__((ext_vector_type(4)));

template <int KIND>
struct GmCfg;
template <>
struct GmCfg<3> {  // Q4_K: 144-byte super-blocks; a lane uses 16 B header + 32 B nibbles
    static constexpr int DW = 12;
    static constexpr int SB_BYTES = 144;
};
template <>
struct GmCfg<2> {  // Q8_0: 8 blocks of 34 bytes; a lane uses two blocks (17 dwords)
    static constexpr int DW = 17;
    static constexpr int SB_BYTES = 272;
};

__device__ __forceinline__ float gm_lo16(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFFu)); }
__device__ __forceinline__ float gm_hi16(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }

// This lane's bytes of super-block `sbl` of row n16 from the wave's LDS
// slice (row stride RS bytes).
template <int KIND>
__device__ __forceinline__ void gm_lds_slice(const unsigned char* rowp, int sbl, int g, uint32_t* w) {
    if constexpr (KIND == 3) {
        const unsigned char* p = rowp + sbl * 144;
        const uint4 h = *(const uint4*)p;
        const uint4 a = *(const uint4*)(p + 16 + 32 * g);
        const uint4 b = *(const uint4*)(p + 32 + 32 * g);
        w[0] = h.x; w[1] = h.y; w[2] = h.z; w[3] = h.w;
        w[4] = a.x; w[5] = a.y; w[6] = a.z; w[7] = a.w;
        w[8] = b.x; w[9] = b.y; w[10] = b.z; w[11] = b.w;
    } else {
        const uint32_t* p = (const uint32_t*)(rowp + sbl * 272 + 68 * g);
#pragma unroll
        for (int i = 0; i < 17; ++i) w[i] = p[i];
    }
}

// Codes of MFMA (chain c, step r) for this lane, as the B operand.
template <int KIND>
__device__ __forceinline__ gm_half8 gm_codes(const uint32_t* w, const uint32_t* u, int c, int r) {
    gm_u4 v;
    if constexpr (KIND == 3) {
        const uint32_t* q = w + 4 + 4 * r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t s = q[i];
            const uint32_t t = (c & 1) ? (s >> 8) : s;
            v[i] = t & ((c & 2) ? 0x00F000F0u : 0x000F000Fu);
        }
    } else {
        // u = w ^ 0x80808080 (byte = q + 128). Block 0 quants: stream bytes
        // 2..33, block 1: 36..67. Values 8r..8r+7 of block c.
        if (c == 0) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int j = 2 * r + i;  // values 4j..4j+3 = bytes 4j+2..4j+5
                v[2 * i] = __builtin_amdgcn_perm(u[j + 1], u[j], 0x0c030c02u);
                v[2 * i + 1] = __builtin_amdgcn_perm(u[j + 1], u[j], 0x0c050c04u);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int j = 9 + 2 * r + i;  // values 4(j-9).. = bytes 4j..4j+3
                v[2 * i] = __builtin_amdgcn_perm(0u, u[j], 0x0c010c00u);
                v[2 * i + 1] = __builtin_amdgcn_perm(0u, u[j], 0x0c030c02u);
            }
        }
    }
    return __builtin_bit_cast(gm_half8, v);
}

// Position (within the 256-value super-block) of element el of the 8 codes
// lane slot g feeds to MFMA r8 = chain*steps + step.
template <int KIND>
__host__ __device__ __forceinline__ int gm_kpos(int r8, int g, int el) {
    if constexpr (KIND == 3) {
        const int c = r8 >> 1, r = r8 & 1;
        const int i = 4 * r + (el >> 1);
        const int b = 4 * i + (c & 1) + 2 * (el & 1);
        return 64 * g + (c >= 2 ? 32 : 0) + b;
    } else {
        const int c = r8 >> 2, r = r8 & 3;
        return 64 * g + 32 * c + 8 * r + el;
    }
}

// Inverse of gm_kpos: where value kk (0..255) of a super-block goes.
template <int KIND>
__device__ __forceinline__ void gm_kinv(int kk, int& r8, int& g, int& el) {
    g = kk >> 6;
    if constexpr (KIND == 3) {
        const int half = (kk >> 5) & 1, b = kk & 31;
        const int i = b >> 2, bb = b & 3;
        const int c = half * 2 + (bb & 1);
        r8 = c * 2 + (i >> 2);
        el = 2 * (i & 3) + (bb >> 1);
    } else {
        r8 = ((kk >> 5) & 1) * 4 + ((kk >> 3) & 3);
        el = kk & 7;
    }
}

// ---------------------------------------------------------- fusion hooks
// Block-wide sum of a double over DPP and one LDS exchange (all threads get the total).
__device__ __forceinline__ double gm_block_sum_dpp(double v, double* red) {
    v = wave_sum(v);
    const int nw = blockDim.x >> 6;
    if (nw == 1) return v;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

// Block-wide sum of a double (all threads get the total).
__device__ __forceinline__ double gm_block_sum(double v, double* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

// Writes activation k of token t (M tokens) into the MFMA A-operand layout:
// its fp16 hi and lo parts at the code-order position of its super-block.
template <int KIND>
__device__ __forceinline__ void gm_put_a(uint16_t* a16, int M, int t, int k, float v) {
    int r8, gg, el;
    gm_kinv<KIND>(k & 255, r8, gg, el);
    const _Float16 hi = (_Float16)v;
    const _Float16 lo = (_Float16)(v - (float)hi);
    const int base = (((((k >> 8) * 8 + r8) * M + t) * 4 + gg) * 2) * 8 + el;
    a16[base] = __builtin_bit_cast(uint16_t, hi);
    a16[base + 8] = __builtin_bit_cast(uint16_t, lo);
}

// The activations of ONE token formed by a prologue go straight into the A
// layout: element i = tid + j*nth is held by consecutive lanes, so 32 lanes
// hold a 32-value group and reduce its sum with shuffles.
template <int KIND>
__device__ __forceinline__ void gm_put_one(uint16_t* a16, float* xsum, int i, float v) {
    gm_put_a<KIND>(a16, 1, 0, i, v);
    float sum = v;
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) sum += __shfl_xor(sum, o, 64);
    if ((i & 31) == 0) xsum[i >> 5] = sum;
}

// Forms the activation vector of ONE token (K values) directly into the
// MFMA layout + group sums; every block computes the same values. Every
// operand is requested before the first one is used (one memory round trip
// instead of one per dependent load): a thread keeps its first elements
// of each input in registers; xf [K floats] is scratch for the rest.
constexpr int GM_SPR = 4;  // attention splits whose partials are held in registers

template <int KIND>
__device__ void gm_prologue(const float* __restrict__ x, int K, const GmFuse& f, float* xf, uint16_t* a16,
                            float* xsum) {
    __shared__ double red[16];
    const int tid = threadIdx.x, nth = blockDim.x;
    if (f.pro == GM_PRO_RMSNORM || f.pro == GM_PRO_GATED) {
        // elementwise.hip k_rmsnorm: double sum of squares, x * inv * w;
        // mamba.hip k_gated_norm: v = y * silu(z), double variance, float rsqrt.
        // Thread tid holds the 8 consecutive elements 8 tid .. 8 tid + 7 (further chunks of
        // 8 nth go through xf), so a 32-value group sits in 4 lanes of a quad.
        const bool gated = f.pro == GM_PRO_GATED;
        const int c0 = 8 * tid;
        const bool mine = c0 < K;
        // the step's start folded in (layer 0 of a decode step): the input is the fp16
        // embedding row of token bctl[0] (elementwise.hip k_embed_half: zero out of range), and
        // the first block stores it as the step's residual stream
        const bool emb = f.emb != nullptr;
        const int tok = emb ? f.bctl[0] : 0;
        const bool tok_ok = tok >= 0 && tok < f.vocab;
        const bool emb_writer = emb && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0;
        auto emb8 = [&](int c, float* o) {
            uint4 h = make_uint4(0, 0, 0, 0);
            if (tok_ok) h = *(const uint4*)(f.emb + (size_t)tok * K + c);
            const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                o[2 * j] = f16_to_f32((uint16_t)(hw[j] & 0xFFFF));
                o[2 * j + 1] = f16_to_f32((uint16_t)(hw[j] >> 16));
            }
            if (emb_writer) {
                *(float4*)(f.emb_out + c) = make_float4(o[0], o[1], o[2], o[3]);
                *(float4*)(f.emb_out + c + 4) = make_float4(o[4], o[5], o[6], o[7]);
            }
        };
        float xr[8], wr[8], zr[8];
        if (mine && emb) {
            const float4 w0 = *(const float4*)(f.pw + c0), w1 = *(const float4*)(f.pw + c0 + 4);
            emb8(c0, xr);
            wr[0] = w0.x; wr[1] = w0.y; wr[2] = w0.z; wr[3] = w0.w; wr[4] = w1.x; wr[5] = w1.y; wr[6] = w1.z; wr[7] = w1.w;
        } else if (mine) {
            const float4 x0 = *(const float4*)(x + c0), x1 = *(const float4*)(x + c0 + 4);
            const float4 w0 = *(const float4*)(f.pw + c0), w1 = *(const float4*)(f.pw + c0 + 4);
            xr[0] = x0.x; xr[1] = x0.y; xr[2] = x0.z; xr[3] = x0.w; xr[4] = x1.x; xr[5] = x1.y; xr[6] = x1.z; xr[7] = x1.w;
            wr[0] = w0.x; wr[1] = w0.y; wr[2] = w0.z; wr[3] = w0.w; wr[4] = w1.x; wr[5] = w1.y; wr[6] = w1.z; wr[7] = w1.w;
            if (gated) {
                const float4 z0 = *(const float4*)(f.pz + c0), z1 = *(const float4*)(f.pz + c0 + 4);
                zr[0] = z0.x; zr[1] = z0.y; zr[2] = z0.z; zr[3] = z0.w; zr[4] = z1.x; zr[5] = z1.y; zr[6] = z1.z; zr[7] = z1.w;
            }
        }
        double ss = 0.0;
        if (mine) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float v = xr[j];
                if (gated) v = v * (zr[j] / (1.0f + expf(-zr[j])));
                xr[j] = v;
                ss += (double)v * v;
            }
        }
        for (int c = c0 + 8 * nth; c < K; c += 8 * nth) {  // chunks beyond the registers
            float er[8];
            if (emb) emb8(c, er);
            for (int j = 0; j < 8; ++j) {
                float v = emb ? er[j] : x[c + j];
                if (gated) v = v * (f.pz[c + j] / (1.0f + expf(-f.pz[c + j])));
                xf[c + j] = v;
                ss += (double)v * v;
            }
        }
        // the step's cache slot, taken once (nothing in this launch reads it)
        if (emb_writer && tid == 0) decode_alloc_slot(f.bctl);
        const double tot = gm_block_sum_dpp(ss, red);
        float inv;
        if (gated) {
            inv = 1.0f / sqrtf((float)(tot / (double)K) + f.eps);
        } else {
            const double invd = 1.0 / sqrt(tot / (double)K + (double)f.eps);
            inv = isfinite(invd) ? (float)invd : 0.0f;
        }
        // values into the A layout; the 32-value sums over the quad (every lane runs the DPP)
        const int rounds = (K + 8 * nth - 1) / (8 * nth);  // the same for every lane
        for (int m = 0; m < rounds; ++m) {
            const int c = c0 + 8 * nth * m;
            float sum = 0.f;
            if (c < K) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float v = (m == 0 ? xr[j] : xf[c + j]) * inv * (m == 0 ? wr[j] : f.pw[c + j]);
                    gm_put_a<KIND>(a16, 1, 0, c + j, v);
                    sum += v;
                }
            }
            sum += dpp_f32<0xB1>(sum);
            sum += dpp_f32<0x4E>(sum);
            if (c < K && (tid & 3) == 0) xsum[c >> 5] = sum;
        }
    } else {
        // attention.hip k_attn_combine for all H heads at once. Output
        // i = h*hd + c. (A) every (m, l) pair goes to LDS and every thread
        // requests the partial outputs of its elements; (B) thread h turns
        // its head's pairs into split weights; (C) ordered weighted sums.
        const int H = f.H, S = f.splits, hd = f.hd;
        float* sm = xf;              // [H][S] running max, then split weight
        float* sl = xf + H * S;      // [H][S] sums
        float* sinv = sl + H * S;    // [H]
        for (int q = tid; q < H * S; q += nth) {
            const int h = q / S, sp = q - h * S;
            const float* p = f.ml + (((size_t)(h / f.G) * S + sp) * f.G + h % f.G) * 2;
            sm[q] = p[0];
            sl[q] = p[1];
        }
        // thread tid: the 8 consecutive elements 8 tid .. (one head), their first GM_SPR splits
        // requested now; further chunks of 8 nth load their partials when merged
        const int c0 = 8 * tid;
        float ov[GM_SPR][8];
        if (c0 < K) {
            const int h = c0 / hd, c = c0 - h * hd;
            const float* op = f.o_part + ((size_t)(h / f.G) * S * f.G + h % f.G) * hd + c;
#pragma unroll
            for (int sp = 0; sp < GM_SPR; ++sp)
                if (sp < S) {
                    const float4 a0 = *(const float4*)(op + (size_t)sp * f.G * hd);
                    const float4 a1 = *(const float4*)(op + (size_t)sp * f.G * hd + 4);
                    ov[sp][0] = a0.x; ov[sp][1] = a0.y; ov[sp][2] = a0.z; ov[sp][3] = a0.w;
                    ov[sp][4] = a1.x; ov[sp][5] = a1.y; ov[sp][6] = a1.z; ov[sp][7] = a1.w;
                }
        }
        __syncthreads();
        if (tid < H) {
            float Mx = -INFINITY;
            for (int sp = 0; sp < S; ++sp)
                if (sl[tid * S + sp] > 0.f) Mx = fmaxf(Mx, sm[tid * S + sp]);
            float L = 0.f;
            for (int sp = 0; sp < S; ++sp) {
                const float l = sl[tid * S + sp];
                const float w = l > 0.f ? expf(sm[tid * S + sp] - Mx) : 0.f;
                sm[tid * S + sp] = w;
                L += w * l;
            }
            sinv[tid] = L > 0.f ? 1.0f / L : 0.0f;
        }
        __syncthreads();
        const int rounds = (K + 8 * nth - 1) / (8 * nth);  // the same for every lane
        for (int m = 0; m < rounds; ++m) {
            const int c = c0 + 8 * nth * m;
            float sum = 0.f;
            if (c < K) {
                const int h = c / hd, cc = c - h * hd;
                const float* op = f.o_part + ((size_t)(h / f.G) * S * f.G + h % f.G) * hd + cc;
                float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                // splits in order; an empty split (weight 0) has no partials written and is skipped
#pragma unroll
                for (int sp = 0; sp < GM_SPR; ++sp) {
                    const float w = sp < S ? sm[h * S + sp] : 0.f;
                    if (w != 0.f) {
#pragma unroll
                        for (int j = 0; j < 8; ++j) acc[j] += w * (m == 0 ? ov[sp][j] : op[(size_t)sp * f.G * hd + j]);
                    }
                }
                for (int sp = GM_SPR; sp < S; ++sp) {
                    const float w = sm[h * S + sp];
                    if (w != 0.f) {
#pragma unroll
                        for (int j = 0; j < 8; ++j) acc[j] += w * op[(size_t)sp * f.G * hd + j];
                    }
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float v = acc[j] * sinv[h];
                    gm_put_a<KIND>(a16, 1, 0, c + j, v);
                    sum += v;
                }
            }
            sum += dpp_f32<0xB1>(sum);
            sum += dpp_f32<0x4E>(sum);
            if (c < K && (tid & 3) == 0) xsum[c >> 5] = sum;
        }
    }
    __syncthreads();
}

// Epilogue operands of one output row, requested at kernel start.
struct GmEpiPre {
    float v[16];  // ADD: v[0] = y[n]; CONV: taps [0,ck), bias ck, window ck+1..
    int slot;
};

__device__ __forceinline__ void gm_epi_prefetch(const float* __restrict__ y, int n, const GmFuse& f, GmEpiPre& e) {
    if (f.epi == GM_EPI_ADD) {
        e.v[0] = y[n];
    } else if (f.epi == GM_EPI_QKV) {
        e.slot = *f.slot;
    } else if (f.epi == GM_EPI_CONV) {
        const int c = n - f.c0;
        if (c >= 0 && c < f.cdim && f.ck <= 8) {
            const int k = f.ck, wl = k > 1 ? k - 1 : 1;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (j < k) e.v[j] = f.conv_w[(size_t)c * k + j];
            e.v[8] = f.conv_b ? f.conv_b[c] : 0.0f;
#pragma unroll
            for (int j = 0; j < 7; ++j)
                if (j < wl) e.v[9 + j] = f.conv_win[(size_t)c * wl + j];
        }
    }
}

// Output n (value v) of a fused GEMV, ONE token; `pre` holds the operands
// fetched at kernel start (use_pre) or, if not, loads them now.
__device__ __forceinline__ void gm_epilogue(float* __restrict__ y, int yi, int n, float v, const GmFuse& f,
                                            const GmEpiPre& e, bool use_pre) {
    const GmEpiPre* pre = use_pre ? &e : nullptr;
    if (f.epi == GM_EPI_ADD) {
        y[yi] = (pre ? pre->v[0] : y[yi]) + v;
    } else if (f.epi == GM_EPI_QKV) {
        if (n < f.n0) {
            y[yi] = v;
        } else {
            const int r = n - f.n0;
            const size_t base = (size_t)(pre ? pre->slot : *f.slot) * f.kvd;
            if (r < f.kvd) f.kc[base + r] = f32_to_f16(v);
            else f.vc[base + r - f.kvd] = f32_to_f16(v);
        }
    } else {  // GM_EPI_CONV: mamba.hip k_step_conv on channel n - c0
#pragma clang fp contract(off)
        const int c = n - f.c0;
        if (c >= 0 && c < f.cdim) {
            const int k = f.ck, wl = k > 1 ? k - 1 : 1;
            float* wc = f.conv_win + (size_t)c * wl;
            if (pre && k <= 8) {
                float acc = pre->v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (j < k) acc += pre->v[j] * ((j == k - 1) ? v : pre->v[9 + j]);
                y[yi] = acc / (1.0f + expf(-acc));
#pragma unroll
                for (int j = 0; j < 7; ++j)
                    if (j + 1 < wl) wc[j] = pre->v[10 + j];
                wc[wl - 1] = v;
            } else {
                float acc = f.conv_b ? f.conv_b[c] : 0.0f;
                for (int j = 0; j < k; ++j) acc += f.conv_w[(size_t)c * k + j] * ((j == k - 1) ? v : wc[j]);
                y[yi] = acc / (1.0f + expf(-acc));
                for (int j = 0; j + 1 < wl; ++j) wc[j] = wc[j + 1];
                wc[wl - 1] = v;
            }
        } else {
            y[yi] = v;
        }
    }
}

// Weight bytes move in "steps": SS consecutive super-blocks of the 16 rows
// of a tile. A wave reads a step with contiguous 16-byte pieces (each row's
// SS*SB_BYTES bytes are contiguous, so a load instruction touches few
// cache lines), parks it in its own LDS slice, and every lane then reads
// its MFMA-layout bytes back from there. The next step's pieces are loaded
// into the same registers while the current step is multiplied.
template <int KIND, int SS>
struct GmStep {
    static constexpr int PPR = SS * GmCfg<KIND>::SB_BYTES / 16;  // 16-byte pieces per row
    static constexpr int PPL = (16 * PPR + 63) / 64;             // pieces per lane
    static constexpr int RS = PPR * 16 + 16;                     // LDS row stride (padded: rows fall in distinct banks)
    static constexpr int BYTES = 16 * RS;                        // LDS slice per wave
};

// LDS layout (bytes): [zero 16][A chunks: NSB*8*M*8 x 16][xsum: NSB*8*M f32]
//                     [red: 2*WB*16*M f32][weight slices: WB x GmStep::BYTES]
// Blocks of up to 16 waves for one token pair, up to 8 (twice the
// registers per lane) for more.
template <int KIND, int TP, int SS, bool FUSED>
__global__ void __launch_bounds__(TP == 1 ? 1024 : 512) k_gemv_mfma(const float* __restrict__ x, const uint8_t* __restrict__ W,
                                                    float* __restrict__ y, int M, int K, int N, size_t rowb,
                                                    int WB, int tpb, int spw, GmFuse f) {
    constexpr int DW = GmCfg<KIND>::DW;
    using St = GmStep<KIND, SS>;
    extern __shared__ __align__(16) unsigned char gm_smem[];
    const int NSB = K >> 8;
    const int nsteps = NSB / SS;
    uint4* zero = (uint4*)gm_smem;
    uint4* achunk = zero + 1;
    const int nchunks = NSB * 8 * M * 8;
    float* xsum = (float*)(achunk + nchunks);
    float* red = xsum + NSB * 8 * M;
    unsigned char* slices = (unsigned char*)(red + 2 * WB * 16 * M);
    float* xf = (float*)(slices + WB * St::BYTES);  // prologue output [K] (M = 1)
    const int tid = threadIdx.x, nth = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int n16 = lane & 15, g = lane >> 4;
    unsigned char* slice = slices + wave * St::BYTES;
    const int st0 = wave * spw;
    const int ns = max(0, min(spw, nsteps - st0));  // steps of this wave per tile
    // this lane's A chunk offset inside one (sb, r8) group (zero if off-diagonal)
    const int e = n16 & 3;
    const bool diag = (n16 >> 2) == g;
    int aoff[TP];
#pragma unroll
    for (int p = 0; p < TP; ++p) {
        const int t = 2 * p + (e >> 1);
        aoff[p] = (diag && t < M) ? ((t * 4 + g) * 2 + (e & 1)) : -1;
    }
    const int ntiles = (N + 15) >> 4;
    const int tile0 = blockIdx.x * tpb;
    const int tile1 = min(ntiles, tile0 + tpb);
    const int items = ns > 0 ? (tile1 - tile0) * ns : 0;
    // epilogue operands of the first tile's outputs (one token)
    GmEpiPre epre;
    if (FUSED && f.epi != GM_EPI_STORE && tid < 16 && tile0 < tile1 && tile0 * 16 + tid < N)
        gm_epi_prefetch(y, tile0 * 16 + tid, f, epre);

    uint4 P[St::PPL];
    auto load_item = [&](int it) {
        const int tile = tile0 + it / ns, step = st0 + it % ns;
        const uint8_t* base = W + (size_t)step * SS * GmCfg<KIND>::SB_BYTES;
#pragma unroll
        for (int i = 0; i < St::PPL; ++i) {
            const int q = lane + 64 * i;
            if (q < 16 * St::PPR) {
                const int r = q / St::PPR, j = q - r * St::PPR;
                int n = tile * 16 + r;
                n = n < N ? n : N - 1;
                const uint8_t* src = base;
                if (FUSED && f.w1 && n >= f.n0) {  // weight segments (tile-aligned)
                    const bool second = n < f.n0 + f.n1;
                    src = (const uint8_t*)(second ? f.w1 : f.w2) + (base - W);
                    n -= second ? f.n0 : f.n0 + f.n1;
                }
                P[i] = __builtin_bit_cast(uint4, __builtin_nontemporal_load((const gm_u4*)(src + (size_t)n * rowb + 16 * j)));
            }
        }
    };
    auto store_item = [&]() {
#pragma unroll
        for (int i = 0; i < St::PPL; ++i) {
            const int q = lane + 64 * i;
            if (q < 16 * St::PPR) {
                const int r = q / St::PPR, j = q - r * St::PPR;
                *(uint4*)(slice + r * St::RS + 16 * j) = P[i];
            }
        }
    };
    // ---- stage the activations: hi/lo fp16 parts in code order + the
    // 32-value sums. Coalesced float4 reads; each group of 8 lanes covers
    // one 32-value group and reduces its sum with shuffles. (K is a
    // multiple of 256, so every wave runs the loop the same number of times.)
    // The conversion runs while the first step's weight bytes are in flight.
    if (tid == 0) *zero = make_uint4(0, 0, 0, 0);
    const int K4 = K >> 2, xtotal = M * K4;
    // the first step's weight bytes are requested before anything else
    if (items > 0) load_item(0);
    uint16_t* a16 = (uint16_t*)achunk;
    if (FUSED && f.pro != GM_PRO_NONE) {
        // one token formed by the prologue straight into the A layout
        gm_prologue<KIND>(x, K, f, xf, a16, xsum);
    } else {
        auto xload = [&](int idx) {
            const int t = idx / K4, k = (idx - t * K4) * 4;
            return *(const float4*)(x + (size_t)t * K + k);
        };
        auto stage = [&](int idx, float4 v4) {
            const int t = idx / K4, k = (idx - t * K4) * 4;
            const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) gm_put_a<KIND>(a16, M, t, k + j, vv[j]);
            float sum = (vv[0] + vv[1]) + (vv[2] + vv[3]);
            sum += __shfl_xor(sum, 1, 64);
            sum += __shfl_xor(sum, 2, 64);
            sum += __shfl_xor(sum, 4, 64);
            if ((idx & 7) == 0) xsum[(k >> 5) * M + t] = sum;
        };
        constexpr int XP = 4;
        float4 xpre[XP];
#pragma unroll
        for (int i = 0; i < XP; ++i)
            if (tid + i * nth < xtotal) xpre[i] = xload(tid + i * nth);
#pragma unroll
        for (int i = 0; i < XP; ++i)
            if (tid + i * nth < xtotal) stage(tid + i * nth, xpre[i]);
        for (int idx = tid + XP * nth; idx < xtotal; idx += nth) stage(idx, xload(idx));
        __syncthreads();
    }

    int buf = 0;
    for (int tile = tile0; tile < tile1; ++tile) {
        float acc[TP][2];
#pragma unroll
        for (int p = 0; p < TP; ++p) acc[p][0] = acc[p][1] = 0.f;
        for (int sidx = 0; sidx < ns; ++sidx) {
            const int it = (tile - tile0) * ns + sidx;
            store_item();
            if (it + 1 < items) load_item(it + 1);
            const unsigned char* rowp = slice + n16 * St::RS;
#pragma unroll
            for (int sbl = 0; sbl < SS; ++sbl) {
            const int sb = (st0 + sidx) * SS + sbl;
            uint32_t w[DW];
            gm_lds_slice<KIND>(rowp, sbl, g, w);
            uint32_t u[DW];
            if constexpr (KIND == 2) {
#pragma unroll
                for (int i = 0; i < DW; ++i) u[i] = w[i] ^ 0x80808080u;
            }
            gm_f4 D[TP][2];  // chain 0: sub-block 2g / block 2g; chain 1: 2g+1
#pragma unroll
            for (int p = 0; p < TP; ++p) D[p][0] = D[p][1] = gm_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int r8 = 0; r8 < 8; ++r8) {
                const int c = KIND == 3 ? (r8 >> 1) : (r8 >> 2);
                const int r = KIND == 3 ? (r8 & 1) : (r8 & 3);
                const gm_half8 b = gm_codes<KIND>(w, u, c, r);
                const uint4* grp = achunk + (size_t)(sb * 8 + r8) * M * 8;
#pragma unroll
                for (int p = 0; p < TP; ++p) {
                    const uint4 av = *(aoff[p] >= 0 ? grp + aoff[p] : zero);
                    D[p][r8 >> 2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(gm_half8, av), b,
                                                                           D[p][r8 >> 2], 0, 0, 0);
                }
            }
            // ---- epilogue: per-sub-block scales
            const float* xs = xsum + (size_t)(sb * 8 + 2 * g) * M;  // sub-blocks 2g, 2g+1
            if constexpr (KIND == 3) {
                const float d = gm_lo16(w[0]), dmin = gm_hi16(w[0]);
                const int j0 = 2 * (g & 1);
                const uint32_t A2 = (w[1] >> (8 * j0)) & 0xFFFFu, B2 = (w[2] >> (8 * j0)) & 0xFFFFu,
                               C2 = (w[3] >> (8 * j0)) & 0xFFFFu;
                const uint32_t scp = g < 2 ? (A2 & 0x3F3Fu) : ((C2 & 0x0F0Fu) | ((A2 >> 2) & 0x3030u));
                const uint32_t mp = g < 2 ? (B2 & 0x3F3Fu) : (((C2 >> 4) & 0x0F0Fu) | ((B2 >> 2) & 0x3030u));
                const float a0 = d * (float)(scp & 0xFFu) * 16777216.f, a1 = d * (float)(scp >> 8) * 16777216.f;
                const float b0 = dmin * (float)(mp & 0xFFu), b1 = dmin * (float)(mp >> 8);
#pragma unroll
                for (int p = 0; p < TP; ++p)
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) {
                        const int t = 2 * p + tt;
                        if (t >= M) break;
                        const float s0 = D[p][0][2 * tt] + D[p][0][2 * tt + 1];
                        const float s1 = (D[p][1][2 * tt] + D[p][1][2 * tt + 1]) * 0.0625f;
                        acc[p][tt] += a0 * s0 + a1 * s1 - (b0 * xs[t] + b1 * xs[M + t]);
                    }
            } else {
                const float d0 = gm_lo16(w[0]), d1 = gm_hi16(w[8]);
#pragma unroll
                for (int p = 0; p < TP; ++p)
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) {
                        const int t = 2 * p + tt;
                        if (t >= M) break;
                        const float s0 = D[p][0][2 * tt] + D[p][0][2 * tt + 1];
                        const float s1 = D[p][1][2 * tt] + D[p][1][2 * tt + 1];
                        acc[p][tt] += d0 * fmaf(s0, 16777216.f, -128.f * xs[t]) +
                                      d1 * fmaf(s1, 16777216.f, -128.f * xs[M + t]);
                    }
            }
            }  // sbl
        }  // steps
        // ---- reduce over the 4 k-slot lanes of a row, then over the waves
#pragma unroll
        for (int p = 0; p < TP; ++p)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                float v = acc[p][tt];
                v += __shfl_xor(v, 16, 64);
                v += __shfl_xor(v, 32, 64);
                acc[p][tt] = v;
            }
        float* rb = red + (size_t)buf * WB * 16 * M;
        if (wave < WB && g == 0) {
#pragma unroll
            for (int p = 0; p < TP; ++p)
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    const int t = 2 * p + tt;
                    if (t < M) rb[(wave * M + t) * 16 + n16] = acc[p][tt];
                }
        }
        __syncthreads();
        for (int i = tid; i < 16 * M; i += nth) {  // a 1-wave block has 64 threads for up to 128 outputs
            const int t = i >> 4, nn = i & 15;
            float v = 0.f;
            for (int wv = 0; wv < WB; ++wv) v += rb[(wv * M + t) * 16 + nn];
            const int n = tile * 16 + nn;
            if (n < N) {
                if (!FUSED || f.epi == GM_EPI_STORE) y[(size_t)t * N + n] = v;
                else gm_epilogue(y, t * N + n, n, v, f, epre, tile == tile0 && i == tid && tid < 16);
            }
        }
        buf ^= 1;
    }
}

// ---------------------------------------------------------------------------
// Single-token Q4_K GEMV on int8 MFMA, weights streamed straight into LDS.
//
// Codes: the low nibbles of a Q4_K byte quad become four int8 codes with one
// AND (u & 0x0F0F0F0F); the high nibbles become 16 c - 128 with one
// three-input XOR (u ^ lo ^ 0x80808080), the -128 being undone by starting
// their accumulator at 128 * (sum of the activation parts).
// Activations: each 32-value sub-block j of x is split exactly into three
// int8 parts, x = s_j (p0 + p1 / 128 + p2 / 16384) + O(s_j 2^-15), s_j =
// max|x| / 127, so every product and sum is an exact integer and the result
// keeps about 22 bits of every activation (the reference accumulates in fp32).
// MFMA (v_mfma_i32_16x16x64_i8, block-diagonal A): lane (n = l % 16, g = l / 16)
// holds 16 codes of row n (chunk g of a super-block) as B; A row m = 4g + e is
// non-zero only in the lanes of group g and carries part e, so lane (n, g)
// receives D[4g + e][n] = part-e dot of its own 16 codes for e = 0, 1, 2 at
// once. A and the per-sub-block scales are the same for every tile a wave
// processes, so they live in registers.
// Streaming: one block per CU slot takes a contiguous range of rows, equal for
// every block up to 8 rows, in tiles of 16 rows (the last one may be short; its
// missing rows are not fetched and not stored), so every CU streams the same bytes;
// wave w owns super-blocks SBW*w .. SBW*w+SBW-1 of every tile and
// keeps NB tiles in flight in its ring of LDS slices, filled by
// global_load_lds_dwordx4 (SGPR base + per-lane offset) from inline assembly
// with explicit in-order vmcnt waits: the compiler's own tracking of LDS DMA
// would drain every transfer before each LDS read, and __syncthreads would
// drain them too (lds_barrier waits for LDS only). Waves do not synchronise
// per tile: every lane leaves its partial sum in LDS, and after each group
// of GD_S tiles (one barrier) the block adds the partials of the group and
// stores its rows of y; groups alternate between two LDS areas, so the next
// group's partials never overwrite ones still being added.
// K a multiple of 256 SBW, K <= 4096.
constexpr int GD_S = 4;      // tiles per reduction group
constexpr int GD_NB = 2;     // ring depth: tiles in flight per wave
constexpr int GD_EARLY = 1;  // tiles requested before x is converted (more delay x itself)
typedef int gd_i4 __attribute__((ext_vector_type(4)));

template <int SBW, bool Q8 = false>
struct GdCfg {
    static constexpr int SBB = Q8 ? 272 : 144;  // bytes per 256 values: 8 Q8_0 blocks / 1 Q4_K super-block
    static constexpr int PR = SBB / 16 * SBW;   // 16-byte pieces per row of a wave's column
    static constexpr int NP = 16 * PR;          // pieces per column (16 rows)
    static constexpr int PPL = (NP + 63) / 64;  // transfers per wave and tile (the last one partial)
};

__device__ __forceinline__ gd_i4 gd_lo_codes(uint4 u) {
    return gd_i4{(int)(u.x & 0x0F0F0F0Fu), (int)(u.y & 0x0F0F0F0Fu), (int)(u.z & 0x0F0F0F0Fu), (int)(u.w & 0x0F0F0F0Fu)};
}
__device__ __forceinline__ gd_i4 gd_hi_codes(uint4 u, gd_i4 lo) {
    return gd_i4{(int)(u.x ^ (uint32_t)lo.x ^ 0x80808080u), (int)(u.y ^ (uint32_t)lo.y ^ 0x80808080u),
                 (int)(u.z ^ (uint32_t)lo.z ^ 0x80808080u), (int)(u.w ^ (uint32_t)lo.w ^ 0x80808080u)};
}
__device__ __forceinline__ uint32_t gd_pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) | ((uint32_t)d << 24);
}

// dynamic LDS of k_gemv_q4k_i8: ring, x, partial sums, parts, part sums, scales, x sums
__host__ __device__ constexpr size_t gd_xred_bytes(int K, int WB) {
    return (size_t)K * 4 + (size_t)2 * GD_S * (WB + 1) * 64 * 4;
}
static size_t gd_lds_bytes(int K, int SBW, int NB, bool q8 = false) {
    const int WB = K / (256 * SBW);
    return (size_t)NB * WB * (q8 ? 272 : 144) * SBW * 16 + gd_xred_bytes(K, WB) + 3 * (size_t)K +
           (size_t)K / 32 * 12 + (size_t)K / 32 * 8;
}
constexpr int GD_Q8_KMAX = 2048;  // Q8_0 rows take 1.9x the ring of Q4_K: two tiles fit LDS up to here

constexpr int GD_ATT_MAX = 1024;  // heads x splits of the attention-merge prologue
constexpr int GD_ATT_PT = 8;      // (max, sum) pairs per thread: GD_ATT_MAX / 128 threads

// FUSED: the activation vector is formed by a prologue (RMSNORM / GATED / the
// attention merge, the arithmetic of gm_prologue) straight into the staging
// area instead of being copied, and every output goes through gm_epilogue
// (STORE / ADD / CONV / QKV).
// Q8: the same kernel for Q8_0 rows (34-byte blocks of 32 int8 codes and an fp16 scale, read
// as 8-block groups of 272 bytes in place of a 144-byte super-block): lane (n, g) takes blocks
// 2g and 2g + 1 of a group as 17 dwords, the codes realigned with alignbyte; they are int8
// already, so no nibble or offset work, and no min term.
template <int SBW, int NB, bool FUSED = false, bool Q8 = false, bool SLICED = false>
__global__ void __launch_bounds__(1024 / SBW) k_gemv_q4k_i8(const float* __restrict__ x, const uint8_t* __restrict__ W,
                                                           float* __restrict__ y, int K, int N, size_t rowb,
                                                           int rpb, GmFuse f) {
    using C = GdCfg<SBW, Q8>;
    constexpr int PR = C::PR, NP = C::NP, PPL = C::PPL, SBB = C::SBB;
    if (SLICED) {
        // K slices (rows longer than one block takes): grid row blockIdx.y covers values
        // [blockIdx.y K, (blockIdx.y + 1) K) of each row and writes its partial sums to y + blockIdx.y N
        const int ks0 = blockIdx.y * K;
        x += ks0;
        W += (size_t)(ks0 / 256) * SBB;
        y += (size_t)blockIdx.y * N;
    }
    extern __shared__ __attribute__((aligned(16))) uint4 gd_lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n16 = lane & 15, g = lane >> 4;
    const int WB = blockDim.x >> 6;  // = K / (256 SBW); K / 4 = SBW * blockDim.x float4 pieces of x
    const int K4 = K >> 2;
    // rows [r_begin, r_end) of y, in tiles of 16 rows (the last one may hold fewer)
    const int r_begin = blockIdx.x * rpb, r_end = min(N, r_begin + rpb);
    const int nt = (r_end - r_begin + 15) >> 4;
    uint4* ring = gd_lds;                                   // [NB][WB][NP]
    float4* sx = (float4*)(ring + (size_t)NB * WB * NP);    // [K / 4], until x is converted
    float4* sred = sx + K4;  // [2][GD_S][16 rows][WB + 1] (4 lane groups each; padded against bank conflicts)
    uint32_t* apart = (uint32_t*)((char*)sx + gd_xred_bytes(K, WB));  // [3][K / 4] four int8 parts each
    int* shs = (int*)(apart + 3 * K4);                      // [K / 32][3] sums of the three parts
    float* ssc = (float*)(shs + 3 * (K >> 5));              // [K / 32] part scales s_j
    float* sxs = ssc + (K >> 5);                            // [K / 32] sums of x
    // x: piece tid + j * blockDim.x (contiguous per wave instruction)
    const bool pro = FUSED && f.pro != GM_PRO_NONE;
    const bool att = FUSED && f.pro == GM_PRO_ATTN;
    float4 pv[SBW], pw[SBW];
    float4 ov[SBW][GM_SPR];  // attention merge: this thread's partials of its first GM_SPR splits
    float2 mlr[GD_ATT_PT];   // attention merge: (max, sum) pairs tid, tid + blockDim.x, ...
    if (att) {
        // attention.hip k_attn_combine for all heads: every operand requested before the first tile
        const int S = f.splits, HS = f.H * f.splits;
#pragma unroll
        for (int i = 0; i < GD_ATT_PT; ++i) {
            const int q = tid + i * blockDim.x;
            if (q < HS) {
                const int h = q / S, sp = q - h * S;
                mlr[i] = *(const float2*)(f.ml + (((size_t)(h / f.G) * S + sp) * f.G + h % f.G) * 2);
            }
        }
#pragma unroll
        for (int j = 0; j < SBW; ++j) {
            const int c = 4 * (tid + j * blockDim.x), h = c / f.hd, cc = c - h * f.hd;
            const float* op = f.o_part + ((size_t)(h / f.G) * S * f.G + h % f.G) * f.hd + cc;
#pragma unroll
            for (int sp = 0; sp < GM_SPR; ++sp)
                if (sp < S) ov[j][sp] = *(const float4*)(op + (size_t)sp * f.G * f.hd);
        }
    } else if (!pro) {
#pragma unroll
        for (int j = 0; j < SBW; ++j)
            lds_dma16s(x, (uint32_t)(tid + j * blockDim.x) * 16u, lds_addr(&sx[wave * 64 + j * blockDim.x]));
    } else {
        // prologue operands requested now; the values are formed while the first tile streams in
        const bool emb = FUSED && f.emb != nullptr;
        const int tok = emb ? f.bctl[0] : 0;
        const bool tok_ok = tok >= 0 && tok < f.vocab;
#pragma unroll
        for (int j = 0; j < SBW; ++j) {
            const int idx = tid + j * blockDim.x;
            if (emb) {  // elementwise.hip k_embed_half: the token's fp16 row (zero out of range)
                pv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (tok_ok) {
                    const uint2 h = ((const uint2*)(f.emb + (size_t)tok * K))[idx];
                    pv[j] = make_float4(f16_to_f32((uint16_t)(h.x & 0xFFFF)), f16_to_f32((uint16_t)(h.x >> 16)),
                                        f16_to_f32((uint16_t)(h.y & 0xFFFF)), f16_to_f32((uint16_t)(h.y >> 16)));
                }
                if (blockIdx.x == 0) ((float4*)f.emb_out)[idx] = pv[j];
            } else {
                pv[j] = ((const float4*)x)[idx];
            }
            pw[j] = ((const float4*)f.pw)[idx];
            if (f.pro == GM_PRO_GATED) {
                const float4 z = ((const float4*)f.pz)[idx];
                // mamba.hip k_gated_norm: v = y * silu(z)
                pv[j].x = pv[j].x * (z.x / (1.0f + expf(-z.x)));
                pv[j].y = pv[j].y * (z.y / (1.0f + expf(-z.y)));
                pv[j].z = pv[j].z * (z.z / (1.0f + expf(-z.z)));
                pv[j].w = pv[j].w * (z.w / (1.0f + expf(-z.w)));
            }
        }
    }
    if (FUSED && f.emb != nullptr && blockIdx.x == 0 && tid == 0) decode_alloc_slot(f.bctl);
    // column `wave` of a tile -> ring slice; piece q = PR r + j of row r
    uint32_t voff[PPL];
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
        const int q = lane + 64 * i, r = q / PR, j = q - r * PR;
        voff[i] = (uint32_t)(r * rowb) + wave * (SBB * SBW) + 16 * j;
    }
    // tile it of the block -> ring slice b
    auto dma = [&](int it, int b) {
        uint4* dst = ring + ((size_t)b * WB + wave) * NP;
        const int r0 = r_begin + 16 * it;
        const uint8_t* base = W + (size_t)r0 * rowb;
        if (FUSED && f.w1) {  // weight segments (16-row aligned): rows [n0, n0+n1) from w1, then w2
            if (r0 >= f.n0 + f.n1) base = (const uint8_t*)f.w2 + (size_t)(r0 - f.n0 - f.n1) * rowb;
            else if (r0 >= f.n0) base = (const uint8_t*)f.w1 + (size_t)(r0 - f.n0) * rowb;
        }
        const int nv = r_end - r0;
        if (nv >= 16) {
#pragma unroll
            for (int i = 0; i < PPL; ++i)
                if (NP % 64 == 0 || i + 1 < PPL || lane + 64 * i < NP) lds_dma16s(base, voff[i], lds_addr(dst + 64 * i));
        } else {
            // short tile: the pieces of rows past the range all read the wave's first piece of row
            // r0 (one request per instruction; their outputs are not stored), so every lane still
            // issues every transfer and the wave's transfer count stays the same
#pragma unroll
            for (int i = 0; i < PPL; ++i) {
                const int q = lane + 64 * i;
                if (NP % 64 == 0 || i + 1 < PPL || q < NP) {
                    const int r = q / PR;
                    lds_dma16s(base, r < nv ? voff[i] : (uint32_t)(wave * (SBB * SBW)), lds_addr(dst + 64 * i));
                }
            }
        }
    };
    // the first min(NB, nt) tiles are issued up front: GD_EARLY of them now, the rest after the
    // conversion of x
    const int early = min(GD_EARLY, nt);
    dma(0, 0);
#pragma unroll
    for (int b = 1; b < GD_EARLY; ++b)
        if (b < early) dma(b, b);
    if (att) {
        __shared__ float gd_att[2 * GD_ATT_MAX + 64];  // [H][S] max then split weight, [H][S] sums, [H] 1/L
        const int H = f.H, S = f.splits, HS = H * S;
        float* sm = gd_att;
        float* sl = gd_att + HS;
        float* sinv = gd_att + 2 * HS;
#pragma unroll
        for (int i = 0; i < GD_ATT_PT; ++i) {
            const int q = tid + i * blockDim.x;
            if (q < HS) {
                sm[q] = mlr[i].x;
                sl[q] = mlr[i].y;
            }
        }
        __syncthreads();
        if (tid < H) {
            float Mx = -INFINITY;
            for (int sp = 0; sp < S; ++sp)
                if (sl[tid * S + sp] > 0.f) Mx = fmaxf(Mx, sm[tid * S + sp]);
            float L = 0.f;
            for (int sp = 0; sp < S; ++sp) {
                const float l = sl[tid * S + sp];
                const float w = l > 0.f ? expf(sm[tid * S + sp] - Mx) : 0.f;
                sm[tid * S + sp] = w;
                L += w * l;
            }
            sinv[tid] = L > 0.f ? 1.0f / L : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < SBW; ++j) {
            const int idx = tid + j * blockDim.x, c = 4 * idx, h = c / f.hd, cc = c - h * f.hd;
            const float* op = f.o_part + ((size_t)(h / f.G) * S * f.G + h % f.G) * f.hd + cc;
            float a[4] = {0.f, 0.f, 0.f, 0.f};
            // splits in order; an empty split (weight 0) has no partials written and is skipped
#pragma unroll
            for (int sp = 0; sp < GM_SPR; ++sp) {
                const float w = sp < S ? sm[h * S + sp] : 0.f;
                if (w != 0.f) {
                    a[0] += w * ov[j][sp].x;
                    a[1] += w * ov[j][sp].y;
                    a[2] += w * ov[j][sp].z;
                    a[3] += w * ov[j][sp].w;
                }
            }
            for (int sp = GM_SPR; sp < S; ++sp) {
                const float w = sm[h * S + sp];
                if (w != 0.f) {
                    const float4 o4 = *(const float4*)(op + (size_t)sp * f.G * f.hd);
                    a[0] += w * o4.x;
                    a[1] += w * o4.y;
                    a[2] += w * o4.z;
                    a[3] += w * o4.w;
                }
            }
            const float iv = sinv[h];
            sx[idx] = make_float4(a[0] * iv, a[1] * iv, a[2] * iv, a[3] * iv);
        }
    } else if (pro) {
        // elementwise.hip k_rmsnorm / mamba.hip k_gated_norm: double sum of squares, x * inv * w
        __shared__ double gd_red[16];
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < SBW; ++j)
            ss += (double)pv[j].x * pv[j].x + (double)pv[j].y * pv[j].y + (double)pv[j].z * pv[j].z +
                  (double)pv[j].w * pv[j].w;
        const double tot = gm_block_sum_dpp(ss, gd_red);
        float inv;
        if (f.pro == GM_PRO_GATED) {
            inv = 1.0f / sqrtf((float)(tot / (double)K) + f.eps);
        } else {
            const double invd = 1.0 / sqrt(tot / (double)K + (double)f.eps);
            inv = isfinite(invd) ? (float)invd : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < SBW; ++j) {
            const int idx = tid + j * blockDim.x;
            sx[idx] = make_float4(pv[j].x * inv * pw[j].x, pv[j].y * inv * pw[j].y, pv[j].z * inv * pw[j].z,
                                  pv[j].w * inv * pw[j].w);
        }
    }
    // ---- x -> three int8 parts per value; scale, x sum and part sums per 32 values (8 threads each)
    // With one super-block per wave, a wave converts exactly the 256 values its own A operands
    // take (its lanes staged them), so no block barrier is needed before the tiles.
    constexpr bool WAVE_LOCAL = SBW == 1;
    lds_dma_wait<PPL>(early);  // x landed (the early tiles in flight)
    if (WAVE_LOCAL) lds_wait_lgkm(); else lds_barrier();
#pragma unroll
    for (int jj = 0; jj < SBW; ++jj) {
        const int idx = tid + jj * blockDim.x;
        const float4 v4 = sx[idx];
        float m = fmaxf(fmaxf(fabsf(v4.x), fabsf(v4.y)), fmaxf(fabsf(v4.z), fabsf(v4.w)));
        float sum = (v4.x + v4.y) + (v4.z + v4.w);
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) {
            m = fmaxf(m, __shfl_xor(m, o, 64));
            sum += __shfl_xor(sum, o, 64);
        }
        const float inv = m > 0.f ? 127.f / m : 0.f;
        int p[3][4];
        const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float t = vv[q] * inv;
            const float a0 = rintf(t);
            const float r1 = (t - a0) * 128.f;
            const float a1 = rintf(r1);
            const float a2 = rintf((r1 - a1) * 128.f);
            p[0][q] = (int)a0; p[1][q] = (int)a1; p[2][q] = (int)a2;
        }
        int ps[3];
#pragma unroll
        for (int e = 0; e < 3; ++e) {
            apart[e * K4 + idx] = gd_pack4(p[e][0], p[e][1], p[e][2], p[e][3]);
            ps[e] = p[e][0] + p[e][1] + p[e][2] + p[e][3];
#pragma unroll
            for (int o = 1; o < 8; o <<= 1) ps[e] += __shfl_xor(ps[e], o, 64);
        }
        if ((idx & 7) == 0) {
            const int sbk = idx >> 3;
            ssc[sbk] = m * (1.f / 127.f);
            sxs[sbk] = sum;
            shs[3 * sbk] = ps[0];
            shs[3 * sbk + 1] = ps[1];
            shs[3 * sbk + 2] = ps[2];
        }
    }
    // the rest of the ring
#pragma unroll
    for (int b = GD_EARLY; b < NB; ++b)
        if (b < nt) dma(b, b);
    if (WAVE_LOCAL) lds_wait_lgkm(); else lds_barrier();
    // A operands of this wave's super-blocks (rows m = 4g + e of group g), scales, high-nibble offsets
    gd_i4 A[SBW][2][2], hinit[SBW];
    float s_lo[SBW], s_hi[SBW], xs_lo[SBW], xs_hi[SBW];
    {
        const int e = n16 & 3;
        const bool on = (n16 >> 2) == g && e < 3;
#pragma unroll
        for (int sbl = 0; sbl < SBW; ++sbl) {
            const int sb = wave * SBW + sbl;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 2; ++r)
                    A[sbl][h][r] = on ? *(const gd_i4*)&apart[e * K4 + ((sb * 256 + 64 * g + 32 * h + 16 * r) >> 2)]
                                      : gd_i4{0, 0, 0, 0};
            const int jl = sb * 8 + 2 * g, jh = jl + 1;
            // parts combine as 16384 p0 + 128 p1 + p2 (exact in int32), hence the 2^-14
            s_lo[sbl] = ssc[jl] * (1.f / 16384.f);
            s_hi[sbl] = ssc[jh] * (1.f / 16384.f);
            xs_lo[sbl] = sxs[jl];
            xs_hi[sbl] = sxs[jh];
            // high-nibble codes are 16 c - 128: their accumulator starts at 128 * (part sums)
            hinit[sbl] = gd_i4{128 * shs[3 * jh], 128 * shs[3 * jh + 1], 128 * shs[3 * jh + 2], 0};
        }
    }
    int b = 0;
    for (int it = 0; it < nt; ++it) {
        // tiles issued after this one: it+1 .. min(it+NB-1, nt-1)
        const int ahead = min(NB - 1, nt - 1 - it);
        lds_dma_wait<PPL>(ahead);
        const unsigned char* rowp = (const unsigned char*)(ring + ((size_t)b * WB + wave) * NP) + n16 * (SBB * SBW);
        uint4 hd[SBW], qa[SBW], qb[SBW];
        uint32_t q8w[Q8 ? SBW : 1][17];
        if constexpr (Q8) {
#pragma unroll
            for (int sbl = 0; sbl < SBW; ++sbl) {
                const uint32_t* rp = (const uint32_t*)(rowp + SBB * sbl + 68 * g);  // blocks 2g, 2g + 1
#pragma unroll
                for (int k = 0; k < 17; ++k) q8w[sbl][k] = rp[k];
            }
        } else {
#pragma unroll
            for (int sbl = 0; sbl < SBW; ++sbl) {
                hd[sbl] = *(const uint4*)(rowp + 144 * sbl);
                qa[sbl] = *(const uint4*)(rowp + 144 * sbl + 16 + 32 * g);
                qb[sbl] = *(const uint4*)(rowp + 144 * sbl + 32 + 32 * g);
            }
        }
        if (it + NB < nt) {  // slice read: refill it
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            dma(it + NB, b);
        }
        float acc = 0.f;
        if constexpr (Q8) {
#pragma unroll
            for (int sbl = 0; sbl < SBW; ++sbl) {
                const uint32_t* w = q8w[sbl];
                // block 2g: d in bytes 0-1, codes in bytes 2-33; block 2g + 1: d in 34-35, codes 36-67
                gd_i4 c0[2], c1[2];
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    c0[r] = gd_i4{(int)__builtin_amdgcn_alignbyte(w[4 * r + 1], w[4 * r], 2),
                                  (int)__builtin_amdgcn_alignbyte(w[4 * r + 2], w[4 * r + 1], 2),
                                  (int)__builtin_amdgcn_alignbyte(w[4 * r + 3], w[4 * r + 2], 2),
                                  (int)__builtin_amdgcn_alignbyte(w[4 * r + 4], w[4 * r + 3], 2)};
                    c1[r] = gd_i4{(int)w[9 + 4 * r], (int)w[10 + 4 * r], (int)w[11 + 4 * r], (int)w[12 + 4 * r]};
                }
                gd_i4 Dl = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[sbl][0][0], c0[0], gd_i4{0, 0, 0, 0}, 0, 0, 0);
                gd_i4 Dh = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[sbl][1][0], c1[0], gd_i4{0, 0, 0, 0}, 0, 0, 0);
                Dl = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[sbl][0][1], c0[1], Dl, 0, 0, 0);
                Dh = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[sbl][1][1], c1[1], Dh, 0, 0, 0);
                const float d0 = gm_lo16(w[0]), d1 = gm_hi16(w[8]);
                // |D0| <= 32 * 127 * 127 < 2^24: each part sum is exact in fp32, and so are the
                // power-of-two weights of 16384 D0 + 128 D1 + D2 (their sum rounds once or twice)
                const float il = (float)Dl[0] * 16384.f + (float)Dl[1] * 128.f + (float)Dl[2];
                const float ih = (float)Dh[0] * 16384.f + (float)Dh[1] * 128.f + (float)Dh[2];
                acc += d0 * s_lo[sbl] * il + d1 * s_hi[sbl] * ih;
            }
        } else
#pragma unroll
        for (int sbl = 0; sbl < SBW; ++sbl) {
            const gd_i4 la = gd_lo_codes(qa[sbl]), lb = gd_lo_codes(qb[sbl]);
            gd_i4 Dl = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[sbl][0][0], la, gd_i4{0, 0, 0, 0}, 0, 0, 0);
            gd_i4 Dh = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[sbl][1][0], gd_hi_codes(qa[sbl], la), hinit[sbl], 0, 0, 0);
            Dl = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[sbl][0][1], lb, Dl, 0, 0, 0);
            Dh = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[sbl][1][1], gd_hi_codes(qb[sbl], lb), Dh, 0, 0, 0);
            // scales of sub-blocks 2g (low nibbles) and 2g+1 (high nibbles)
            const uint4 h4 = hd[sbl];
            const float d = gm_lo16(h4.x), dmin = gm_hi16(h4.x);
            const int j0 = 2 * (g & 1);
            const uint32_t A2 = (h4.y >> (8 * j0)) & 0xFFFFu, B2 = (h4.z >> (8 * j0)) & 0xFFFFu,
                           C2 = (h4.w >> (8 * j0)) & 0xFFFFu;
            const uint32_t scp = g < 2 ? (A2 & 0x3F3Fu) : ((C2 & 0x0F0Fu) | ((A2 >> 2) & 0x3030u));
            const uint32_t mp = g < 2 ? (B2 & 0x3F3Fu) : (((C2 >> 4) & 0x0F0Fu) | ((B2 >> 2) & 0x3030u));
            // |D0| <= 32 * 15 * 127, |D1|, |D2| <= 32 * 15 * 64: 16384 D0 + 128 D1 + D2 fits in int32;
            // the high-nibble sums are 16x (exact), so their weights are 1024, 8 and 1/16
            const int il = Dl[0] * 16384 + Dl[1] * 128 + Dl[2];
            const int ih = Dh[0] * 1024 + Dh[1] * 8 + (Dh[2] >> 4);
            acc += d * ((float)(scp & 0xFFu) * s_lo[sbl] * (float)il + (float)(scp >> 8) * s_hi[sbl] * (float)ih) -
                   dmin * ((float)(mp & 0xFFu) * xs_lo[sbl] + (float)(mp >> 8) * xs_hi[sbl]);
        }
        // partial of (row n16, lane group g) -> slot; a group of GD_S tiles is added up at once
        const int slot = it & (GD_S - 1), grp = (it / GD_S) & 1;
        float4* red = sred + (size_t)(grp * GD_S + slot) * 16 * (WB + 1);
        ((float*)&red[n16 * (WB + 1) + wave])[g] = acc;
        if (slot == GD_S - 1 || it + 1 >= nt) {
            lds_barrier();
            // thread (output o, wave w = tid % 16) adds w's four lane groups; 16 lanes add the waves
            const int w = tid & 15;
            for (int o = tid >> 4; o < 16 * (slot + 1); o += blockDim.x >> 4) {  // uniform per 16 lanes
                const int tl = o >> 4, row = o & 15;
                float v = 0.f;
                if (w < WB) {
                    const float4 p4 = sred[(size_t)(grp * GD_S + tl) * 16 * (WB + 1) + row * (WB + 1) + w];
                    v = (p4.x + p4.y) + (p4.z + p4.w);
                }
                v += __shfl_xor(v, 1, 64);
                v += __shfl_xor(v, 2, 64);
                v += __shfl_xor(v, 4, 64);
                v += __shfl_xor(v, 8, 64);
                const int n = r_begin + 16 * (it - (slot - tl)) + row;
                if (w == 0 && n < r_end) {
                    if constexpr (FUSED) gm_epilogue(y, n, n, v, f, GmEpiPre{}, false);
                    else y[n] = v;
                }
            }
        }
        b = b + 1 == NB ? 0 : b + 1;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no transfer into LDS outlives the block
}

// dynamic LDS budget: 160 KB per workgroup less a reserve for the static
// arrays of the fusion prologue
constexpr size_t GM_LDS_MAX = 160 * 1024 - 512;

template <int KIND, int SS>
static size_t gm_lds_bytes(int K, int M, int WB, bool pro) {
    const size_t nsb = K / 256;
    return 16 + nsb * 8 * M * 8 * 16 + nsb * 8 * M * 4 + 2 * (size_t)WB * 16 * M * 4 +
           (size_t)WB * GmStep<KIND, SS>::BYTES + (pro ? (size_t)K * 4 : 0);
}

// Waves per block and steps per wave: as many waves as there are steps (up
// to 16), fewer if the block's LDS would not fit. 0 if nothing fits.
template <int KIND, int SS>
static int gm_split(int K, int M, bool pro, int& WB, int& spw) {
    const int nsteps = K / 256 / SS;
    const int wcap = M <= 2 ? 16 : 8;
    const int wmax = wcap;
    for (int wb = nsteps < wmax ? nsteps : wmax; wb >= 1; --wb) {
        spw = (nsteps + wb - 1) / wb;
        WB = (nsteps + spw - 1) / spw;
        if (gm_lds_bytes<KIND, SS>(K, M, WB, pro) <= GM_LDS_MAX) return 1;
    }
    return 0;
}

template <int KIND, int TP, int SS, bool FUSED>
static int gm_launch(const float* x, const void* w, float* y, int M, int K, int N, const GmFuse& f) {
    auto kern = k_gemv_mfma<KIND, TP, SS, FUSED>;
    const bool pro = f.pro != GM_PRO_NONE;
    int WB, spw;
    if (!gm_split<KIND, SS>(K, M, pro, WB, spw))
        return fail(GH_EINVAL, "gemv_mfma: K=%d M=%d does not fit LDS", K, M);
    const size_t lds = gm_lds_bytes<KIND, SS>(K, M, WB, pro);
    static bool attr_set = false;
    if (!attr_set) {
        GH_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)GM_LDS_MAX));
        attr_set = true;
    }
    const int ntiles = (N + 15) / 16;
    const int wpc = 16;  // waves per CU
    int bpc = wpc / WB;
    if (bpc < 1) bpc = 1;
    const int by_lds = (int)(GM_LDS_MAX / lds);
    if (bpc > by_lds) bpc = by_lds;
    int blocks = num_cus() * bpc;
    if (blocks > ntiles) blocks = ntiles;
    const int tpb = (ntiles + blocks - 1) / blocks;
    blocks = (ntiles + tpb - 1) / tpb;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * WB), lds, stream(), x, (const uint8_t*)w, y, M, K, N,
                       row_bytes(KIND, K), WB, tpb, spw, f);
    GH_LAUNCHED("k_gemv_mfma");
    return GH_OK;
}

// Q4_K moves two super-blocks per step when K allows, Q8_0 one
template <int KIND>
static bool gm_fits(int K, int M, bool pro) {
    int WB, spw;
    if constexpr (KIND == 3) {
        if ((K / 256) % 2 == 0) return gm_split<KIND, 2>(K, M, pro, WB, spw);
    }
    return gm_split<KIND, 1>(K, M, pro, WB, spw);
}

template <int KIND, int TP, bool FUSED = false>
static int gm_ss(const float* x, const void* w, float* y, int M, int K, int N, const GmFuse& f = GmFuse()) {
    if constexpr (KIND == 3) {
        if ((K / 256) % 2 == 0) return gm_launch<KIND, TP, 2, FUSED>(x, w, y, M, K, N, f);
    }
    return gm_launch<KIND, TP, 1, FUSED>(x, w, y, M, K, N, f);
}

template <int KIND>
static int gm_kind(const float* x, const void* w, float* y, int M, int K, int N) {
    const int TP = (M + 1) / 2;
    if (TP == 1) return gm_ss<KIND, 1>(x, w, y, M, K, N);
    if (TP == 2) return gm_ss<KIND, 2>(x, w, y, M, K, N);
    if (TP == 3) return gm_ss<KIND, 3>(x, w, y, M, K, N);
    return gm_ss<KIND, 4>(x, w, y, M, K, N);
}

int g8_sum_launch(const float* part, float* y, int n, int S);  // gemv8.hip

// S > 1 (plain form only): each row is cut into S equal K slices on the grid's second
// dimension; the partial sums go to a workspace and are added in slice order.
template <int SBW, int NB, bool FUSED = false, bool Q8 = false, bool SLICED = false>
static int gd_launch(const float* x, const uint8_t* w, float* y, int Kfull, int N, const GmFuse& f = GmFuse{},
                     int S = 1) {
    static int configured = 0;
    static int per_cu[17];  // resident blocks per CU by K / (256 SBW)
    const int K = Kfull / S;
    if (S < 1 || (!SLICED && S > 1) || (FUSED && SLICED) || Kfull % S != 0 || K > (Q8 ? GD_Q8_KMAX : 4096) ||
        K % (256 * SBW) != 0)
        return fail(GH_EUNSUPPORTED, "k_gemv_q4k_i8: K=%d in %d slices", Kfull, S);
    const size_t lds = gd_lds_bytes(K, SBW, NB, Q8);
    if (!configured) {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemv_q4k_i8<SBW, NB, FUSED, Q8, SLICED>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)gd_lds_bytes(Q8 ? GD_Q8_KMAX : 4096, SBW, NB, Q8));
        if (e != hipSuccess) return fail(GH_EHIP, "k_gemv_q4k_i8 LDS attribute: %s", hipGetErrorString(e));
        configured = 1;
    }
    const int wb = K / (256 * SBW);
    if (!per_cu[wb]) {
        int nb = 0;
        hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_gemv_q4k_i8<SBW, NB, FUSED, Q8, SLICED>, 64 * wb, lds);
        per_cu[wb] = e == hipSuccess && nb > 0 ? nb : 1;
    }
    // contiguous row ranges, equal up to 8 rows (16 with weight segments): every block
    // streams the same number of bytes, so no CU runs a tile more than the others
    const int slots = per_cu[wb] * num_cus() / S;
    const int align = FUSED && f.w1 ? 16 : 8;
    const int rpb = ((N + slots - 1) / slots + align - 1) / align * align;
    const int blocks = (N + rpb - 1) / rpb;
    float* out = y;
    if (S > 1) {
        out = (float*)workspace(WS_GEMM_PART, (size_t)S * N * 4);
        if (!out) return fail(GH_ENOMEM, "k_gemv_q4k_i8: workspace");
    }
    hipLaunchKernelGGL((k_gemv_q4k_i8<SBW, NB, FUSED, Q8, SLICED>), dim3(blocks, S), dim3(64 * wb), lds, stream(), x, w, out,
                       K, N, row_bytes(Q8 ? 2 : 3, Kfull), rpb, f);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(GH_EHIP, "launch of k_gemv_q4k_i8 failed: %s", hipGetErrorString(e));
    return S > 1 ? g8_sum_launch(out, y, N, S) : GH_OK;
}

// variant 1: one super-block per wave; 2: two super-blocks per wave (needs K % 512 == 0)
static int gemv_q4k_i8(const float* x, const uint8_t* w, float* y, int K, int N, int variant) {
    if (variant == 2 && K % 512 == 0) return gd_launch<2, GD_NB>(x, w, y, K, N);
    return gd_launch<1, GD_NB>(x, w, y, K, N);
}

// Returns 1 if handled (Q4_K / Q8_0, 1 <= M <= 8, K a multiple of 256).
// Token groups whose activations do not fit LDS together are run as
// separate launches over the same weights.
int gemv8_dispatch(const float* x, const void* w, float* y, int M, int K, int N, int kind, int* rc);  // gemv8.hip

int gemv_mfma_dispatch(const float* x, const void* w, float* y, int M, int K, int N, int kind, int* rc) {
    if (gemv8_dispatch(x, w, y, M, K, N, kind, rc)) return 1;
    if (M == 1 && kind == 3 && K % 256 == 0 && K <= 4096) {
        *rc = gemv_q4k_i8(x, (const uint8_t*)w, y, K, N, 1);
        return 1;
    }
    if (M == 1 && kind == 3 && K % 256 == 0 && K > 4096) {
        // longer rows: the smallest count of equal K slices that each fit a block
        for (int S = 2; S <= 8; ++S)
            if ((K / 256) % S == 0 && K / S <= 4096) {
                *rc = gd_launch<1, GD_NB, false, false, true>(x, (const uint8_t*)w, y, K, N, GmFuse{}, S);
                return 1;
            }
    }
    if (M == 1 && kind == 2 && K % 256 == 0 && K <= GD_Q8_KMAX && ((uintptr_t)w & 15) == 0) {
        *rc = gd_launch<1, GD_NB, false, true>(x, (const uint8_t*)w, y, K, N);
        return 1;
    }
    if (M == 1 && kind == 2 && K % 256 == 0 && K > GD_Q8_KMAX && ((uintptr_t)w & 15) == 0) {
        for (int S = 2; S <= 8; ++S)
            if ((K / 256) % S == 0 && K / S <= GD_Q8_KMAX) {
                *rc = gd_launch<1, GD_NB, false, true, true>(x, (const uint8_t*)w, y, K, N, GmFuse{}, S);
                return 1;
            }
    }
    if ((kind != 2 && kind != 3) || M < 1 || M > 8 || K % 256 != 0) return 0;
    int mc = M;
    while (mc >= 1 && !(kind == 3 ? gm_fits<3>(K, mc, false) : gm_fits<2>(K, mc, false))) --mc;
    if (mc < 1) return 0;
    // y is [M][N]; a token group [t0, t0+mc) is a contiguous slice of x and y
    for (int t0 = 0; t0 < M; t0 += mc) {
        const int m = M - t0 < mc ? M - t0 : mc;
        const float* xs = x + (size_t)t0 * K;
        float* ys = y + (size_t)t0 * N;
        *rc = kind == 3 ? gm_kind<3>(xs, w, ys, m, K, N) : gm_kind<2>(xs, w, ys, m, K, N);
        if (*rc) return 1;
    }
    return 1;
}

int gemv_fused(const float* x, const void* w, float* y, int K, int N, int kind, const GmFuse& f) {
    if ((kind != 2 && kind != 3) || K % 256 != 0) return fail(GH_EUNSUPPORTED, "gemv_fused: kind %d K=%d", kind, K);
    const bool att_ok = f.pro != GM_PRO_ATTN || (f.H * f.hd == K && f.hd % 4 == 0 && f.H <= 64 &&
                                                 f.H * f.splits <= GD_ATT_PT * (K / 256) * 64 &&
                                                 f.H * f.splits <= GD_ATT_MAX && (((uintptr_t)f.o_part) & 15) == 0);
    const bool emb_ok = !f.emb || (f.pro == GM_PRO_RMSNORM && f.bctl && f.emb_out && f.vocab > 0 &&
                                   (((uintptr_t)f.emb | (uintptr_t)f.emb_out) & 15) == 0);
    const bool i8_ok = (kind == 3 ? K <= 4096 : K <= GD_Q8_KMAX) && att_ok && emb_ok &&
                       (!f.w1 || (f.n0 % 16 == 0 && f.n1 % 16 == 0)) &&
                       (((uintptr_t)x | (uintptr_t)f.pw | (uintptr_t)f.pz | (uintptr_t)w | (uintptr_t)f.w1 |
                         (uintptr_t)f.w2) & 15) == 0;
    if (i8_ok) {
        // norm prologue, weight segments, residual / conv / K-V cache epilogue on the int8-MFMA
        // streaming GEMV
        return kind == 3 ? gd_launch<1, GD_NB, true>(x, (const uint8_t*)w, y, K, N, f)
                         : gd_launch<1, GD_NB, true, true>(x, (const uint8_t*)w, y, K, N, f);
    }
    // the folded step start needs the norm prologue and aligned rows (no launch made otherwise)
    if (f.emb && !emb_ok) return GH_EUNSUPPORTED;
    if (f.w1 && (f.n0 % 16 || f.n1 % 16)) return fail(GH_EINVAL, "gemv_fused: segments must be multiples of 16 rows");
    if (f.pro == GM_PRO_ATTN && (f.splits > 64 || f.H * f.hd != K))
        return fail(GH_EUNSUPPORTED, "gemv_fused: attention merge of %d splits", f.splits);
    if (!(kind == 3 ? gm_fits<3>(K, 1, f.pro != GM_PRO_NONE) : gm_fits<2>(K, 1, f.pro != GM_PRO_NONE)))
        return fail(GH_EUNSUPPORTED, "gemv_fused: K=%d does not fit LDS", K);
    return kind == 3 ? gm_ss<3, 1, true>(x, w, y, 1, K, N, f) : gm_ss<2, 1, true>(x, w, y, 1, K, N, f);
}

}  // namespace gh
