// Q4_K / Q8_0 GEMV for 2..8 tokens (batched decode, k_gemv8): y[t][n] = sum_k x[t][k] w[n][k],
// linear_forward_q4 (core/ops.cpp:360-408) at M <= 8.
//
// The weights are dequantised to fp16 in registers (the reference's CPU path
// rounds every dequantised weight to fp16, core/ops.cpp:304-338) and
// multiplied on the matrix cores as a dense 16-row GEMM: A row 2t + e is
// token t's activation part e (x = hi + lo, two fp16 numbers, so the products
// keep ~22 bits of each activation), so one v_mfma_f32_16x16x32_f16 per
// 32-value sub-block covers all 8 tokens of 16 weight rows. Lane (n, g) holds
// B = 8 weights of row n (values 8g..8g+7 of the sub-block) and receives
// D[4g..4g+3][n] = the hi and lo parts of tokens 2g and 2g+1.
//
// Work split: a tile is 16 rows; wave w of a block owns super-blocks
// SBW w .. SBW w + SBW - 1 of every tile (its A operands stay in registers
// for the whole launch); blocks are persistent and walk tiles b, b + G, ...
// whose bytes arrive in LDS by direct transfers, R tiles ahead (below).
// Weight values: (1024 + q) is made an fp16 number by one v_and_or_b32 per
// pair of codes, then q d sc - dmin m = (1024 + q) s + nb with s = d sc,
// nb = -(1024 s + dmin m), rounded to fp16.
//
// Q8_0 (k_gemv8<SBW, true>): 256 values are 8 blocks of 34 bytes (a 272-byte group); lane (n, g)
// reads blocks 2g and 2g + 1 of its row as 17 dwords (68 bytes, 4-byte aligned) and MFMA
// k-step m (0..7) takes codes 8 (m % 4) .. + 7 of block 2g + m / 4 from every lane, the A
// operands permuted to match. A code becomes an fp16 integer exactly (0x6400 | (q + 128),
// minus 1152) and one fp16 multiply by the block scale rounds q d once: the fp16 weight the
// reference's quant_materialize forms.
#include <stdlib.h>

#include "gemm_tile.h"
#include "lds_dma.h"

namespace gh {

typedef float g8_f4 __attribute__((ext_vector_type(4)));

// Weight tiles stream into LDS by direct transfers (global_load_lds_dwordx4 from inline
// assembly: the compiler neither moves them nor waits for them; the loop waits with explicit
// vmcnt counts, in issue order). A wave's part of a tile is 16 rows x SB bytes (its SBW
// super-blocks / 272-byte groups of each row), cut into 16-byte pieces; piece c = 64 i + lane
// (row c / (SB / 16)) is transfer i of the lane, so every transfer instruction reads about
// 1 KB of consecutive row segments and lands contiguous in LDS. Each wave keeps its next
// tiles in flight in a private ring of R slots; a block's tiles are b, b + G, b + 2G, ...
// A slot's bytes move to registers before its refill is requested, so the refill is in
// flight while the tile is decoded and multiplied. The waves' partial sums of two tiles meet
// in LDS (two such areas alternate) and are added in wave order after one barrier.
constexpr int G8_LDS = 160 * 1024;
constexpr int G8_RED = 2 * 2 * 8 * 8 * 16 * 4;  // [area][tile][wave][token][row] floats
template <int SB>
struct G8Geo {
    static constexpr int CH = SB / 16;           // pieces per row
    static constexpr int NCH = 16 * CH;          // pieces per wave tile (= uint4 per ring slot)
    static constexpr int LPL = (NCH + 63) / 64;  // transfers per lane per tile (the last one partial)
    static constexpr int R0 = (G8_LDS - G8_RED - 2048) / (8 * NCH * 16);
    static constexpr int R = R0 > 4 ? 4 : R0;  // ring slots (LDS of 8 waves)
    static_assert(R >= 2, "gemv8: a wave tile does not fit two LDS slots");
};

// Transfers of tile `tile` (16 rows from row 16 tile, bytes [col0, col0 + SB) of each row)
// into `slot`; rows past N repeat row N - 1 (their sums are not stored). Every lane with a
// piece issues every transfer, so a tile is LPL transfers of the wave's count.
template <int SB>
__device__ __forceinline__ void g8_issue(const uint8_t* W, size_t rowb, int N, int tile, size_t col0, uint4* slot,
                                         int lane) {
    using Gq = G8Geo<SB>;
    const uintptr_t bp = (uintptr_t)(W + (size_t)tile * 16 * rowb + col0);  // wave-uniform: into SGPRs
    // (readfirstlane returns int: each half goes through uint32_t, or the low half sign-extends)
    const uint32_t bhi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(bp >> 32));
    const uint32_t blo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)bp);
    const uint8_t* base = (const uint8_t*)(((uintptr_t)bhi << 32) | (uintptr_t)blo);
    const int rmax = N - 1 - tile * 16;
#pragma unroll
    for (int i = 0; i < Gq::LPL; ++i) {
        const int c = 64 * i + lane;
        if (Gq::NCH % 64 == 0 || i + 1 < Gq::LPL || c < Gq::NCH) {
            int rr = c / Gq::CH;
            const int pc = c - rr * Gq::CH;
            rr = rr < rmax ? rr : rmax;
            lds_dma16s(base, (uint32_t)(rr * rowb) + 16u * pc, lds_addr(slot + 64 * i));
        }
    }
}

// codes 4i .. 4i + 3 of a dword -> two packed fp16 pairs (q0, q1), (q2, q3), exact
__device__ __forceinline__ void g8_q8_pairs(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const uint32_t u = w ^ 0x80808080u;  // q + 128 as unsigned bytes
    lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
}
typedef _Float16 g8_h2 __attribute__((ext_vector_type(2)));

// One tile's bytes of this lane: Q4_K, per super-block the 16-byte header and the four
// 8-byte code runs 32 p + 8 g; Q8_0, per 272-byte group blocks 2g and 2g + 1 (17 dwords).
template <int SBW, bool Q8>
struct G8Raw {
    uint32_t w[SBW][Q8 ? 17 : 12];
};

// K slices: grid row blockIdx.y takes values [blockIdx.y K, (blockIdx.y + 1) K) of rows of
// ldx activations and writes its partial sums to y + blockIdx.y M N.
template <int SBW, bool Q8>
__global__ void __launch_bounds__(512) k_gemv8(const float* __restrict__ x, const uint8_t* __restrict__ W,
                                                float* __restrict__ y, int M, int K, int N, size_t rowb, int ldx) {
    constexpr int GB = Q8 ? 272 : 144;  // bytes per 256 values
    using Gq = G8Geo<SBW * GB>;
    const int ks0 = blockIdx.y * K;  // first value of this slice
    x += ks0;
    W += (size_t)(ks0 / 256) * GB;
    y += (size_t)blockIdx.y * M * N;
    __shared__ float red[2][2][8][8][16];  // [area][tile][wave][token][row]
    __shared__ uint4 ring[8][Gq::R][Gq::NCH];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, WB = blockDim.x >> 6;
    const int n16 = lane & 15, g = lane >> 4;
    const int ntiles = (N + 15) >> 4;
    const int G = (int)gridDim.x;
    const int nt = (int)blockIdx.x < ntiles ? (ntiles - (int)blockIdx.x + G - 1) / G : 0;
    const size_t col0 = (size_t)(wave * SBW) * GB;
    // the first tile is requested before the activations are converted (the compiler's wait
    // for their loads counts the earlier transfers too), the next R - 1 after
    if (nt > 0) g8_issue<SBW * GB>(W, rowb, N, blockIdx.x, col0, ring[wave][0], lane);
    // ---- A operands of this wave's super-blocks / groups: row n16 = token n16/2, part n16%2
    // (x = hi + lo, two fp16 numbers). Q4_K k-step j takes values 32 j + 8 g + {0,2,1,3,4,6,5,7}
    // (the order the codes come out of a dword); Q8_0 k-step m takes values
    // 32 (2g + m/4) + 8 (m%4) + 0..7 of the group.
    f16x8 A[SBW][8];
    {
        const int t = n16 >> 1, part = n16 & 1;
        const bool live = t < M;
#pragma unroll
        for (int s = 0; s < SBW; ++s) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int k0 = (wave * SBW + s) * 256 + (Q8 ? 32 * (2 * g + (j >> 2)) + 8 * (j & 3) : 8 * g + 32 * j);
                float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
                if (live) {
                    const float4* p = (const float4*)(x + (size_t)t * ldx + k0);
                    v0 = p[0];
                    v1 = p[1];
                }
                float v[8];
                if (Q8) {
                    v[0] = v0.x, v[1] = v0.y, v[2] = v0.z, v[3] = v0.w, v[4] = v1.x, v[5] = v1.y, v[6] = v1.z, v[7] = v1.w;
                } else {
                    v[0] = v0.x, v[1] = v0.z, v[2] = v0.y, v[3] = v0.w, v[4] = v1.x, v[5] = v1.z, v[6] = v1.y, v[7] = v1.w;
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const _Float16 hi = (_Float16)v[e];
                    A[s][j][e] = part ? (_Float16)(v[e] - (float)hi) : hi;
                }
            }
        }
    }
    // the A operands are complete before the next transfers go out (the compiler's wait for
    // the activation loads would otherwise come after them and drain them too)
#pragma unroll
    for (int s = 0; s < SBW; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) asm volatile("" ::"v"(A[s][j]));
    for (int k = 1; k < Gq::R && k < nt; ++k)
        g8_issue<SBW * GB>(W, rowb, N, blockIdx.x + k * G, col0, ring[wave][k], lane);
    uint32_t magic = 0x64006400u;
    asm volatile("" : "+v"(magic));
    const g8_h2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
    for (int k = 0; k < nt; ++k) {
        const int slot = k % Gq::R;
        const int ahead = nt - 1 - k < Gq::R - 1 ? nt - 1 - k : Gq::R - 1;  // tiles requested after this one
        lds_dma_wait<Gq::LPL>(ahead);
        G8Raw<SBW, Q8> raw;
        {
            const uint32_t* lrow = (const uint32_t*)((const uint8_t*)ring[wave][slot] + n16 * (SBW * GB));
#pragma unroll
            for (int s = 0; s < SBW; ++s) {
                if (Q8) {
#pragma unroll
                    for (int i = 0; i < 17; ++i) raw.w[s][i] = lrow[(GB * s + 68 * g) / 4 + i];
                } else {
                    const uint4 hd = *(const uint4*)(lrow + (GB * s) / 4);
                    raw.w[s][0] = hd.x, raw.w[s][1] = hd.y, raw.w[s][2] = hd.z, raw.w[s][3] = hd.w;
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        const uint2 q = *(const uint2*)(lrow + (GB * s + 16 + 32 * p + 8 * g) / 4);
                        raw.w[s][4 + 2 * p] = q.x, raw.w[s][5 + 2 * p] = q.y;
                    }
                }
            }
        }
        lds_wait_lgkm();  // the slot is in registers: it takes tile k + R
        if (k + Gq::R < nt) g8_issue<SBW * GB>(W, rowb, N, blockIdx.x + (k + Gq::R) * G, col0, ring[wave][slot], lane);
        g8_f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < SBW; ++s) {
            const uint32_t* d = raw.w[s];
            if constexpr (Q8) {
                const _Float16 s0 = __builtin_bit_cast(_Float16, (uint16_t)(d[0] & 0xFFFF));  // block 2g
                const _Float16 s1 = __builtin_bit_cast(_Float16, (uint16_t)(d[8] >> 16));     // block 2g + 1
#pragma unroll
                for (int m = 0; m < 8; ++m) {
                    const int q = m & 3;
                    uint32_t c0, c1;
                    if (m < 4) {  // block 2g: codes at byte 2 + c
                        c0 = __builtin_amdgcn_alignbyte(d[2 * q + 1], d[2 * q], 2);
                        c1 = __builtin_amdgcn_alignbyte(d[2 * q + 2], d[2 * q + 1], 2);
                    } else {  // block 2g + 1: codes at byte 36 + c (dword aligned)
                        c0 = d[9 + 2 * q];
                        c1 = d[10 + 2 * q];
                    }
                    const _Float16 sc = m < 4 ? s0 : s1;
                    const g8_h2 sc2 = {sc, sc};
                    uint32_t pr[4];
                    g8_q8_pairs(c0, pr[0], pr[1]);
                    g8_q8_pairs(c1, pr[2], pr[3]);
                    f16x8 b;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const g8_h2 cq = __builtin_bit_cast(g8_h2, pr[i]) - off;  // the codes, exact
                        const g8_h2 wv = cq * sc2;                                // q d, rounded once
                        b[2 * i] = wv[0];
                        b[2 * i + 1] = wv[1];
                    }
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[s][m], b, acc, 0, 0, 0);
                }
            } else {
                const float dd = f16_to_f32((uint16_t)(d[0] & 0xFFFF)), dm = f16_to_f32((uint16_t)(d[0] >> 16));
                auto scb = [&](int i) { return (int)((d[1 + (i >> 2)] >> (8 * (i & 3))) & 0xFF); };
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    int scv, mv;
                    if (j < 4) {
                        scv = scb(j) & 63;
                        mv = scb(j + 4) & 63;
                    } else {
                        scv = (scb(j + 4) & 0xF) | ((scb(j - 4) >> 6) << 4);
                        mv = (scb(j + 4) >> 4) | ((scb(j) >> 6) << 4);
                    }
                    const float sc = dd * (float)scv, nb = -fmaf(1024.f, sc, dm * (float)mv);
                    const int p = j >> 1, sh = 4 * (j & 1);  // sub-block 2p: low nibbles, 2p+1: high
                    const uint32_t u0 = d[4 + 2 * p] >> sh, u1 = d[5 + 2 * p] >> sh;
                    const uint32_t c[4] = {gq_and_or(u0, 0x000F000Fu, magic), gq_and_or(u0 >> 8, 0x000F000Fu, magic),
                                           gq_and_or(u1, 0x000F000Fu, magic), gq_and_or(u1 >> 8, 0x000F000Fu, magic)};
                    f16x8 b;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        b[2 * i] = (_Float16)fmaf(gq_lo(c[i]), sc, nb);
                        b[2 * i + 1] = (_Float16)fmaf(gq_hi(c[i]), sc, nb);
                    }
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[s][j], b, acc, 0, 0, 0);
                }
            }
        }
        // tokens 2g, 2g+1 of row n16: hi + lo parts; two tiles per LDS area
        const int ar = (k >> 1) & 1, ti = k & 1;
        red[ar][ti][wave][2 * g][n16] = acc[0] + acc[1];
        red[ar][ti][wave][2 * g + 1][n16] = acc[2] + acc[3];
        if (ti == 1 || k == nt - 1) {
            lds_barrier();  // LDS only: the transfers in flight stay in flight
            for (int i = tid; i < 128 * (ti + 1); i += blockDim.x) {
                const int tt = i >> 7, t = (i >> 4) & 7, nn = i & 15;
                const int n = (blockIdx.x + (k - ti + tt) * G) * 16 + nn;
                float v = 0.f;
                for (int w = 0; w < WB; ++w) v += red[ar][tt][w][t][nn];
                if (t < M && n < N) y[(size_t)t * N + n] = v;
            }
        }
    }
}

// sum of the K-slice partials, in slice order
__global__ void __launch_bounds__(256) k_g8_sum(const float* __restrict__ part, float* __restrict__ y, int n, int S) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float v = part[i];
    for (int s = 1; s < S; ++s) v += part[(size_t)s * n + i];
    y[i] = v;
}

int g8_sum_launch(const float* part, float* y, int n, int S) {
    hipLaunchKernelGGL(k_g8_sum, dim3(cdiv(n, 256)), dim3(256), 0, stream(), part, y, n, S);
    GH_LAUNCHED("k_g8_sum");
    return GH_OK;
}

template <int SBW, bool Q8>
static int g8_launch(const float* x, const void* w, float* y, int M, int K, int N, int S) {
    const int Ks = K / S, WB = Ks / (256 * SBW);
    static int per_cu[17];
    const auto kern = k_gemv8<SBW, Q8>;
    if (!per_cu[WB]) {
        int nb = 0;
        hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, 64 * WB, 0);
        per_cu[WB] = e == hipSuccess && nb > 0 ? nb : 1;
    }
    const int ntiles = (N + 15) / 16;
    const int slots = per_cu[WB] * num_cus() / S;  // the K slices share the chip
    float* out = y;
    if (S > 1) {
        out = (float*)workspace(WS_GEMM_PART, (size_t)S * M * N * 4);
        if (!out) return fail(GH_ENOMEM, "gemv8: workspace");
    }
    hipLaunchKernelGGL(kern, dim3(ntiles < slots ? ntiles : (slots > 0 ? slots : 1), S), dim3(64 * WB), 0, stream(),
                       x, (const uint8_t*)w, out, M, Ks, N, row_bytes(Q8 ? 2 : 3, K), K);
    GH_LAUNCHED(Q8 ? "k_gemv8<Q8_0>" : "k_gemv8<Q4_K>");
    if (S > 1) {
        hipLaunchKernelGGL(k_g8_sum, dim3(cdiv(M * N, 256)), dim3(256), 0, stream(), out, y, M * N, S);
        GH_LAUNCHED("k_g8_sum");
    }
    return GH_OK;
}

// Returns 1 if handled: Q4_K or Q8_0 (16-byte aligned rows), 2 <= M <= 8, K a multiple of 256;
// above 4096 values the row is cut into equal K slices (the smallest count whose slice fits a
// block), their partial sums added by a second launch in slice order.
int gemv8_dispatch(const float* x, const void* w, float* y, int M, int K, int N, int kind, int* rc) {
    if ((kind != 3 && kind != 2) || M < 2 || M > 8 || K % 256 != 0 || (((uintptr_t)x) & 15)) return 0;
    if (kind == 2 && ((uintptr_t)w & 15)) return 0;
    const int nsb = K / 256;
    // waves of SBW super-blocks, at most 8 waves (two per SIMD: the A operands stay in registers)
    // Q4_K rows of 16 super-blocks or more start at two slices: each block then converts half of
    // the activations (the launch's fixed part), worth the extra sum launch (c2 M=8 17.0 -> 16.2 us;
    // for Q8_0 it is not: 18.2 -> 19.0)
    for (int S = (kind == 3 && nsb >= 16) ? 2 : 1; S <= 8; ++S) {
        if (nsb % S) continue;
        const int ns = nsb / S;
        if (ns <= 8) {
            *rc = kind == 2 ? g8_launch<1, true>(x, w, y, M, K, N, S) : g8_launch<1, false>(x, w, y, M, K, N, S);
            return 1;
        }
        if (ns % 2 == 0 && ns <= 16) {
            *rc = kind == 2 ? g8_launch<2, true>(x, w, y, M, K, N, S) : g8_launch<2, false>(x, w, y, M, K, N, S);
            return 1;
        }
    }
    return 0;
}

}  // namespace gh
