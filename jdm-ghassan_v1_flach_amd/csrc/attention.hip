// GQA attention over the KV cache.
//
// Decode (one query token per sequence), split-K "flash decoding":
// a block owns one kv head and a contiguous run of logical positions, reads
// each K and V row ONCE for all `group` query heads of that kv head (the
// reference re-reads them per q head, cuda/attention.cu:621-810), keeps the
// scores of its run in LDS, and writes (max, sum, unnormalised o) partials
// that a small combine kernel merges. Lanes are laid out as positions x
// 16-byte channel groups, so one wave load instruction reads whole K/V rows
// contiguously. The same kernel serves the reference's fp16 ring cache
// (core/attn_cpu.cpp:151-254: pinned prefix + rolling ring) and the paged
// bf16 ragged-batch extension (page table per sequence).
//
// Prefill (attention_forward_ex, core/attn_cpu.cpp:29-94): causal flash
// attention on the matrix cores. A block is one q head x 128 queries, each
// wave 32 queries; per 64-key tile S^T = K Q^T (v_mfma_f32_32x32x16_f16),
// online softmax in registers, O += P V with P taken straight from the S^T
// accumulator layout (no LDS round trip) and V staged transposed in LDS.
#include <stdlib.h>

#include "gh_common.h"
#include "lds_dma.h"

namespace gh {

// ============================================================== decode
struct DecodeArgs {
    const float* q;           // [S][H][hd]
    const uint16_t* k;        // ring: [cache_max][KV][hd]  paged: [pages][page_size][KV][hd]
    const uint16_t* v;
    float* o_part;            // [S][KV][splits][G][hd]
    float* ml_part;           // [S][KV][splits][G][2]
    int H, KV, G, splits, chunk;
    float scale;
    // ring
    int ring_start, pinned, cur_len, cache_max, j0;
    // paged
    const int32_t* page_table;
    const int32_t* seq_lens;
    int max_pages, page_size;
    // ring cache with its length / ring start / pinned prefix read from the
    // device (graph-captured decode); null: the host scalars above are used
    const int32_t* ctl;
};

template <bool BF16>
__device__ __forceinline__ void widen8(const uint4 r, float* f) {
    const uint32_t u[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (BF16) {
            f[2 * i] = bf16_to_f32((uint16_t)(u[i] & 0xFFFF));
            f[2 * i + 1] = bf16_to_f32((uint16_t)(u[i] >> 16));
        } else {
            f[2 * i] = f16_to_f32((uint16_t)(u[i] & 0xFFFF));
            f[2 * i + 1] = f16_to_f32((uint16_t)(u[i] >> 16));
        }
    }
}

constexpr int DEC_CHUNK_MAX = 512, DEC_GMAX = 8;
constexpr int DEC_B = 4;  // steps of K / V rows loaded per batch

template <int HD, bool PAGED>
__global__ void __launch_bounds__(256) k_attn_decode(DecodeArgs a) {
    constexpr int LPP = HD / 8;     // lanes per position (16 B each)
    constexpr int PPS = 64 / LPP;   // positions per wave step
    __shared__ float sc[DEC_GMAX][DEC_CHUNK_MAX];
    __shared__ float sm[DEC_GMAX], sl[DEC_GMAX];
    __shared__ float red[4][DEC_GMAX][HD];

    const int split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane / LPP, cg = lane % LPP;
    const int G = a.G;

    if (!PAGED && a.ctl) {  // decode control block: token, len, start, pinned
        a.cur_len = a.ctl[1];
        a.ring_start = a.ctl[2];
        a.pinned = min(a.ctl[3], a.cur_len);
    }
    int jb, je;  // logical positions [jb, je) of this block
    if (PAGED) {
        const int L = a.seq_lens[seq];
        jb = split * a.chunk;
        je = min(L, jb + a.chunk);
    } else {
        jb = a.j0 + split * a.chunk;
        je = min(a.cur_len, jb + a.chunk);
    }
    const int n = je - jb;
    const size_t part = ((size_t)seq * a.KV + kvh) * a.splits + split;
    if (n <= 0) {
        if (threadIdx.x < G) {
            a.ml_part[(part * G + threadIdx.x) * 2] = -INFINITY;
            a.ml_part[(part * G + threadIdx.x) * 2 + 1] = 0.f;
        }
        return;
    }
    const int ring_cap = a.cache_max - a.pinned;
    auto row_of = [&](int j) -> size_t {  // element offset of row (position j, kvh)
        size_t slot;
        if (PAGED) {
            const int page = a.page_table[(size_t)seq * a.max_pages + j / a.page_size];
            slot = (size_t)page * a.page_size + j % a.page_size;
        } else {
            slot = j < a.pinned ? (size_t)j
                                : (size_t)a.pinned + (size_t)((a.ring_start + (j - a.pinned)) % (ring_cap > 0 ? ring_cap : 1));
        }
        return (slot * a.KV + kvh) * HD;
    };

    float qr[DEC_GMAX][8];
    const float* qb = a.q + ((size_t)seq * a.H + (size_t)kvh * G) * HD + cg * 8;
#pragma unroll
    for (int g = 0; g < DEC_GMAX; ++g) {
        if (g < G) {
            const float4 x0 = *(const float4*)(qb + (size_t)g * HD), x1 = *(const float4*)(qb + (size_t)g * HD + 4);
            qr[g][0] = x0.x; qr[g][1] = x0.y; qr[g][2] = x0.z; qr[g][3] = x0.w;
            qr[g][4] = x1.x; qr[g][5] = x1.y; qr[g][6] = x1.z; qr[g][7] = x1.w;
        }
    }
    // ---- scores; the K rows of DEC_B steps are requested together (one
    // memory round trip per batch instead of per step)
    for (int base0 = wave * PPS; base0 < n; base0 += 4 * PPS * DEC_B) {
        uint4 kr[DEC_B];
#pragma unroll
        for (int b = 0; b < DEC_B; ++b) {
            const int p = base0 + b * 4 * PPS + sub;
            if (p < n) kr[b] = *(const uint4*)(a.k + row_of(jb + p) + cg * 8);
        }
#pragma unroll
        for (int b = 0; b < DEC_B; ++b) {
            const int p = base0 + b * 4 * PPS + sub;
            if (base0 + b * 4 * PPS >= n) break;  // wave-uniform
            const bool ok = p < n;
            float kf[8];
            if (ok) {
                widen8<PAGED>(kr[b], kf);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) kf[i] = 0.f;
            }
#pragma unroll
            for (int g = 0; g < DEC_GMAX; ++g) {
                if (g >= G) break;
                float sc_ = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) sc_ = fmaf(qr[g][i], kf[i], sc_);
#pragma unroll
                for (int o = LPP >> 1; o > 0; o >>= 1) sc_ += __shfl_xor(sc_, o, 64);
                if (ok && cg == 0) sc[g][p] = sc_ * a.scale;
            }
        }
    }
    __syncthreads();
    // ---- softmax statistics of this run (one wave per head)
    for (int g = wave; g < G; g += 4) {
        float m = -INFINITY;
        for (int p = lane; p < n; p += 64) m = fmaxf(m, sc[g][p]);
        m = wave_max(m);
        float l = 0.f;
        for (int p = lane; p < n; p += 64) {
            const float e = expf(sc[g][p] - m);
            sc[g][p] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            sm[g] = m;
            sl[g] = l;
        }
    }
    __syncthreads();
    // ---- o = sum p v over the run
    float acc[DEC_GMAX][8];
#pragma unroll
    for (int g = 0; g < DEC_GMAX; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
    for (int base0 = wave * PPS; base0 < n; base0 += 4 * PPS * DEC_B) {
        uint4 vr[DEC_B];
#pragma unroll
        for (int b = 0; b < DEC_B; ++b) {
            const int p = base0 + b * 4 * PPS + sub;
            if (p < n) vr[b] = *(const uint4*)(a.v + row_of(jb + p) + cg * 8);
        }
#pragma unroll
        for (int b = 0; b < DEC_B; ++b) {
            const int p = base0 + b * 4 * PPS + sub;
            if (p < n) {
                float vf[8];
                widen8<PAGED>(vr[b], vf);
#pragma unroll
                for (int g = 0; g < DEC_GMAX; ++g) {
                    if (g >= G) break;
                    const float w = sc[g][p];
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[g][i] = fmaf(w, vf[i], acc[g][i]);
                }
            }
        }
    }
#pragma unroll
    for (int g = 0; g < DEC_GMAX; ++g) {
        if (g >= G) break;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float v = acc[g][i];
#pragma unroll
            for (int o = LPP; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
            if (sub == 0) red[wave][g][cg * 8 + i] = v;
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < G * HD; e += 256) {
        const int g = e / HD, c = e % HD;
        a.o_part[(part * G + g) * HD + c] = red[0][g][c] + red[1][g][c] + red[2][g][c] + red[3][g][c];
    }
    if (threadIdx.x < G) {
        a.ml_part[(part * G + threadIdx.x) * 2] = sm[threadIdx.x];
        a.ml_part[(part * G + threadIdx.x) * 2 + 1] = sl[threadIdx.x];
    }
}


// ---------------------------------------------------------------- decode v2
// head_dim 64 / 128: the same split-K partials as k_attn_decode, in one pass
// over the run with an online softmax per wave:
//  - K and V rows of a group of 16 positions are moved together by LDS DMA
//    into a wave-private ring of DEC2_NST stages, requested DEC2_NST groups
//    ahead; K's 16-byte pieces are stored with an XOR swizzle so the 16 rows
//    of an MFMA operand read hit distinct LDS banks;
//  - scores on the matrix cores: S = K q^T by v_mfma_f32_16x16x32_{bf16,f16}
//    (A = the 16 K rows, B = the G query heads as columns), q split into two
//    parts of the cache's type (hi + lo) so the products keep fp32-level
//    accuracy; no per-position lane reductions;
//  - running max / sum per head, P handed to the P V layout through a small
//    wave-private LDS area; P V on the vector units (a lane owns 8 channels
//    of a few rows per group), accumulators rescaled when the max grows;
//  - the 4 waves' (max, sum, o) merged in LDS into the block's partial.
// Wave w processes the groups w, w+4, ... of the block's run.
constexpr int DEC2_NST = 2;

template <bool BF>
struct Dec2Op;
template <>
struct Dec2Op<true> {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    typedef __bf16 s;
    __device__ static float4 mfma(v8 a, v8 b, float4 c) {
        typedef float f4 __attribute__((ext_vector_type(4)));
        const f4 r = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, __builtin_bit_cast(f4, c), 0, 0, 0);
        return __builtin_bit_cast(float4, r);
    }
};
template <>
struct Dec2Op<false> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    typedef _Float16 s;
    __device__ static float4 mfma(v8 a, v8 b, float4 c) {
        typedef float f4 __attribute__((ext_vector_type(4)));
        const f4 r = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, __builtin_bit_cast(f4, c), 0, 0, 0);
        return __builtin_bit_cast(float4, r);
    }
};

constexpr int DEC2_CHUNK_MAX = 2048;  // positions per block (no score buffer bounds it)

template <int HD, bool PAGED, int GMAX>
__global__ void __launch_bounds__(256) k_attn_decode2(DecodeArgs a) {
    using Op = Dec2Op<PAGED>;  // the paged cache is bf16, the ring cache fp16
    constexpr int PPR = HD / 8;        // 16-byte pieces per row
    constexpr int RPI = 64 / PPR;      // rows per transfer instruction
    constexpr int IPS = 16 / RPI;      // transfer instructions per 16 rows
    constexpr int KS = HD / 32;        // MFMA k-steps
    constexpr int NST = DEC2_NST;
    constexpr int SH = PPR == 16 ? 0 : 1;         // K piece m of row r sits at m ^ ((r >> SH) & (PPR - 1))
    constexpr int QI = (GMAX * HD / 4 + 63) / 64;  // transfers of the query block (fp32, G <= GMAX)
    static_assert(QI * 64 <= 2 * 16 * PPR, "query block fits a ring stage");
    __shared__ __attribute__((aligned(16))) uint4 ring[4][NST][2][16 * PPR];  // [wave][stage][K, V][rows]
    __shared__ __attribute__((aligned(16))) float pex[4][GMAX][20];  // per wave: P [head][position], [16] = rescale
    __shared__ int spage[PAGED ? DEC2_CHUNK_MAX + 1 : 1];

    const int split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.G;
    if (!PAGED && a.ctl) {  // decode control block: token, len, start, pinned
        a.cur_len = a.ctl[1];
        a.ring_start = a.ctl[2];
        a.pinned = min(a.ctl[3], a.cur_len);
    }
    int jb, je;  // logical positions [jb, je) of this block
    if (PAGED) {
        const int L = a.seq_lens[seq];
        jb = split * a.chunk;
        je = min(L, jb + a.chunk);
    } else {
        jb = a.j0 + split * a.chunk;
        je = min(a.cur_len, jb + a.chunk);
    }
    const int n = je - jb;
    const size_t part = ((size_t)seq * a.KV + kvh) * a.splits + split;
    if (n <= 0) {
        if (tid < G) {
            a.ml_part[(part * G + tid) * 2] = -INFINITY;
            a.ml_part[(part * G + tid) * 2 + 1] = 0.f;
        }
        return;
    }
    int pg0 = 0;
    if (PAGED) {  // the run's page numbers, staged before any transfer is in flight
        pg0 = jb / a.page_size;
        const int npg = (je - 1) / a.page_size - pg0 + 1;
        for (int i = tid; i < npg; i += 256) spage[i] = a.page_table[(size_t)seq * a.max_pages + pg0 + i];
        __syncthreads();
    }
    const int ring_cap = a.cache_max - a.pinned;
    auto row_of = [&](int j) -> size_t {  // element offset of row (position j, kvh)
        size_t slot;
        if (PAGED) {
            slot = (size_t)spage[j / a.page_size - pg0] * a.page_size + j % a.page_size;
        } else {
            slot = j < a.pinned ? (size_t)j
                                : (size_t)a.pinned + (size_t)((a.ring_start + (j - a.pinned)) % (ring_cap > 0 ? ring_cap : 1));
        }
        return (slot * a.KV + kvh) * HD;
    };
    const int ngroups = (n + 15) >> 4;
    const int ngw = wave < ngroups ? (ngroups - wave + 3) >> 2 : 0;  // this wave's groups: wave, wave+4, ...
    // K and V rows of group k of this wave -> ring stage st (rows past the run re-read its last row)
    auto dma = [&](int k, int st) {
        const int gi = wave + 4 * (k < ngw ? k : ngw - 1);
#pragma unroll
        for (int i = 0; i < IPS; ++i) {
            const int slot = i * 64 + lane, r = slot / PPR, t = slot % PPR;
            const size_t row = row_of(jb + min(gi * 16 + r, n - 1));
            lds_dma16(a.k + row + (t ^ ((r >> SH) & (PPR - 1))) * 8, lds_addr(&ring[wave][st][0][i * 64]));
            lds_dma16(a.v + row + t * 8, lds_addr(&ring[wave][st][1][i * 64]));
        }
    };
    // ---- query block -> the wave's last ring stage (read before that stage is first filled)
    {
        const float* qb = a.q + ((size_t)seq * a.H + (size_t)kvh * G) * HD;
        float* qs = (float*)&ring[wave][NST - 1][0][0];
#pragma unroll
        for (int i = 0; i < QI; ++i) {
            const int piece = min(i * 64 + lane, G * HD / 4 - 1);
            lds_dma16(qb + 4 * piece, lds_addr(qs + i * 256));
        }
    }
    if (ngw > 0)
#pragma unroll
        for (int st = 0; st < NST - 1; ++st) dma(st, st);
    lds_dma_wait<2 * IPS>(ngw > 0 ? NST - 1 : 0);  // the query block landed
    const int n16 = lane & 15, kg = lane >> 4;
    typename Op::v8 bh[KS], bl[KS];  // B: column n16 = head n16 (zero past G), channels 32 s + 8 kg + i
    {
        const float* qs = (const float*)&ring[wave][NST - 1][0][0] + n16 * HD;
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float qv = n16 < G ? qs[32 * s + 8 * kg + i] : 0.f;
                const typename Op::s h = (typename Op::s)qv;
                bh[s][i] = h;
                bl[s][i] = (typename Op::s)(qv - (float)h);
            }
    }
    lds_wait_lgkm();
    if (ngw > 0) dma(NST - 1, NST - 1);
    const int sub = lane / PPR, cg = lane % PPR;  // P V: channels 8 cg .. 8 cg + 7 of rows sub + RPI r
    float acc[GMAX][8];
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
    float run_m = -INFINITY, run_l = 0.f;  // of head n16 (lanes n16 < G)
    for (int k = 0; k < ngw; ++k) {
        lds_dma_wait<2 * IPS>((k + 1 < NST || k + 1 < ngw) ? 1 : 0);
        const int st = k % NST;
        uint4 ar[KS], vr[16 / RPI];
#pragma unroll
        for (int s = 0; s < KS; ++s) ar[s] = ring[wave][st][0][n16 * PPR + ((4 * s + kg) ^ ((n16 >> SH) & (PPR - 1)))];
#pragma unroll
        for (int r = 0; r < 16 / RPI; ++r) vr[r] = ring[wave][st][1][(sub + RPI * r) * PPR + cg];
        if (k + NST < ngw) {
            lds_wait_lgkm();
            dma(k + NST, st);
        }
        float4 d = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const typename Op::v8 av = __builtin_bit_cast(typename Op::v8, ar[s]);
            d = Op::mfma(av, bh[s], d);
            d = Op::mfma(av, bl[s], d);
        }
        // lane (head n16, row group kg) holds positions p0 + e of the group
        const int gp0 = (wave + 4 * k) * 16, p0 = gp0 + 4 * kg;
        float sv[4] = {d.x * a.scale, d.y * a.scale, d.z * a.scale, d.w * a.scale};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (p0 + e >= n) sv[e] = -INFINITY;
        float gm = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        gm = fmaxf(gm, __shfl_xor(gm, 16, 64));
        gm = fmaxf(gm, __shfl_xor(gm, 32, 64));
        const float nm = fmaxf(run_m, gm);  // finite: the group has at least one position
        const float f = expf(run_m - nm);
        float pv[4], ps = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            pv[e] = expf(sv[e] - nm);
            ps += pv[e];
        }
        ps += __shfl_xor(ps, 16, 64);
        ps += __shfl_xor(ps, 32, 64);
        run_l = run_l * f + ps;
        run_m = nm;
        if (n16 < G) {
            *(float4*)&pex[wave][n16][4 * kg] = make_float4(pv[0], pv[1], pv[2], pv[3]);
            if (kg == 0) pex[wave][n16][16] = f;
        }
        lds_wait_lgkm();  // the wave's own P (no other wave touches pex[wave])
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            if (g >= G) break;
            const float fg = pex[wave][g][16];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[g][i] *= fg;
        }
#pragma unroll
        for (int r = 0; r < 16 / RPI; ++r) {
            float vf[8];
            widen8<PAGED>(vr[r], vf);
#pragma unroll
            for (int g = 0; g < GMAX; ++g) {
                if (g >= G) break;
                const float w = pex[wave][g][sub + RPI * r];  // 0 past the run
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[g][i] = fmaf(w, vf[i], acc[g][i]);
            }
        }
        lds_wait_lgkm();  // pex is rewritten by the next group
    }
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        if (g >= G) break;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma unroll
            for (int o = PPR; o < 64; o <<= 1) acc[g][i] += __shfl_xor(acc[g][i], o, 64);
        }
    }
    // ---- merge the 4 waves: (m_w, l_w, o_w) -> (M, sum l_w e^(m_w - M), sum o_w e^(m_w - M))
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // re-read stages of a short run
    lds_barrier();  // every wave is done with its ring: it becomes the merge area
    float* red = (float*)&ring[0][0][0][0];  // [4][GMAX][HD]
    float* wml = red + 4 * GMAX * HD;    // [4][GMAX][2]
    if (sub == 0)
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            if (g >= G) break;
#pragma unroll
            for (int i = 0; i < 8; ++i) red[(wave * GMAX + g) * HD + cg * 8 + i] = acc[g][i];
        }
    if (kg == 0 && n16 < G) {
        wml[(wave * GMAX + n16) * 2] = run_m;
        wml[(wave * GMAX + n16) * 2 + 1] = run_l;
    }
    lds_barrier();
    for (int e = tid; e < G * HD; e += 256) {
        const int g = e / HD, c = e % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, wml[(w * GMAX + g) * 2]);
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float mw = wml[(w * GMAX + g) * 2];
            if (mw > -INFINITY) o += red[(w * GMAX + g) * HD + c] * expf(mw - M);
        }
        a.o_part[(part * G + g) * HD + c] = o;
    }
    if (tid < G) {
        float M = -INFINITY, L = 0.f;
        for (int w = 0; w < 4; ++w) M = fmaxf(M, wml[(w * GMAX + tid) * 2]);
        for (int w = 0; w < 4; ++w) {
            const float mw = wml[(w * GMAX + tid) * 2];
            if (mw > -INFINITY) L += wml[(w * GMAX + tid) * 2 + 1] * expf(mw - M);
        }
        a.ml_part[(part * G + tid) * 2] = M;
        a.ml_part[(part * G + tid) * 2 + 1] = L;
    }
}

// Merge the split partials: o = sum_s e^(m_s-M) o_s / sum_s e^(m_s-M) l_s.
// One block per (head, sequence): the split weights are computed once into
// LDS, then every thread reduces one channel over the splits (coalesced).
// An empty context (no positions) gives zeros (core/attn_cpu.cpp:244-246).
constexpr int COMB_MAX_SPLITS = 1024;
__global__ void __launch_bounds__(256) k_attn_combine(const float* __restrict__ o_part, const float* __restrict__ ml,
                                                      float* __restrict__ out, int H, int KV, int G, int splits,
                                                      int hd) {
    __shared__ float sw[COMB_MAX_SPLITS];
    __shared__ float red[4];
    const int h = blockIdx.x, seq = blockIdx.y;
    const int kvh = h / G, g = h % G;
    const size_t base = ((size_t)seq * KV + kvh) * splits;
    float M = -INFINITY;
    for (int s = threadIdx.x; s < splits; s += 256) {
        const float* p = ml + ((base + s) * G + g) * 2;
        if (p[1] > 0.f) M = fmaxf(M, p[0]);
    }
    M = wave_max(M);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float L = 0.f;
    for (int s = threadIdx.x; s < splits; s += 256) {
        const float* p = ml + ((base + s) * G + g) * 2;
        const float w = p[1] > 0.f ? expf(p[0] - M) : 0.f;
        sw[s] = w;
        L += w * p[1];
    }
    L = wave_sum(L);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = L;
    __syncthreads();
    L = red[0] + red[1] + red[2] + red[3];
    const float inv = L > 0.f ? 1.0f / L : 0.0f;
    // thread (part, channel): the splits part, part + np, ... of one channel, COMB_U loads in
    // flight at a time (an empty split's o is never written: it is selected away, not multiplied)
    constexpr int COMB_U = 8;
    __shared__ float cred[256];
    const int np = hd <= 256 ? 256 / hd : 1;
    const int c = threadIdx.x % hd, pt = threadIdx.x / hd;
    float acc = 0.f;
    if (pt < np && c < hd) {
        for (int s0 = pt; s0 < splits; s0 += COMB_U * np) {
            float ov[COMB_U], wv[COMB_U];
#pragma unroll
            for (int u = 0; u < COMB_U; ++u) {
                const int s = s0 + u * np;
                wv[u] = s < splits ? sw[s] : 0.f;
                ov[u] = s < splits ? o_part[((base + s) * G + g) * hd + c] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < COMB_U; ++u) acc += wv[u] != 0.f ? wv[u] * ov[u] : 0.f;
        }
    }
    cred[threadIdx.x] = acc;
    __syncthreads();
    for (int cc = threadIdx.x; cc < hd; cc += 256) {
        float v = 0.f;
        for (int q = 0; q < np; ++q) v += cred[q * hd + cc];
        out[((size_t)seq * H + h) * hd + cc] = v * inv;
    }
}

// shortest run of positions per split (a multiple of 64)
int attn_chunk_min() { return 64; }

static int pick_chunk(int len, int blocks_other, int cap = DEC_CHUNK_MAX) {
    // enough blocks to fill the chip, runs of 64..512 positions
    const int target = 2 * num_cus();
    int per = cdiv(target, blocks_other > 0 ? blocks_other : 1);
    int chunk = cdiv(len > 0 ? len : 1, per > 0 ? per : 1);
    chunk = (chunk + 63) / 64 * 64;
    if (chunk < attn_chunk_min()) chunk = attn_chunk_min();
    if (chunk > cap) chunk = cap;
    return chunk;
}

template <int HD, bool PAGED>
static void launch_dec2(const DecodeArgs& a, dim3 grid) {
    if (a.G <= 4) hipLaunchKernelGGL((k_attn_decode2<HD, PAGED, 4>), grid, dim3(256), 0, stream(), a);
    else hipLaunchKernelGGL((k_attn_decode2<HD, PAGED, 8>), grid, dim3(256), 0, stream(), a);
}

// Split-K decode. out == null: partials only, the merge is left to the
// consumer (the fused output projection merges them in its prologue);
// otherwise k_attn_combine merges them into out. (A merge by the last block
// of each kv head was slower: the device-scope fence every block then needs
// writes back L2.)
// Floats of split-K partials (o, then (max, sum) pairs at a 64-float boundary) one decode
// launch needs; sets a.chunk / a.splits.
static size_t decode_partial_floats(DecodeArgs& a, int hd, int S, int span, size_t* ml_off) {
    const bool v2 = (hd == 64 || hd == 128) && a.G <= 8;
    a.chunk = pick_chunk(span, a.KV * S, v2 ? DEC2_CHUNK_MAX : DEC_CHUNK_MAX);
    a.splits = cdiv(span > 0 ? span : 1, a.chunk);
    const size_t no = (size_t)S * a.KV * a.splits * a.G * hd;
    *ml_off = (no + 63) / 64 * 64;
    return *ml_off + (size_t)S * a.KV * a.splits * a.G * 2;
}

// ws: caller-provided partials buffer of decode_partial_floats() floats, or null for the
// backend's grow-only workspace.
template <bool PAGED>
static int launch_decode(DecodeArgs& a, int hd, int S, int span, float* out, float* ws = nullptr) {
    const bool v2 = (hd == 64 || hd == 128) && a.G <= 8;
    size_t ml_off = 0;
    const size_t nf = decode_partial_floats(a, hd, S, span, &ml_off);
    float* o = ws;
    float* ml = ws ? ws + ml_off : nullptr;
    if (!ws) {
        o = (float*)workspace(WS_ATTN_O, ml_off * 4);
        ml = (float*)workspace(WS_ATTN_ML, (nf - ml_off) * 4);
    }
    if (!o || !ml) return fail(GH_ENOMEM, "attention decode: workspace");
    a.o_part = o;
    a.ml_part = ml;
    const dim3 grid(a.splits, a.KV, S);
    switch (hd) {
        case 16: hipLaunchKernelGGL((k_attn_decode<16, PAGED>), grid, dim3(256), 0, stream(), a); break;
        case 32: hipLaunchKernelGGL((k_attn_decode<32, PAGED>), grid, dim3(256), 0, stream(), a); break;
        case 64:
            if (v2) launch_dec2<64, PAGED>(a, grid);
            else hipLaunchKernelGGL((k_attn_decode<64, PAGED>), grid, dim3(256), 0, stream(), a);
            break;
        case 128:
            if (v2) launch_dec2<128, PAGED>(a, grid);
            else hipLaunchKernelGGL((k_attn_decode<128, PAGED>), grid, dim3(256), 0, stream(), a);
            break;
        default: return fail(GH_EUNSUPPORTED, "attention decode: head_dim %d (supported: 16, 32, 64, 128)", hd);
    }
    GH_LAUNCHED("k_attn_decode");
    if (!out) return GH_OK;
    if (a.splits > COMB_MAX_SPLITS) return fail(GH_EUNSUPPORTED, "attention decode: %d splits", a.splits);
    hipLaunchKernelGGL(k_attn_combine, dim3(a.H, S), dim3(256), 0, stream(), o, ml, out, a.H, a.KV, a.G, a.splits, hd);
    GH_LAUNCHED("k_attn_combine");
    return GH_OK;
}
template <bool PAGED>
static int launch_decode_partials(DecodeArgs& a, int hd, int S, int span) {
    return launch_decode<PAGED>(a, hd, S, span, nullptr);
}

// ============================================================== prefill
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t gh_u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int PF_BQ = 128, PF_BK = 64;

// q/k/v/out fp32, [B][T][H|KV][HD]
template <int HD>
__global__ void __launch_bounds__(256) k_attn_prefill_mfma(const float* __restrict__ q, const float* __restrict__ k,
                                                           const float* __restrict__ v, float* __restrict__ out,
                                                           int T, int H, int KV, float scale, int window) {
    constexpr int KS = HD + 8;  // LDS row stride of K (bf16)
    constexpr int VS = PF_BK + 8;
    __shared__ __attribute__((aligned(16))) _Float16 sK[PF_BK * KS];
    __shared__ __attribute__((aligned(16))) _Float16 sVt[HD * VS];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nqt = cdiv(T, PF_BQ);
    const int qt = nqt - 1 - (int)blockIdx.x;  // heavy (late) tiles first
    const int h = blockIdx.y, b = blockIdx.z;
    const int G = H / KV, kvh = h / G;
    const int q0 = qt * PF_BQ + wave * 32;
    const size_t qs = (size_t)T * H * HD, kvs = (size_t)T * KV * HD;
    const float* qb = q + b * qs;
    const float* kb = k + b * kvs;
    const float* vb = v + b * kvs;

    // B operand of S^T = K Q^T: lane holds query j = lane%32, dims 16s + 8(lane/32) + 0..7
    const int qj = q0 + (lane & 31), hf = lane >> 5;
    f16x8 qreg[HD / 16];
#pragma unroll
    for (int s = 0; s < HD / 16; ++s) {
        if (qj < T) {
            const float* src = qb + ((size_t)qj * H + h) * HD + 16 * s + 8 * hf;
            const float4 a0 = *(const float4*)src, a1 = *(const float4*)(src + 4);
            qreg[s][0] = (_Float16)a0.x; qreg[s][1] = (_Float16)a0.y; qreg[s][2] = (_Float16)a0.z; qreg[s][3] = (_Float16)a0.w;
            qreg[s][4] = (_Float16)a1.x; qreg[s][5] = (_Float16)a1.y; qreg[s][6] = (_Float16)a1.z; qreg[s][7] = (_Float16)a1.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) qreg[s][e] = (_Float16)0.f;
        }
    }
    f32x16 oacc[HD / 32];
#pragma unroll
    for (int c = 0; c < HD / 32; ++c)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[c][e] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;  // for query qj (both halves keep copies)

    const int kend = min(T, qt * PF_BQ + PF_BQ);  // causal: keys < last query of the tile + 1
    int kbeg = 0;
    if (window > 0) kbeg = max(0, qt * PF_BQ - window + 1) / PF_BK * PF_BK;
    for (int k0 = kbeg; k0 < kend; k0 += PF_BK) {
        __syncthreads();
        // stage K [64][HD] and V^T [HD][64] as fp16 (the cache precision)
        for (int e = threadIdx.x; e < PF_BK * HD / 4; e += 256) {
            const int r = e / (HD / 4), c4 = (e % (HD / 4)) * 4;
            const int key = k0 + r;
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (key < T) {
                kv = *(const float4*)(kb + ((size_t)key * KV + kvh) * HD + c4);
                vv = *(const float4*)(vb + ((size_t)key * KV + kvh) * HD + c4);
            }
            _Float16* kd = sK + r * KS + c4;
            kd[0] = (_Float16)kv.x; kd[1] = (_Float16)kv.y; kd[2] = (_Float16)kv.z; kd[3] = (_Float16)kv.w;
            sVt[(c4 + 0) * VS + r] = (_Float16)vv.x;
            sVt[(c4 + 1) * VS + r] = (_Float16)vv.y;
            sVt[(c4 + 2) * VS + r] = (_Float16)vv.z;
            sVt[(c4 + 3) * VS + r] = (_Float16)vv.w;
        }
        __syncthreads();
        if (k0 > q0 + 31) continue;  // whole tile in this wave's future (uniform per wave)
        // S^T tiles: keys 32t + row(e), query lane%32
        f32x16 st[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int e = 0; e < 16; ++e) st[t][e] = 0.f;
#pragma unroll
            for (int s = 0; s < HD / 16; ++s) {
                const f16x8 ka = *(const f16x8*)(sK + (32 * t + (lane & 31)) * KS + 16 * s + 8 * hf);
                st[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qreg[s], st[t], 0, 0, 0);
            }
        }
        // mask + scale; key of element e in tile t: k0 + 32t + 8(e/4) + 4hf + e%4
        float tmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int key = k0 + 32 * t + 8 * (e >> 2) + 4 * hf + (e & 3);
                const bool vis = key <= qj && key < T && (window <= 0 || key > qj - window);
                const float s = vis ? st[t][e] * scale : -INFINITY;
                st[t][e] = s;
                tmax = fmaxf(tmax, s);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = (m_new == -INFINITY) ? 1.f : expf(m_run - m_new);
        float psum = 0.f;
        f16x8 pa[4];  // A operands of P V for the 4 k-slices of 16 keys
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float p = (st[t][e] == -INFINITY) ? 0.f : expf(st[t][e] - m_new);
                psum += p;
                pa[2 * t + (e >> 3)][e & 7] = (_Float16)p;
            }
        psum += __shfl_xor(psum, 32, 64);
        l_run = l_run * alpha + psum;
        m_run = m_new;
        // rescale O rows: the O layout holds query rows 8(e/4)+4hf+e%4 of the
        // wave's 32; lane r holds alpha of query row r
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float ar = __shfl(alpha, 8 * (e >> 2) + 4 * hf + (e & 3), 64);
#pragma unroll
            for (int c = 0; c < HD / 32; ++c) oacc[c][e] *= ar;
        }
        // O += P V. k-slice u (16 keys) of P holds, for lane half hf, keys
        // 32(u/2) + 8(2(u%2) + i/4) + 4hf + i%4 (i = 0..7); V^T is read with the same keys.
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int kbase = 32 * (u >> 1) + 16 * (u & 1) + 4 * hf;
#pragma unroll
            for (int c = 0; c < HD / 32; ++c) {
                const _Float16* vr = sVt + (32 * c + (lane & 31)) * VS;
                f16x8 vb8;
                const f16x4 lo = *(const f16x4*)(vr + kbase), hi = *(const f16x4*)(vr + kbase + 8);
                vb8[0] = lo[0]; vb8[1] = lo[1]; vb8[2] = lo[2]; vb8[3] = lo[3];
                vb8[4] = hi[0]; vb8[5] = hi[1]; vb8[6] = hi[2]; vb8[7] = hi[3];
                oacc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa[u], vb8, oacc[c], 0, 0, 0);
            }
        }
    }
    // normalise rows by 1/l and store. O element (c, e): query row 8(e/4)+4hf+e%4, channel 32c + lane%32
    const float linv = l_run > 0.f ? 1.0f / l_run : 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int r = 8 * (e >> 2) + 4 * hf + (e & 3);
        const float inv = __shfl(linv, r, 64);
        const int qi = q0 + r;
        if (qi >= T) continue;
        float* dst = out + b * qs + ((size_t)qi * H + h) * HD;
#pragma unroll
        for (int c = 0; c < HD / 32; ++c) dst[32 * c + (lane & 31)] = oacc[c][e] * inv;
    }
}

// ---- fp16 K / V^T staging for the prefill: K16 [B][KV][Tp][HD] and
// Vt16 [B][KV][HD][Tp] (Tp = T rounded up to 64, zero-filled), written once
// so every (query tile, head) block copies its key tiles with 16-byte loads.
template <int HD>
__global__ void __launch_bounds__(256) k_kv_f16(const float* __restrict__ k, const float* __restrict__ v,
                                                _Float16* __restrict__ K16, _Float16* __restrict__ Vt16, int T,
                                                int KV, int Tp) {
    __shared__ float sv[PF_BK][HD + 1];
    const int t0 = blockIdx.x * PF_BK, kvh = blockIdx.y, b = blockIdx.z;
    const size_t kvs = (size_t)T * KV * HD;
    _Float16* kd = K16 + (((size_t)b * KV + kvh) * Tp + t0) * HD;
    for (int e = threadIdx.x; e < PF_BK * HD / 4; e += 256) {
        const int r = e / (HD / 4), c4 = (e % (HD / 4)) * 4;
        const int key = t0 + r;
        float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
        if (key < T) {
            kv = *(const float4*)(k + b * kvs + ((size_t)key * KV + kvh) * HD + c4);
            vv = *(const float4*)(v + b * kvs + ((size_t)key * KV + kvh) * HD + c4);
        }
        f16x4 h4;
        h4[0] = (_Float16)kv.x; h4[1] = (_Float16)kv.y; h4[2] = (_Float16)kv.z; h4[3] = (_Float16)kv.w;
        *(f16x4*)(kd + (size_t)r * HD + c4) = h4;
        sv[r][c4] = vv.x; sv[r][c4 + 1] = vv.y; sv[r][c4 + 2] = vv.z; sv[r][c4 + 3] = vv.w;
    }
    __syncthreads();
    // V^T rows keep each 16-key group in MFMA k-slot order: slot s holds key
    // 8((s & 7) >> 2) + 4(s >> 3) + (s & 3), the key the P operand carries in slot s (P comes
    // from the S accumulator, whose lane holds keys 4h + i and 8 + 4h + i), so one 16-byte read
    // of V^T is the B operand of the P.V MFMA
    _Float16* vd = Vt16 + ((size_t)b * KV + kvh) * HD * Tp + t0;
    for (int e = threadIdx.x; e < HD * (PF_BK / 8); e += 256) {
        const int c = e / (PF_BK / 8), r8 = (e % (PF_BK / 8)) * 8;
        f16x8 h8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int sl = (r8 & 15) + i;  // slot within the 16-key group
            const int key = (r8 & ~15) + 8 * ((sl & 7) >> 2) + 4 * (sl >> 3) + (sl & 3);
            h8[i] = (_Float16)sv[key][c];
        }
        *(f16x8*)(vd + (size_t)c * Tp + r8) = h8;
    }
}

// Causal flash attention over the fp16 K / V^T tiles. Block = 128 queries
// (4 waves x 32) of one head; key tiles of 64 are double-buffered in LDS:
// the next tile's 16-byte pieces are loaded into registers while the
// current tile is multiplied. MFMA layout as k_attn_prefill_mfma. Softmax
// in the log2 domain (scores pre-multiplied by scale*log2(e), one v_exp_f32
// per score); masks only on the tiles that cross the diagonal or the
// window; the running output is rescaled only when a row maximum moved.
template <int HD>
__global__ void __launch_bounds__(256, 2) k_attn_prefill_f16(const float* __restrict__ q, const _Float16* __restrict__ K16,
                                                          const _Float16* __restrict__ Vt16, float* __restrict__ out,
                                                          int T, int Tp, int H, int KV, float scale, int window) {
    constexpr int KS = HD + 8;
    constexpr int VS = PF_BK + 8;
    constexpr int KPT = PF_BK * HD / 8 / 256;  // 16-byte pieces per thread (K), same for V^T
    __shared__ __attribute__((aligned(16))) _Float16 sK[2][PF_BK * KS];
    __shared__ __attribute__((aligned(16))) _Float16 sVt[2][HD * VS];
    __shared__ __attribute__((aligned(16))) float salpha[4][32];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, tid = threadIdx.x;
    const int nqt = cdiv(T, PF_BQ);
    // block bx takes q-tile nqt - 1 - bx (late, heavy) and then q-tile bx (early, light): every
    // block does the same causal work, in one round of the grid
    for (int pass = 0; pass < 2; ++pass) {
        const int qt = pass == 0 ? nqt - 1 - (int)blockIdx.x : (int)blockIdx.x;
        if (pass == 1) {
            if (qt >= nqt - 1 - (int)blockIdx.x) break;
            __syncthreads();  // every wave is done with the first tile's LDS buffers
        }
        const int h = blockIdx.y, b = blockIdx.z;
        const int G = H / KV, kvh = h / G;
        const int q0 = qt * PF_BQ + wave * 32;
        const size_t qs = (size_t)T * H * HD;
        const float* qb = q + b * qs;
        const _Float16* kbase = K16 + ((size_t)b * KV + kvh) * Tp * HD;
        const _Float16* vbase = Vt16 + ((size_t)b * KV + kvh) * HD * Tp;

        const int kend = min(T, qt * PF_BQ + PF_BQ);
        int kbeg = 0;
        if (window > 0) kbeg = max(0, qt * PF_BQ - window + 1) / PF_BK * PF_BK;
        // per-thread piece coordinates (fixed): K row kr, dims kc; V^T dim vc, keys vr
        int kr[KPT], kc[KPT], vc[KPT], vr[KPT];
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int e = tid + 256 * i;
            kr[i] = e / (HD / 8); kc[i] = (e % (HD / 8)) * 8;
            vc[i] = e / (PF_BK / 8); vr[i] = (e % (PF_BK / 8)) * 8;
        }
        gh_u32x4 pk[KPT], pv[KPT];  // (ext-vector: an array of uint4 structs stays in scratch)
        if (kbeg < kend) {
#pragma unroll
            for (int i = 0; i < KPT; ++i) {
                pk[i] = *(const gh_u32x4*)(kbase + (size_t)(kbeg + kr[i]) * HD + kc[i]);
                pv[i] = *(const gh_u32x4*)(vbase + (size_t)vc[i] * Tp + kbeg + vr[i]);
            }
        }

        const int qj = q0 + (lane & 31), hf = lane >> 5;
        f16x8 qreg[HD / 16];
#pragma unroll
        for (int s = 0; s < HD / 16; ++s) {
            if (qj < T) {
                const float* src = qb + ((size_t)qj * H + h) * HD + 16 * s + 8 * hf;
                // q pre-multiplied by scale * log2(e): the scores come out of the MFMA in log2 units
                const float4 a0 = *(const float4*)src, a1 = *(const float4*)(src + 4);
                const float c = scale * 1.4426950408889634f;
                qreg[s][0] = (_Float16)(a0.x * c); qreg[s][1] = (_Float16)(a0.y * c); qreg[s][2] = (_Float16)(a0.z * c);
                qreg[s][3] = (_Float16)(a0.w * c); qreg[s][4] = (_Float16)(a1.x * c); qreg[s][5] = (_Float16)(a1.y * c);
                qreg[s][6] = (_Float16)(a1.z * c); qreg[s][7] = (_Float16)(a1.w * c);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) qreg[s][e] = (_Float16)0.f;
            }
        }
        f32x16 oacc[HD / 32];
#pragma unroll
        for (int c = 0; c < HD / 32; ++c)
#pragma unroll
            for (int e = 0; e < 16; ++e) oacc[c][e] = 0.f;
        float m_run = -INFINITY, l_run = 0.f;

        int buf = 0;
        for (int k0 = kbeg; k0 < kend; k0 += PF_BK, buf ^= 1) {
#pragma unroll
            for (int i = 0; i < KPT; ++i) {
                *(gh_u32x4*)(sK[buf] + kr[i] * KS + kc[i]) = pk[i];
                *(gh_u32x4*)(sVt[buf] + vc[i] * VS + vr[i]) = pv[i];
            }
            __syncthreads();
            if (k0 + PF_BK < kend) {
                const int kn = k0 + PF_BK;
#pragma unroll
                for (int i = 0; i < KPT; ++i) {
                    pk[i] = *(const gh_u32x4*)(kbase + (size_t)(kn + kr[i]) * HD + kc[i]);
                    pv[i] = *(const gh_u32x4*)(vbase + (size_t)vc[i] * Tp + kn + vr[i]);
                }
            }
            if (k0 > q0 + 31) continue;  // whole tile in this wave's future (uniform per wave)
            const _Float16* cK = sK[buf];
            const _Float16* cV = sVt[buf];
            f32x16 st[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int e = 0; e < 16; ++e) st[t][e] = 0.f;
#pragma unroll
                for (int s = 0; s < HD / 16; ++s) {
                    const f16x8 ka = *(const f16x8*)(cK + (32 * t + (lane & 31)) * KS + 16 * s + 8 * hf);
                    st[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qreg[s], st[t], 0, 0, 0);
                }
            }
            // masks only where the tile crosses the diagonal, the sequence end or the window
            const bool edge = (k0 + PF_BK > q0) || (k0 + PF_BK > T) || (window > 0 && k0 <= q0 + 31 - window + 1);
            if (edge) {
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int key = k0 + 32 * t + 8 * (e >> 2) + 4 * hf + (e & 3);
                        const bool vis = key <= qj && key < T && (window <= 0 || key > qj - window);
                        if (!vis) st[t][e] = -INFINITY;
                    }
            }
            // row maximum over the lane's 32 keys as a tree (no 32-long dependent chain)
            float mx[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) mx[e] = fmaxf(st[0][e], st[1][e]);
#pragma unroll
            for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
                for (int e = 0; e < w; ++e) mx[e] = fmaxf(mx[e], mx[e + w]);
            float tmax = mx[0];
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
            const float m_new = fmaxf(m_run, tmax);
            const float msub = (m_new == -INFINITY) ? 0.f : m_new;  // fully masked row: exp2(-inf) = 0
            const float alpha = __builtin_amdgcn_exp2f(m_run - msub);
            f16x8 pa[4];
            float ps[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float p0 = __builtin_amdgcn_exp2f(st[0][e] - msub), p1 = __builtin_amdgcn_exp2f(st[1][e] - msub);
                pa[e >> 3][e & 7] = (_Float16)p0;
                pa[2 + (e >> 3)][e & 7] = (_Float16)p1;
                ps[e] = p0 + p1;
            }
#pragma unroll
            for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
                for (int e = 0; e < w; ++e) ps[e] += ps[e + w];
            float psum = ps[0];
            psum += __shfl_xor(psum, 32, 64);
            l_run = l_run * alpha + psum;
            const bool moved = m_new != m_run;
            m_run = m_new;
            if (__ballot(moved)) {  // some row maximum moved: rescale (alpha = 1 for the others)
                // the alphas of the wave's 32 rows through LDS: a lane needs rows 8j + 4hf + 0..3
                if (hf == 0) salpha[wave][lane & 31] = alpha;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 a4 = *(const float4*)&salpha[wave][8 * j + 4 * hf];
                    const float ar[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int c = 0; c < HD / 32; ++c) oacc[c][4 * j + i] *= ar[i];
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
#pragma unroll
                for (int c = 0; c < HD / 32; ++c) {
                    const f16x8 vb8 = *(const f16x8*)(cV + (32 * c + (lane & 31)) * VS + 16 * u + 8 * hf);
                    oacc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa[u], vb8, oacc[c], 0, 0, 0);
                }
            }
        }
        const float linv = l_run > 0.f ? 1.0f / l_run : 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int r = 8 * (e >> 2) + 4 * hf + (e & 3);
            const float inv = __shfl(linv, r, 64);
            const int qi = q0 + r;
            if (qi >= T) continue;
            float* dst = out + b * qs + ((size_t)qi * H + h) * HD;
#pragma unroll
            for (int c = 0; c < HD / 32; ++c) dst[32 * c + (lane & 31)] = oacc[c][e] * inv;
        }
    }
}

// Any head_dim (<= 256, multiple of 4): one wave per (query, head), online
// softmax over keys, fp32 throughout. Used for shapes the MFMA kernel does
// not cover.
__global__ void __launch_bounds__(64) k_attn_prefill_simple(const float* __restrict__ q, const float* __restrict__ k,
                                                            const float* __restrict__ v, float* __restrict__ out,
                                                            int T, int H, int KV, int hd, float scale, int window) {
    const int t = blockIdx.x, h = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
    const int kvh = h / (H / KV);
    const size_t qs = (size_t)T * H * hd, kvs = (size_t)T * KV * hd;
    const float* qh = q + b * qs + ((size_t)t * H + h) * hd;
    float qv[4], o[4] = {0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < 4; ++i) qv[i] = (lane + 64 * i < hd) ? qh[lane + 64 * i] : 0.f;
    float m = -INFINITY, l = 0.f;
    const int j0 = (window > 0) ? max(t - window + 1, 0) : 0;
    for (int j = j0; j <= t; ++j) {
        const float* kh = k + b * kvs + ((size_t)j * KV + kvh) * hd;
        float s = 0.f;
        for (int i = 0; i < 4; ++i)
            if (lane + 64 * i < hd) s = fmaf(qv[i], kh[lane + 64 * i], s);
        s = wave_sum(s) * scale;
        const float mn = fmaxf(m, s), al = expf(m - mn), p = expf(s - mn);
        l = l * al + p;
        const float* vh = v + b * kvs + ((size_t)j * KV + kvh) * hd;
        for (int i = 0; i < 4; ++i)
            if (lane + 64 * i < hd) o[i] = o[i] * al + p * vh[lane + 64 * i];
        m = mn;
    }
    float* oh = out + b * qs + ((size_t)t * H + h) * hd;
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    for (int i = 0; i < 4; ++i)
        if (lane + 64 * i < hd) oh[lane + 64 * i] = o[i] * inv;
}

// Decode over the fp16 ring cache with (len, ring start, pinned) taken from
// the device control block; the grid covers the whole cache capacity so the
// launch shape does not depend on the length (capturable in a graph).
int attn_decode_devctl(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int H, int KV, int hd,
                       int cache_max, const int32_t* ctl, float scale) {
    DecodeArgs a{};
    a.q = q; a.k = kc; a.v = vc; a.H = H; a.KV = KV; a.G = H / KV; a.scale = scale;
    a.cache_max = cache_max; a.ctl = ctl; a.j0 = 0;
    return launch_decode<false>(a, hd, 1, cache_max, out);
}

// Partials of the ring-cache decode (device control block), for a merge in
// the consumer: o_part [KV][splits][G][hd], ml [KV][splits][G][2].
int attn_decode_partials_devctl(const float* q, const uint16_t* kc, const uint16_t* vc, int H, int KV, int hd,
                                int cache_max, const int32_t* ctl, float scale, const float** o_part,
                                const float** ml, int* splits) {
    DecodeArgs a{};
    a.q = q; a.k = kc; a.v = vc; a.H = H; a.KV = KV; a.G = H / KV; a.scale = scale;
    a.cache_max = cache_max; a.ctl = ctl; a.j0 = 0;
    const int rc = launch_decode_partials<false>(a, hd, 1, cache_max);
    if (rc) return rc;
    *o_part = a.o_part;
    *ml = a.ml_part;
    *splits = a.splits;
    return GH_OK;
}

int attention_prefill(const float* q, const float* k, const float* v, float* out, int B, int T, int H, int KV, int hd,
                      float scale, int window) {
    if (hd == 64 || hd == 128) {
        const int Tp = cdiv(T, PF_BK) * PF_BK;
        _Float16* kv16 = (_Float16*)workspace(WS_ATTN_KV16, (size_t)B * KV * Tp * hd * 2 * 2);
        if (!kv16) return fail(GH_ENOMEM, "attention prefill: workspace");
        _Float16* K16 = kv16;
        _Float16* Vt16 = kv16 + (size_t)B * KV * Tp * hd;
        const dim3 gs(Tp / PF_BK, KV, B), grid(cdiv(cdiv(T, PF_BQ), 2), H, B);  // q-tiles in pairs
        if (hd == 64) {
            hipLaunchKernelGGL(k_kv_f16<64>, gs, dim3(256), 0, stream(), k, v, K16, Vt16, T, KV, Tp);
            hipLaunchKernelGGL(k_attn_prefill_f16<64>, grid, dim3(256), 0, stream(), q, K16, Vt16, out, T, Tp, H, KV,
                               scale, window);
        } else {
            hipLaunchKernelGGL(k_kv_f16<128>, gs, dim3(256), 0, stream(), k, v, K16, Vt16, T, KV, Tp);
            hipLaunchKernelGGL(k_attn_prefill_f16<128>, grid, dim3(256), 0, stream(), q, K16, Vt16, out, T, Tp, H, KV,
                               scale, window);
        }
        GH_LAUNCHED("k_attn_prefill_f16");
        return GH_OK;
    }
    if (hd == 64 || hd == 128) {
        const dim3 grid(cdiv(T, PF_BQ), H, B);
        if (hd == 64) hipLaunchKernelGGL(k_attn_prefill_mfma<64>, grid, dim3(256), 0, stream(), q, k, v, out, T, H, KV, scale, window);
        else hipLaunchKernelGGL(k_attn_prefill_mfma<128>, grid, dim3(256), 0, stream(), q, k, v, out, T, H, KV, scale, window);
        GH_LAUNCHED("k_attn_prefill_mfma");
        return GH_OK;
    }
    GH_REQUIRE(hd <= 256, "attention_forward_ex: head_dim %d > 256", hd);
    hipLaunchKernelGGL(k_attn_prefill_simple, dim3(T, H, B), dim3(64), 0, stream(), q, k, v, out, T, H, KV, hd, scale,
                       window);
    GH_LAUNCHED("k_attn_prefill_simple");
    return GH_OK;
}

}  // namespace gh

using namespace gh;

extern "C" {

int gh_attention_forward_ex(const float* q, const float* k, const float* v, float* out, float* probs, int B, int T,
                            int H, int KV, int hd, float scale, int window, const int32_t* segment_ids) {
    GH_REQUIRE(probs == nullptr, "attention_forward_ex: probs output is a training feature, not supported");
    GH_REQUIRE(segment_ids == nullptr, "attention_forward_ex: segment masks are not supported");
    GH_REQUIRE(q && k && v && out, "attention_forward_ex: null pointer");
    GH_REQUIRE(B >= 0 && T >= 0 && H > 0 && KV > 0 && H % KV == 0 && hd > 0 && hd % 4 == 0,
               "attention_forward_ex: bad shape B=%d T=%d H=%d KV=%d hd=%d", B, T, H, KV, hd);
    if (B == 0 || T == 0) return GH_OK;
    return attention_prefill(q, k, v, out, B, T, H, KV, hd, scale, window);
}

static int ring_decode_args(DecodeArgs& a, const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int H,
                            int KV, int hd, int ring_start, int pinned, int cur_len, int cache_max, float scale,
                            int window) {
    // core/attn_cpu.cpp:211-222
    GH_REQUIRE(H > 0 && KV > 0 && hd > 0, "attention_decode_ring_fp16: empty shape");
    GH_REQUIRE(H % KV == 0, "attention_decode_ring_fp16: H must be a multiple of KV");
    GH_REQUIRE(cur_len >= 0 && cache_max >= 0 && cur_len <= cache_max,
               "attention_decode_ring_fp16: length exceeds cache capacity");
    GH_REQUIRE(pinned >= 0 && pinned <= cur_len, "attention_decode_ring_fp16: pinned prefix out of range");
    const int cap = cache_max - pinned;
    if (cur_len > pinned) {
        GH_REQUIRE(cap > 0, "attention_decode_ring_fp16: ring has no rolling slots");
        GH_REQUIRE(ring_start >= 0 && ring_start < cap, "attention_decode_ring_fp16: ring start out of range");
    }
    GH_REQUIRE(H / KV <= DEC_GMAX, "attention_decode_ring_fp16: group size %d > %d", H / KV, DEC_GMAX);
    GH_REQUIRE(q && kc && vc && out, "attention_decode_ring_fp16: null pointer");
    a = DecodeArgs{};
    a.q = q; a.k = kc; a.v = vc; a.H = H; a.KV = KV; a.G = H / KV; a.scale = scale;
    a.ring_start = ring_start; a.pinned = pinned; a.cur_len = cur_len; a.cache_max = cache_max;
    a.j0 = (window > 0 && cur_len > window) ? cur_len - window : 0;
    return GH_OK;
}

int gh_attention_decode_ring_fp16(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int H, int KV,
                                  int hd, int ring_start, int pinned, int cur_len, int cache_max, float scale,
                                  float* scratch, int window) {
    (void)scratch;
    DecodeArgs a;
    const int rc = ring_decode_args(a, q, kc, vc, out, H, KV, hd, ring_start, pinned, cur_len, cache_max, scale, window);
    if (rc) return rc;
    return launch_decode<false>(a, hd, 1, cur_len - a.j0, out);
}

// The allocation-free variant: the split-K partials live in `scratch`, a file-scope device
// array each GPU holds once for the life of the process. Its device address is looked up per
// device with hipGetSymbolAddress (the array's name is only a host-side stand-in) on the first
// call on that device. Every call on a GPU uses the same array: calls that overlap on one GPU
// (several streams, several host threads) race on it. Nothing in it needs to start at zero:
// every launch writes all the partials the merge reads.
constexpr size_t NOALLOC_DEC_SCRATCH_BYTES = (size_t)4 << 20;
static __device__ __align__(256) float scratch[NOALLOC_DEC_SCRATCH_BYTES / 4];
constexpr int NOALLOC_MAX_DEVICES = 64;
static float* g_scratch_dev[NOALLOC_MAX_DEVICES];

static int noalloc_scratch(float** out) {
    int dev = 0;
    GH_HIP(hipGetDevice(&dev));
    GH_REQUIRE(dev >= 0 && dev < NOALLOC_MAX_DEVICES, "attention decode (no-alloc): device %d out of range", dev);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(GH_EHIP, "attention decode (no-alloc): hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_dev[dev] = (float*)p;
    }
    *out = g_scratch_dev[dev];
    return GH_OK;
}

int gh_attention_decode_ring_fp16_noalloc(const float* q, const uint16_t* kc, const uint16_t* vc, float* out, int H,
                                          int KV, int hd, int ring_start, int pinned, int cur_len, int cache_max,
                                          float scale, int window) {
    DecodeArgs a;
    int rc = ring_decode_args(a, q, kc, vc, out, H, KV, hd, ring_start, pinned, cur_len, cache_max, scale, window);
    if (rc) return rc;
    size_t ml_off = 0;
    const size_t need = decode_partial_floats(a, hd, 1, cur_len - a.j0, &ml_off) * 4;
    GH_REQUIRE(need <= NOALLOC_DEC_SCRATCH_BYTES,
               "attention_decode_ring_fp16_noalloc: %zu bytes of partials (H=%d hd=%d, %d splits) exceed the %zu-byte "
               "static scratch", need, H, hd, a.splits, NOALLOC_DEC_SCRATCH_BYTES);
    float* ws = nullptr;
    rc = noalloc_scratch(&ws);
    if (rc) return rc;
    return launch_decode<false>(a, hd, 1, cur_len - a.j0, out, ws);
}

int gh_attention_decode_paged_bf16(const float* q, const uint16_t* kp, const uint16_t* vp, const int32_t* page_table,
                                   const int32_t* seq_lens, int n_seqs, int max_pages, int page_size, int max_len,
                                   float* out, int H, int KV, int hd, float scale) {
    GH_REQUIRE(H > 0 && KV > 0 && hd > 0 && H % KV == 0, "attention_decode_paged_bf16: bad heads");
    GH_REQUIRE(H / KV <= DEC_GMAX, "attention_decode_paged_bf16: group size %d > %d", H / KV, DEC_GMAX);
    GH_REQUIRE(n_seqs >= 0 && page_size > 0 && max_pages > 0 && max_len >= 0 && max_len <= max_pages * page_size,
               "attention_decode_paged_bf16: bad paging arguments");
    GH_REQUIRE(q && kp && vp && page_table && seq_lens && out, "attention_decode_paged_bf16: null pointer");
    if (n_seqs == 0) return GH_OK;
    DecodeArgs a{};
    a.q = q; a.k = kp; a.v = vp; a.H = H; a.KV = KV; a.G = H / KV; a.scale = scale;
    a.page_table = page_table; a.seq_lens = seq_lens; a.max_pages = max_pages; a.page_size = page_size;
    return launch_decode<true>(a, hd, n_seqs, max_len, out);
}

}  // extern "C"
