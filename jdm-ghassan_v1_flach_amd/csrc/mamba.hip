// Mamba-2 (Granite-4.0 hybrid) on CDNA4: causal depthwise conv1d, the
// chunked SSD scan and the single-token state update.
//
// The reference runs the selective scan as the sequential per-token
// recurrence (core/mamba_cpu.cpp:120-170, cuda/mamba.cu:148-222: one block
// per (b,h,p) row, serial over T). Here a prefill uses the chunked "state
// space duality" form (chunk L = 256, n_groups = 1):
//   a_t = A_h dt_t,  cum_t = inclusive sum of a within the chunk,
//   y_t = sum_{tau<=t} (C_t.B_tau) e^(cum_t-cum_tau) dt_tau x_tau
//         + e^(cum_t) C_t S_in + D x_t
//   S_out = e^(cum_end) S_in + sum_tau e^(cum_end-cum_tau) dt_tau x_tau B_tau^T
// in three launches: (1) G = C B^T per chunk (shared by all heads, fp16) beside
// the per-chunk state contributions dS on the matrix cores; (2) a pass carrying
// the state across chunks (S_in of every chunk, fp16); (3) per (chunk, head,
// half of the p columns) the chunk's outputs (intra-chunk M X and the C S_in
// correction on the matrix cores), reading X once.
// Decode is one fused conv+update kernel between the two projections.
#include "gemv_fuse.h"

namespace gh {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

int linear_any(const float* x, const void* w, float* y, int M, int K, int N, int kind);
int linear_acc(const float* x, const void* w, float* y, int M, int K, int N, int kind);  // y += x W^T
// gemm.hip: y (+)= norm(x) W^T with the norm on the skinny GEMM's row prologue; mode 1 RMSNorm
// (k_rmsnorm), 2 the RMS norm of already gated rows (k_gated_norm's second half);
// GH_EUNSUPPORTED (nothing launched) off that path, which skinny_takes tells beforehand
int linear_norm_skinny(const float* x, int mode, const float* nw, float eps, const void* w, float* y, int M, int K,
                       int N, int kind, int accumulate);
bool skinny_takes(const void* x, const void* w, int M, int K, int kind);

__device__ __forceinline__ float softplus_ref(float v) {
    // core/mamba_cpu.cpp:139-140 (identity above 20)
    return (v > 20.0f) ? v : log1pf(expf(v));
}

// ================================================================ conv1d
// out[t][c] = silu(b_c + sum_j w[c][j] * raw[t-(k-1)+j][c]), raw = the bc
// part of the projection; the window starts at zero for every sequence
// (core/mamba_cpu.cpp:70-118). Every (t, c) is independent. With `win` (one sequence) the
// threads of the last row also leave the conv window for decode: the last k-1 raw rows.
__global__ void k_conv1d(const float* __restrict__ proj, int proj_ld, int col0, const float* __restrict__ w,
                         const float* __restrict__ b, float* __restrict__ out, int B, int T, int C, int k,
                         float* __restrict__ win) {
#pragma clang fp contract(off)
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int row = blockIdx.y;  // b*T + t
    if (c >= C) return;
    const int t = row % T;
    float acc = b ? b[c] : 0.0f;
    for (int j = 0; j < k; ++j) {
        const int tt = t - (k - 1) + j;
        const float v = tt >= 0 ? proj[(size_t)(row - (k - 1) + j) * proj_ld + col0 + c] : 0.0f;
        acc += w[(size_t)c * k + j] * v;
    }
    out[(size_t)row * C + c] = acc / (1.0f + expf(-acc));
    if (win && row == T - 1) {
        const int wl = k > 1 ? k - 1 : 1;
        for (int j = 0; j < wl; ++j) {
            const int tw = T - wl + j;
            win[(size_t)c * wl + j] = tw >= 0 ? proj[(size_t)tw * proj_ld + col0 + c] : 0.f;
        }
    }
}

// The per-position decay data of (chunk c, head h), by one wave: dt = softplus(dt_raw +
// dt_bias), A = -exp(A_log), cum = the chunk-local inclusive sums of A dt. Into the LDS arrays
// ldt / lcum ([L]) of the calling block, and for the chunk-output blocks as four contiguous
// arrays of 256 (log2 units, zeros past the sequence end) that they load whole: W[0] cum,
// W[1] dt, W[2] the factored intra-chunk weight e^(r_s - cum_tau) dt_tau (r_s = cum at the first
// position of tau's 16-step); F[s] = 1 when every position of 16-step s keeps
// r_s - cum_tau < 100 (log2), i.e. the factored form cannot overflow (one writer per step).
__device__ __forceinline__ void ssd_prep_wave(const float* __restrict__ dt_in, int dt_ld,
                                              const float* __restrict__ dt_bias, const float* __restrict__ A_in,
                                              const float* __restrict__ a_log, float* __restrict__ W,
                                              int* __restrict__ F, int T, int L, int c, int h, int lane, float* ldt,
                                              float* lcum) {
    constexpr float LOG2E = 1.4426950408889634f;
    const int t0 = c * L, len = min(L, T - t0);
    const float A = A_in ? A_in[h] : -expf(a_log[h]);
    // the raw dt of all positions (up to 4 per lane) are requested before the first scan step
    float raws[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = 64 * j + lane;
        raws[j] = i < len ? dt_in[(size_t)(t0 + i) * dt_ld + h] : 0.f;
    }
    float carry = 0.f;  // L <= 256 (ssd_run checks it): at most 4 steps
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = 64 * j + lane;
        const bool v = i < len;
        float dt = 0.f, a = 0.f;
        if (v) {
            const float raw = raws[j];
            dt = dt_bias ? softplus_ref(raw + dt_bias[h]) : raw;
            a = A * dt;
        }
        float inc = a;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float u = __shfl_up(inc, o, 64);
            if (lane >= o) inc += u;
        }
        const float cm = carry + inc;
        if (v) {
            ldt[i] = dt;
            lcum[i] = cm;
        }
        const float cv = v ? cm * LOG2E : 0.f;
        const float rs = __shfl(cv, lane & ~15, 64);  // cum at the step's first position (0 past the end)
        W[i] = cv;
        W[256 + i] = v ? dt : 0.f;
        W[512 + i] = v ? __builtin_amdgcn_exp2f(rs - cv) * dt : 0.f;
        const uint64_t bad = __ballot(v && !((rs - cv) < 100.0f));
        if ((lane & 15) == 0) F[4 * j + (lane >> 4)] = ((bad >> (lane & 48)) & 0xFFFFull) == 0;
        carry += __shfl(inc, 63, 64);
    }
}

// G[c][t][tau] = C_t . B_tau inside chunk c: 64x64 tiles, 4 waves x 32x32 on
// the matrix cores (fp16 operands, fp32 accumulation; G only enters the
// scan as an fp16 operand). C and B rows are staged into LDS with 16-byte loads.
// G and the fp16 C rows are written in MFMA-fragment order, the layout in which the chunk
// outputs take them as A operands: fragment (chunk c, 32-row block rb, 16-column step ks) is
// 64 lanes x 8 halves, lane (r, kh) holding row 32 rb + r, columns 16 ks + 8 kh .. + 7; one
// fragment is one contiguous 1 KB load for a wave (a row-major layout makes each lane of that
// load touch a different row).
__device__ __forceinline__ size_t ssd_frag(int c, int rb, int ks, int nrb, int nks) {
    return (((size_t)c * nrb + rb) * nks + ks) * 512;
}
template <int N>
__device__ __forceinline__ void ssd_cb_block(const float* __restrict__ Bm, const float* __restrict__ Cm, int ld,
                                             _Float16* __restrict__ G, _Float16* __restrict__ C16, int T, int L,
                                             int c, int ti, int si, _Float16* sC, _Float16* sB) {
    constexpr int SN = N + 8;
    const int t0 = c * L, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int e = threadIdx.x; e < 64 * N / 4; e += 256) {
        const int r = (4 * e) / N, k = (4 * e) % N;
        const int tr = t0 + ti + r, sr = t0 + si + r;
        const float4 cv = (ti + r < L && tr < T) ? *(const float4*)(Cm + (size_t)tr * ld + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 bv = (si + r < L && sr < T) ? *(const float4*)(Bm + (size_t)sr * ld + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        f16x4 hc, hb;
        hc[0] = (_Float16)cv.x; hc[1] = (_Float16)cv.y; hc[2] = (_Float16)cv.z; hc[3] = (_Float16)cv.w;
        hb[0] = (_Float16)bv.x; hb[1] = (_Float16)bv.y; hb[2] = (_Float16)bv.z; hb[3] = (_Float16)bv.w;
        *(f16x4*)(sC + r * SN + k) = hc;
        *(f16x4*)(sB + r * SN + k) = hb;
    }
    __syncthreads();
    const int wt = (wave >> 1) * 32, ws = (wave & 1) * 32;
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
    for (int ks = 0; ks < N / 16; ++ks) {
        const int ko = ks * 16 + 8 * (lane >> 5);
        const f16x8 a = *(const f16x8*)(sC + (wt + (lane & 31)) * SN + ko);
        const f16x8 b = *(const f16x8*)(sB + (ws + (lane & 31)) * SN + ko);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
        // the A operand is exactly a C fragment: the si = 0 tiles write the chunk's C rows once
        // (rows past the sequence end are zeros), shared by every head's chunk outputs
        if (si == 0 && ws == 0) *(f16x8*)(C16 + ssd_frag(c, (ti + wt) / 32, ks, L / 32, N / 16) + 8 * lane) = a;
    }
    // G tile -> LDS [t][tau] fp16 (sC is free once every wave has its operands), then out in
    // fragment order, 16 bytes per store
    constexpr int ST = 64 + 8;
    _Float16* sT = sC;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int tl = wt + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3), sl = ws + (lane & 31);
        sT[tl * ST + sl] = (_Float16)acc[e];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int q = threadIdx.x + 256 * j, rbl = q >> 8, ksl = (q >> 6) & 3, ln = q & 63;
        const f16x8 v = *(const f16x8*)(sT + (32 * rbl + (ln & 31)) * ST + 16 * ksl + 8 * (ln >> 5));
        *(f16x8*)(G + ssd_frag(c, ti / 32 + rbl, si / 16 + ksl, L / 32, L / 16) + 8 * ln) = v;
    }
}

// dS[c][h][p][n] = sum_tau e^(cum_end - cum_tau) dt_tau x_tau[p] B_tau[n]
// (P = 64 rows, N cols in 32-wide MFMA tiles), fp16 operands, fp32 acc.
// Stages a [64 rows][W] fp32 tile (row stride ld, a multiple of 4; rows >=
// nvalid read as 0, optionally scaled per row by sw) into LDS as fp16
// TRANSPOSED [W][S]: thread = (4 columns, a run of R = W / 16 consecutive
// rows); each row piece is one 16-byte load (the 64 lanes of a wave cover
// whole rows), and each of the thread's 4 columns is written as one run of R
// halves.
template <int W, int S, bool SCALE>
__device__ __forceinline__ void stage_t64(const float* __restrict__ src, int ld, int nvalid, const float* sw,
                                          _Float16* dst) {
    constexpr int Q = W / 4, G = 256 / Q, R = 64 / G;  // float4 per row, row groups, rows per thread
    static_assert(R == 4 || R == 8, "stage_t64: W must be 64 or 128");
    const int cq = threadIdx.x % Q, g = threadIdx.x / Q;
    float4 v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int r = g * R + i;
        v[i] = r < nvalid ? *(const float4*)(src + (size_t)r * ld + 4 * cq) : make_float4(0.f, 0.f, 0.f, 0.f);
        if (SCALE) {
            const float w = sw[r];
            v[i].x *= w; v[i].y *= w; v[i].z *= w; v[i].w *= w;
        }
    }
    typedef _Float16 hrun __attribute__((ext_vector_type(R)));
    hrun h0, h1, h2, h3;
#pragma unroll
    for (int i = 0; i < R; ++i) {
        h0[i] = (_Float16)v[i].x;
        h1[i] = (_Float16)v[i].y;
        h2[i] = (_Float16)v[i].z;
        h3[i] = (_Float16)v[i].w;
    }
    _Float16* d = dst + (4 * cq) * S + g * R;
    *(hrun*)d = h0;
    *(hrun*)(d + S) = h1;
    *(hrun*)(d + 2 * S) = h2;
    *(hrun*)(d + 3 * S) = h3;
}

// stage_t64 in two halves: the loads (into registers, issued early) and the
// transposed fp16 stores (optionally scaled per row by sw from LDS).
template <int W>
struct Stage64 {
    static constexpr int Q = W / 4, G = 256 / Q, R = 64 / G;
    float4 v[R];
    __device__ __forceinline__ void load(const float* __restrict__ src, int ld, int nvalid, int ltid = -1) {
        const int tx = ltid < 0 ? (int)threadIdx.x : ltid;
        const int cq = tx % Q, g = tx / Q;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int r = g * R + i;
            v[i] = r < nvalid ? *(const float4*)(src + (size_t)r * ld + 4 * cq) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    template <int S>
    __device__ __forceinline__ void store(_Float16* dst, const float* sw, int ltid = -1) const {
        const int tx = ltid < 0 ? (int)threadIdx.x : ltid;
        const int cq = tx % Q, g = tx / Q;
        typedef _Float16 hrun __attribute__((ext_vector_type(R)));
        hrun h0, h1, h2, h3;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const float w = sw ? sw[g * R + i] : 1.0f;
            h0[i] = (_Float16)(v[i].x * w);
            h1[i] = (_Float16)(v[i].y * w);
            h2[i] = (_Float16)(v[i].z * w);
            h3[i] = (_Float16)(v[i].w * w);
        }
        _Float16* d = dst + (4 * cq) * S + g * R;
        *(hrun*)d = h0;
        *(hrun*)(d + S) = h1;
        *(hrun*)(d + 2 * S) = h2;
        *(hrun*)(d + 3 * S) = h3;
    }
};

// The first launch of the scan. Blocks [0, nch H): the chunk state of (chunk, head)
// with the dt / cum prep of that pair done by its first wave (written out for the
// chunk-output launch, kept in LDS here); blocks after that: the G tiles of k_ssd
// cb (they need nothing from the prep), side by side in the same launch.
// dS[c][h][p][n] = sum_tau e^(cum_end - cum_tau) dt_tau x_tau[p] B_tau[n]
// (P = 64 rows, N cols in 32-wide MFMA tiles), fp16 operands, fp32 acc.
template <int N>
__global__ void __launch_bounds__(256) k_ssd_state_cb(const float* __restrict__ xs, int ldx,
                                                      const float* __restrict__ Bm, const float* __restrict__ Cm,
                                                      int ldb, const float* __restrict__ dt_in, int dt_ld,
                                                      const float* __restrict__ dt_bias, const float* __restrict__ A_in,
                                                      const float* __restrict__ a_log, float* __restrict__ W,
                                                      int* __restrict__ F, _Float16* __restrict__ G,
                                                      _Float16* __restrict__ C16, float* __restrict__ dS,
                                                      float* __restrict__ decay, int T, int H, int L,
                                                      float* __restrict__ state, _Float16* __restrict__ Sin16) {
    constexpr int P = 64, TK = 64, S = TK + 8, SN = N + 8;
    constexpr int U_STATE = (P * S + N * S) * 2, U_CB = 2 * 64 * SN * 2;
    __shared__ __attribute__((aligned(16))) unsigned char smem[U_STATE > U_CB ? U_STATE : U_CB];
    const int nch = (T + L - 1) / L;
    if ((int)blockIdx.x >= nch * H) {
        const int nt = L / 64;
        int b = blockIdx.x - nch * H;
        if (nch % 8 == 0 && (nch * H) % 8 == 0) {
            // the tiles of chunk c on XCD c % 8 (block index modulo 8), so one L2 holds that
            // chunk's B and C rows for all its tiles
            const int x = b % 8, k = b / 8;
            b = (x + 8 * (k / (nt * nt))) * nt * nt + k % (nt * nt);
        }
        ssd_cb_block<N>(Bm, Cm, ldb, G, C16, T, L, b / (nt * nt), (b / nt) % nt * 64, b % nt * 64,
                        (_Float16*)smem, (_Float16*)smem + 64 * SN);
        return;
    }
    _Float16* sX = (_Float16*)smem;  // [p][tau]
    _Float16* sB = sX + P * S;       // [n][tau]
    __shared__ float sw[TK], ldt[256], lcum[256];
    const int c = blockIdx.x % nch, h = blockIdx.x / nch;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t0 = c * L, len = min(L, T - t0);
    if (wave == 0)
        ssd_prep_wave(dt_in, dt_ld, dt_bias, A_in, a_log, W + ((size_t)c * H + h) * 768, F + ((size_t)c * H + h) * 16,
                      T, L, c, h, lane, ldt, lcum);
    constexpr int NT = (P / 32) * (N / 32);  // output tiles
    constexpr int TPW = NT / 4;              // tiles per wave
    f32x16 acc[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;
    // the B rows of a chunk are the same for every head: head h starts at tile h mod ntk, so the
    // blocks of one chunk do not all read the same lines at once (that serialises them)
    const int ntk = (len + TK - 1) / TK;
    // the next tile's cum / dt, X rows and B rows are loaded into registers while the current
    // tile is multiplied (no global round trip inside the loop)
    Stage64<P> rx;
    Stage64<N> rb;
    auto prefetch = [&](int kk) {
        const int k0 = ((kk + h) % ntk) * TK;
        rx.load(xs + (size_t)(t0 + k0) * ldx + h * P, ldx, len - k0);
        rb.load(Bm + (size_t)(t0 + k0) * ldb, ldb, len - k0);
    };
    prefetch(0);
    __syncthreads();  // the prep wave's ldt / lcum
    const float cend = lcum[len - 1];
    for (int kk = 0; kk < ntk; ++kk) {
        const int k0 = ((kk + h) % ntk) * TK;
        __syncthreads();  // the previous tile's operands are consumed
        if (threadIdx.x < TK) {
            const int tau = k0 + (int)threadIdx.x;
            sw[threadIdx.x] = tau < len ? expf(cend - lcum[tau]) * ldt[tau] : 0.f;
        }
        __syncthreads();
        rx.template store<S>(sX, sw);
        rb.template store<S>(sB, nullptr);
        __syncthreads();
        if (kk + 1 < ntk) prefetch(kk + 1);
#pragma unroll
        for (int ks = 0; ks < TK / 16; ++ks) {
            const int ko = ks * 16 + 8 * (lane >> 5);
#pragma unroll
            for (int i = 0; i < TPW; ++i) {
                const int tile = wave * TPW + i;
                const int pt = tile % (P / 32), nt = tile / (P / 32);
                const f16x8 a = *(const f16x8*)(sX + (pt * 32 + (lane & 31)) * S + ko);
                const f16x8 b = *(const f16x8*)(sB + (nt * 32 + (lane & 31)) * S + ko);
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[i], 0, 0, 0);
            }
        }
    }
    float* out = dS + ((size_t)c * H + h) * P * N;
    const float dec = expf(cend);
    // a single chunk (state != null): the inter-chunk pass of this head runs here, with
    // k_ssd_state_pass's arithmetic: S_in = state (fp16 for the outputs), state = state dec + dS.
    // Every state value of the lane is loaded before the first store (the compiler cannot tell
    // the stores from the later loads, and would otherwise wait for each load in turn).
    if (state) {
        float sv[TPW][16];
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            const int tile = wave * TPW + i;
            const int pt = tile % (P / 32), nt = tile / (P / 32);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int p = pt * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                sv[i][e] = state[((size_t)h * P + p) * N + nt * 32 + (lane & 31)];
            }
        }
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            const int tile = wave * TPW + i;
            const int pt = tile % (P / 32), nt = tile / (P / 32);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int p = pt * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                const size_t si = ((size_t)h * P + p) * N + nt * 32 + (lane & 31);
                Sin16[si] = (_Float16)sv[i][e];
                state[si] = sv[i][e] * dec + acc[i][e];
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            const int tile = wave * TPW + i;
            const int pt = tile % (P / 32), nt = tile / (P / 32);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int p = pt * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                out[(size_t)p * N + nt * 32 + (lane & 31)] = acc[i][e];
            }
        }
    }
    if (threadIdx.x == 0) decay[(size_t)c * H + h] = dec;
}

// Inter-chunk pass: S_in[c] = the state entering chunk c (written as fp16, the chunk outputs
// MFMA operand), S <- S * decay[c] + dS[c] in fp32 from the incoming state, the final state
// written back. A thread carries 4 consecutive (h, p, n) elements; the dS of all chunks are
// requested before the first step (only the recurrence is serial).
__global__ void __launch_bounds__(256) k_ssd_state_pass(float* __restrict__ state, const float* __restrict__ dS,
                                                        const float* __restrict__ decay, _Float16* __restrict__ Sin16,
                                                        int nch, int H, int PN) {
    const int64_t i4 = (int64_t)blockIdx.x * 256 + threadIdx.x;  // float4 index into [H][PN]
    if (i4 >= (int64_t)H * PN / 4) return;
    const int h = (int)(4 * i4 / PN);
    float4 s = ((const float4*)state)[i4];
    for (int c0 = 0; c0 < nch; c0 += 16) {
        float4 dv[16];
        float dc[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int c = c0 + j;
            if (c < nch) {
                dv[j] = ((const float4*)(dS + (size_t)c * H * PN))[i4];
                dc[j] = decay[(size_t)c * H + h];
            }
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int c = c0 + j;
            if (c < nch) {
                f16x4 hv;
                hv[0] = (_Float16)s.x; hv[1] = (_Float16)s.y; hv[2] = (_Float16)s.z; hv[3] = (_Float16)s.w;
                ((f16x4*)(Sin16 + (size_t)c * H * PN))[i4] = hv;
                s = make_float4(s.x * dc[j] + dv[j].x, s.y * dc[j] + dv[j].y, s.z * dc[j] + dv[j].z,
                                s.w * dc[j] + dv[j].w);
            }
        }
    }
    ((float4*)state)[i4] = s;
}

// Chunk outputs: y[t][p] = sum_{tau<=t} G[t][tau] e^(cum_t-cum_tau) dt_tau x_tau[p]
//                         + e^(cum_t) sum_n C_t[n] S_in[p][n] + D x_t[p].
// A block takes one (chunk, head) and one half of its 64 p columns, all 256 rows: it reads
// the chunk's X columns once (a block per 64-row tile re-read the X rows, G rows and S_in
// each tile needed), and two blocks fit a CU, so one block's loads overlap the other's
// compute. X^T [p][tau] and S_in [p][n] of the block's columns sit in LDS as fp16 (the MFMA B
// operands), D x in fp32 for the epilogue; the A operands come straight from the fp16 G / C
// fragments in global memory (shared by all heads, one contiguous 1 KB load per wave and
// step) and are weighted in registers. Wave w owns the 32-row block w (32 t rows x 32 p, one
// 32x32 MFMA tile, fp32 accumulation). The decay factor is split per 16-position step (one
// exponential per row and step rather than per element).
template <int N, bool GATE = false>
__global__ void __launch_bounds__(512) k_ssd_out(const float* __restrict__ xs, int ldx,
                                                 const _Float16* __restrict__ C16, const _Float16* __restrict__ G,
                                                 const float* __restrict__ W, const int* __restrict__ F,
                                                 const _Float16* __restrict__ Sin16, const float* __restrict__ D,
                                                 float* __restrict__ y, int ldy, int T, int H, int L,
                                                 const float* __restrict__ gate, int ldg) {
    constexpr int P = 64, PH = 32, PN = P * N, SX = 256 + 8, SS = N + 8, SD = PH + 4;
    __shared__ __attribute__((aligned(16))) _Float16 sXt[PH * SX];
    __shared__ __attribute__((aligned(16))) _Float16 sS[PH * SS];
    __shared__ __attribute__((aligned(16))) float sDx[256 * SD];
    __shared__ __attribute__((aligned(16))) float sWt[768];
    __shared__ int sfast[16];
    float* scum = sWt;  // cum (log2 units), dt, factored intra-chunk weight: 256 each
    float* sdt = sWt + 256;
    float* sw = sWt + 512;
    const int nch = (T + L - 1) / L, nitems = nch * H;
    // block b -> item (chunk, head) and p half. The dispatcher places block b on XCD b % 8. With
    // nch a multiple of 8, XCD x takes the chunks x, x + 8, ... of every head (its L2 then
    // fetches only those chunks' G / C fragments, which all heads share), the two halves of an
    // item on its consecutive blocks b, b + 8; otherwise items go round the XCDs, halves again
    // on blocks b and b + 8 (one L2 for the item's X reads).
    const int b = blockIdx.x;
    int c, h, ph;
    if (nch % 8 == 0) {
        const int k = b / 8;  // the block's place on its XCD
        ph = k % 2;
        h = (k / 2) % H;
        c = b % 8 + 8 * (k / (2 * H));
        if (c >= nch) return;
    } else {
        const int it = (b / 16) * 8 + (b % 8);
        ph = (b / 8) % 2;
        if (it >= nitems) return;
        c = nch - 1 - it / H;
        h = it % H;
    }
    const int pc0 = PH * ph;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = c * L, len = min(L, T - t0);
    const int rb = wave, kh = 8 * (lane >> 5), col = lane & 31;
    const bool active = 32 * rb < len;  // wave-uniform
    const int t = 32 * rb + col;        // this lane's A row (chunk-local)
    const bool trow = t < len;
    const int nk = 2 * (rb + 1);        // 16-wide tau steps of the causal range
    // the gate values of this lane's outputs (see the stores), requested first
    float zv[GATE ? 16 : 1];
    if constexpr (GATE) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int tl = 32 * rb + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            zv[e] = tl < len ? gate[(size_t)(t0 + tl) * ldg + h * P + pc0 + col] : 0.f;
        }
    }

    // ---- this wave's C fragments and the first 8 G fragments of its causal range, requested first
    f16x8 craw[N / 16], graw[8];
    const _Float16* gr = G + ssd_frag(c, rb, 0, L / 32, L / 16) + 8 * lane;
    if (active) {
        const _Float16* cr = C16 + ssd_frag(c, rb, 0, L / 32, N / 16) + 8 * lane;
#pragma unroll
        for (int ks = 0; ks < N / 16; ++ks) craw[ks] = *(const f16x8*)(cr + 512 * ks);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
            if (ks < nk) graw[ks] = *(const f16x8*)(gr + 512 * ks);
    }
    // ---- block staging: the chunk's X rows, columns pc0 .. pc0 + 31 -> X^T [p][tau] fp16 and
    // D x [tau][p] fp32; S_in rows pc0 .. -> sS [p][n]; cum (log2 units) / dt
    {
        const int cq = tid % 8, g = tid / 8;  // 4 columns, rows 4 g .. 4 g + 3
        float4 v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 4 * g + i;
            v[i] = r < len ? *(const float4*)(xs + (size_t)(t0 + r) * ldx + h * P + pc0 + 4 * cq)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        const uint2* src = (const uint2*)(Sin16 + ((size_t)c * H + h) * PN + (size_t)pc0 * N);
        constexpr int SJ = PH * N / 4 / 512;  // uint2 (4 halves) per thread
        uint2 sv[SJ];
#pragma unroll
        for (int j = 0; j < SJ; ++j) sv[j] = src[tid + 512 * j];
        // e^(cum_t - cum_tau) = e^(cum_t - r_s) e^(r_s - cum_tau) with r_s = cum at the first
        // position of tau's 16-step: the second factor (times dt_tau) is sw[tau], the first is
        // one exponential per (row, step); a step whose decay spread makes e^(r_s - cum_tau) too
        // large for fp32 is marked in sfast and takes the element-by-element form. All of it
        // comes precomputed from the chunk-state launch, as contiguous arrays.
        if (tid < 384) ((float2*)sWt)[tid] = ((const float2*)(W + ((size_t)c * H + h) * 768))[tid];
        if (tid < 16) sfast[tid] = F[((size_t)c * H + h) * 16 + tid];
#pragma unroll
        for (int j = 0; j < SJ; ++j) {
            const int e = 4 * (tid + 512 * j), p = e / N, n = e % N;
            *(uint2*)(sS + p * SS + n) = sv[j];
        }
        typedef _Float16 hrun __attribute__((ext_vector_type(4)));
        hrun h0, h1, h2, h3;
        const float Dh = D[h];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h0[i] = (_Float16)v[i].x;
            h1[i] = (_Float16)v[i].y;
            h2[i] = (_Float16)v[i].z;
            h3[i] = (_Float16)v[i].w;
            *(float4*)(sDx + (4 * g + i) * SD + 4 * cq) = make_float4(Dh * v[i].x, Dh * v[i].y, Dh * v[i].z, Dh * v[i].w);
        }
        _Float16* d = sXt + (4 * cq) * SX + 4 * g;
        *(hrun*)d = h0;
        *(hrun*)(d + SX) = h1;
        *(hrun*)(d + 2 * SX) = h2;
        *(hrun*)(d + 3 * SX) = h3;
    }
    __syncthreads();
    if (!active) return;

    const float ct = scum[t];
    const float et = trow ? __builtin_amdgcn_exp2f(ct) : 0.f;
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    // inter-chunk term: A = e^(cum_t) C_t, B = S_in
#pragma unroll
    for (int ks = 0; ks < N / 16; ++ks) {
        f16x8 a;
#pragma unroll
        for (int i = 0; i < 8; ++i) a[i] = (_Float16)((float)craw[ks][i] * et);
        const f16x8 bo = *(const f16x8*)(sS + col * SS + 16 * ks + kh);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bo, acc, 0, 0, 0);
    }
    // intra-chunk term over tau < 32 (rb + 1): A = G e^(cum_t - cum_tau) dt_tau (tau <= t). No
    // branch per element (the LDS operands read as vectors, the causal mask a select on the two
    // diagonal steps only: a conditional load per element serialises the wave).
    auto mma = [&](const f16x8& a, int tau0) {
        const f16x8 bo = *(const f16x8*)(sXt + col * SX + tau0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bo, acc, 0, 0, 0);
    };
    f16x8 gn[8];
    const _Float16* gr2 = gr + 512 * 8;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
        if (8 + ks < nk) gn[ks] = *(const f16x8*)(gr2 + 512 * ks);
    bool fast = true;  // wave-uniform: every step of this row block takes the factored form
    for (int ks = 0; ks < nk; ++ks) fast = fast && sfast[ks] != 0;
    auto gfrag = [&](int ks) -> const f16x8& { return ks < 8 ? graw[ks] : gn[ks - 8]; };
    if (fast) {
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) {
            if (ks >= nk) continue;
            const int tau0 = 16 * ks + kh;
            const float rf = trow ? __builtin_amdgcn_exp2f(ct - scum[16 * ks]) : 0.f;
            const float4 w0 = *(const float4*)(sw + tau0), w1 = *(const float4*)(sw + tau0 + 4);
            const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            const f16x8 g = gfrag(ks);
            f16x8 a;
            if (ks >= nk - 2) {  // the two steps that cross the diagonal
#pragma unroll
                for (int i = 0; i < 8; ++i) a[i] = (_Float16)(tau0 + i <= t ? (float)g[i] * rf * wv[i] : 0.f);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) a[i] = (_Float16)((float)g[i] * rf * wv[i]);
            }
            mma(a, tau0);
        }
    } else {
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) {
            if (ks >= nk) continue;
            const int tau0 = 16 * ks + kh;
            const float4 c0 = *(const float4*)(scum + tau0), c1 = *(const float4*)(scum + tau0 + 4);
            const float4 d0 = *(const float4*)(sdt + tau0), d1 = *(const float4*)(sdt + tau0 + 4);
            const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            const float dv[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
            const f16x8 g = gfrag(ks);
            f16x8 a;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float e = __builtin_amdgcn_exp2f(fminf(ct - cv[i], 0.f));  // tau <= t: <= 0
                a[i] = (_Float16)(trow && tau0 + i <= t ? (float)g[i] * e * dv[i] : 0.f);
            }
            mma(a, tau0);
        }
    }
    // + D x, store. acc element e: t row 32 rb + 8(e/4) + 4(lane/32) + e%4, p col pc0 + lane%32.
    // With `gate`, the stored value is the gated one, y * silu(z) (the first step of the Mamba-2
    // gated norm, mamba.hip k_gated_norm's arithmetic), z = gate[t][h P + p].
    if constexpr (GATE) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int tl = 32 * rb + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            if (tl < len)
                y[(size_t)(t0 + tl) * ldy + h * P + pc0 + col] =
                    (acc[e] + sDx[tl * SD + col]) * (zv[e] / (1.0f + expf(-zv[e])));
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int tl = 32 * rb + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        if (tl < len) y[(size_t)(t0 + tl) * ldy + h * P + pc0 + col] = acc[e] + sDx[tl * SD + col];
    }
}

// Runs the chunked scan over rows [0, T) of one sequence.
static int ssd_run(const float* xs, int ldx, const float* Bm, const float* Cm, int ldbc, const float* dt_raw, int dt_ld,
                   const float* dt_bias, const float* A, const float* a_log, const float* D, float* state, float* y,
                   int ldy, int T, int H, int P, int N, int L, const float* gate = nullptr, int ldg = 0) {
    GH_REQUIRE(P == 64, "ssd scan: head_dim %d (the kernels are built for 64)", P);
    GH_REQUIRE(N == 64 || N == 128, "ssd scan: d_state %d (64 or 128)", N);
    GH_REQUIRE(L >= 64 && L <= 256 && L % 64 == 0, "ssd scan: chunk %d (64..256, multiple of 64)", L);
    GH_REQUIRE(ldx % 4 == 0 && ldbc % 4 == 0, "ssd scan: row strides must be multiples of 4");
    const int nch = cdiv(T, L);
    const size_t PN = (size_t)P * N;
    // workspace: decay data W [nch][H][3][256] fp32 + fast flags F [nch][H][16]; dS
    // [nch][H][P][N] fp32; decay [nch][H] fp32; Sin [nch][H][P][N], G [nch][L][L] and C16
    // [nch][L][N] fp16 (G, C16 in fragment order)
    const size_t f_W = (size_t)nch * H * 768, f_F = (size_t)nch * H * 16, f_S = (size_t)nch * H * PN;
    const size_t f_dec = ((size_t)nch * H + 63) / 64 * 64;
    const size_t h_G = (size_t)nch * L * L, h_C = (size_t)nch * L * N;
    float* ws = (float*)workspace(WS_MAMBA_CHUNK, (f_W + f_F + f_S + f_dec) * 4 + (f_S + h_G + h_C) * 2 + 256);
    if (!ws) return fail(GH_ENOMEM, "ssd scan: workspace");
    float* W = ws;
    int* F = (int*)(W + f_W);
    float* dS = (float*)(F + f_F);
    float* decay = dS + f_S;
    _Float16* Sin16 = (_Float16*)(decay + f_dec);
    _Float16* G = Sin16 + f_S;
    _Float16* C16 = G + h_G;
    const unsigned nb1 = (unsigned)(nch * H + nch * (L / 64) * (L / 64));  // chunk states, then G tiles
    const unsigned nbp = (unsigned)(((size_t)H * PN / 4 + 255) / 256);
    const bool one = nch == 1;  // a single chunk: the state pass runs in the chunk-state blocks
    if (N == 128) {
        hipLaunchKernelGGL(k_ssd_state_cb<128>, dim3(nb1), dim3(256), 0, stream(), xs, ldx, Bm, Cm, ldbc, dt_raw, dt_ld,
                           dt_bias, A, a_log, W, F, G, C16, dS, decay, T, H, L, one ? state : nullptr, Sin16);
        if (!one)
            hipLaunchKernelGGL(k_ssd_state_pass, dim3(nbp), dim3(256), 0, stream(), state, dS, decay, Sin16, nch, H,
                               (int)PN);
        if (gate)
            hipLaunchKernelGGL((k_ssd_out<128, true>), dim3((unsigned)(2 * cdiv(nch * H, 8) * 8)), dim3(512), 0, stream(), xs,
                               ldx, C16, G, W, F, Sin16, D, y, ldy, T, H, L, gate, ldg);
        else
            hipLaunchKernelGGL((k_ssd_out<128, false>), dim3((unsigned)(2 * cdiv(nch * H, 8) * 8)), dim3(512), 0, stream(), xs,
                               ldx, C16, G, W, F, Sin16, D, y, ldy, T, H, L, nullptr, 0);
    } else {
        hipLaunchKernelGGL(k_ssd_state_cb<64>, dim3(nb1), dim3(256), 0, stream(), xs, ldx, Bm, Cm, ldbc, dt_raw, dt_ld,
                           dt_bias, A, a_log, W, F, G, C16, dS, decay, T, H, L, one ? state : nullptr, Sin16);
        if (!one)
            hipLaunchKernelGGL(k_ssd_state_pass, dim3(nbp), dim3(256), 0, stream(), state, dS, decay, Sin16, nch, H,
                               (int)PN);
        if (gate)
            hipLaunchKernelGGL((k_ssd_out<64, true>), dim3((unsigned)(2 * cdiv(nch * H, 8) * 8)), dim3(512), 0, stream(), xs,
                               ldx, C16, G, W, F, Sin16, D, y, ldy, T, H, L, gate, ldg);
        else
            hipLaunchKernelGGL((k_ssd_out<64, false>), dim3((unsigned)(2 * cdiv(nch * H, 8) * 8)), dim3(512), 0, stream(), xs,
                               ldx, C16, G, W, F, Sin16, D, y, ldy, T, H, L, nullptr, 0);
    }
    GH_LAUNCHED("k_ssd_*");
    return GH_OK;
}

// ============================================================ gated norm
// rmsnorm(y * silu(z)) * w with the sum of squares in double and the
// inverse root in fp32 (core/mamba_cpu.cpp:172-193). One block per row.
__global__ void __launch_bounds__(256) k_gated_norm(const float* __restrict__ y, int ldy, const float* __restrict__ z,
                                                    int ldz, const float* __restrict__ w, float* __restrict__ out,
                                                    int n, float eps) {
    const int r = blockIdx.x;
    const float* yr = y + (size_t)r * ldy;
    const float* zr = z + (size_t)r * ldz;
    float* o = out + (size_t)r * n;
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float g = zr[i] / (1.0f + expf(-zr[i]));
        const float v = yr[i] * g;
        o[i] = v;
        ss += (double)v * v;
    }
    __shared__ double red[4];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const double var = (red[0] + red[1] + red[2] + red[3]) / (double)n;
    const float inv = 1.0f / sqrtf((float)var + eps);
    for (int i = threadIdx.x; i < n; i += 256) o[i] = o[i] * inv * w[i];
}

// ======================================================== decode step
// Conv over the carried window [conv_dim][k-1] + the new raw value, SiLU,
// window shift (inference/generator.cpp:534-559). One thread per channel.
__global__ void k_step_conv(const float* __restrict__ raw, const float* __restrict__ w, const float* __restrict__ b,
                            float* __restrict__ win, float* __restrict__ out, int C, int k) {
#pragma clang fp contract(off)
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    const int wl = k > 1 ? k - 1 : 1;
    float* wc = win + (size_t)c * wl;
    const float rv = raw[c];
    float acc = b ? b[c] : 0.0f;
    for (int j = 0; j < k; ++j) acc += w[(size_t)c * k + j] * ((j == k - 1) ? rv : wc[j]);
    out[c] = acc / (1.0f + expf(-acc));
    for (int j = 0; j + 1 < wl; ++j) wc[j] = wc[j + 1];
    wc[wl - 1] = rv;
}

// State update of one token (inference/generator.cpp:570-594):
// s = e^(A dt) s + (B dt) x,  y = C.s + D x. Block = (head, 16 rows of P);
// thread = (row, 8 consecutive states); the 1.5 MB state streams through
// once in 16-byte loads/stores.
template <int N>
__global__ void __launch_bounds__(256) k_step_scan(const float* __restrict__ xbc, const float* __restrict__ dtr,
                                                   const float* __restrict__ dt_bias, const float* __restrict__ a_log,
                                                   const float* __restrict__ D, float* __restrict__ ssm,
                                                   float* __restrict__ y, int d_inner, int P) {
    constexpr int TPR = N / 8;          // threads per state row
    constexpr int ROWS = 256 / TPR;     // rows per block
    const int h = blockIdx.y, r0 = blockIdx.x * ROWS;
    const int tr = threadIdx.x / TPR, tc = threadIdx.x % TPR;
    const int p = r0 + tr;
    if (p >= P) return;
    const float a = -expf(a_log[h]);
    const float dtb = dtr[h] + dt_bias[h];
    const float dt = (dtb > 20.0f) ? dtb : log1pf(expf(dtb));
    const float dA = expf(a * dt);
    const int i = h * P + p;
    const float xv = xbc[i];
    const float* Bm = xbc + d_inner;
    const float* Cm = Bm + N;
    float* srow = ssm + (size_t)i * N + tc * 8;
    float4 s0 = *(float4*)srow, s1 = *(float4*)(srow + 4);
    float s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int n = tc * 8 + j;
        s[j] = dA * s[j] + (Bm[n] * dt) * xv;
        acc = fmaf(Cm[n], s[j], acc);
    }
    *(float4*)srow = make_float4(s[0], s[1], s[2], s[3]);
    *(float4*)(srow + 4) = make_float4(s[4], s[5], s[6], s[7]);
    acc = group_sum(acc, TPR);
    if (tc == 0) y[i] = acc + D[h] * xv;
}

// One sequence of T tokens: in_proj, conv1d (+ optionally the conv window
// left for decode), chunked scan, gated norm, out_proj. kind 0-3 packed,
// 4 fp16 weights.
// pre_nw: x is first RMS-normalised with these weights (eps pre_eps), on the in_proj GEMM's row
// prologue where the skinny path takes it, else by one k_rmsnorm launch; null: x is used as is.
int mamba_forward_impl(const float* x, const void* w_in, const float* conv_w, const float* conv_b,
                       const float* dt_bias, const float* a_log, const float* D, const float* norm_w, const void* w_out,
                       float* state, float* conv_state, float* out, int T, int d, int d_inner, int conv_dim,
                       int n_heads, int d_head, int d_state, int k, float eps, int kind, bool accumulate,
                       const float* pre_nw, float pre_eps) {
    GH_REQUIRE(conv_dim - d_inner == 2 * d_state, "mamba: inconsistent conv_dim / d_state (n_groups must be 1)");
    GH_REQUIRE(n_heads * d_head == d_inner, "mamba: n_heads * d_head != d_inner");
    const int proj = d_inner + conv_dim + n_heads;
    float* pr = (float*)workspace(WS_MAMBA_PROJ, (size_t)T * proj * 4);
    float* xbc = (float*)workspace(WS_MAMBA_XBC, (size_t)T * conv_dim * 4);
    float* yb = (float*)workspace(WS_MAMBA_Y, (size_t)T * d_inner * 4 * 2);
    if (!pr || !xbc || !yb) return fail(GH_ENOMEM, "mamba: workspace");
    float* normed = yb + (size_t)T * d_inner;
    int rc = GH_EUNSUPPORTED;
    if (pre_nw) {
        rc = linear_norm_skinny(x, 1, pre_nw, pre_eps, w_in, pr, T, d, proj, kind, 0);
        if (rc == GH_EUNSUPPORTED) {  // the norm as its own launch, into the (later) gated-norm rows
            float* xn = (float*)workspace(WS_MAMBA_XN, (size_t)T * d * 4);
            if (!xn) return fail(GH_ENOMEM, "mamba: workspace");
            rc = gh_rmsnorm_forward(x, pre_nw, xn, nullptr, T, d, pre_eps);
            if (!rc) rc = linear_any(xn, w_in, pr, T, d, proj, kind);
        }
    } else {
        rc = linear_any(x, w_in, pr, T, d, proj, kind);
    }
    if (rc) return rc;
    hipLaunchKernelGGL(k_conv1d, dim3(cdiv(conv_dim, 256), T), dim3(256), 0, stream(), pr, proj, d_inner, conv_w,
                       conv_b, xbc, 1, T, conv_dim, k, conv_state);
    GH_LAUNCHED("k_conv1d");
    // where the skinny GEMM takes out_proj, the scan's stores apply the gate (y * silu(z)) and the
    // GEMM's row prologue the RMS norm; otherwise k_gated_norm does both as its own launch
    const bool gate_fused = skinny_takes(yb, w_out, T, d_inner, kind) && ((uintptr_t)norm_w & 15) == 0;
    rc = ssd_run(xbc, conv_dim, xbc + d_inner, xbc + d_inner + d_state, conv_dim, pr + d_inner + conv_dim, proj,
                 dt_bias, nullptr, a_log, D, state, yb, d_inner, T, n_heads, d_head, d_state, 256,
                 gate_fused ? pr : nullptr, proj);
    if (rc) return rc;
    if (gate_fused) return linear_norm_skinny(yb, 2, norm_w, eps, w_out, out, T, d_inner, d, kind, accumulate ? 1 : 0);
    hipLaunchKernelGGL(k_gated_norm, dim3(T), dim3(256), 0, stream(), yb, d_inner, pr, proj, norm_w, normed, d_inner,
                       eps);
    GH_LAUNCHED("k_gated_norm");
    return accumulate ? linear_acc(normed, w_out, out, T, d_inner, d, kind)
                      : linear_any(normed, w_out, out, T, d_inner, d, kind);
}

// Single-token Mamba-2 layer as three launches: (1) [RMSNorm] + in_proj
// with the conv step + SiLU + window shift in its epilogue, (2) the state
// update, (3) gated norm + out_proj [+ residual add into `out`]. Returns
// GH_EUNSUPPORTED (launching nothing) if the shapes do not fit the fused GEMV.
int mamba_step_fused(const float* x, const float* nw, float norm_eps, const void* w_in, const float* conv_w,
                     const float* conv_b, const float* dt_bias, const float* a_log, const float* D,
                     const float* norm_w, const void* w_out, float* conv_state, float* ssm_state, float* out,
                     bool add, int d, int d_inner, int conv_dim, int n_heads, int d_head, int d_state, int k,
                     float eps, int kind, const GmFuse* begin) {
    if ((kind != 2 && kind != 3) || d % 256 || d_inner % 256 || (d_state != 64 && d_state != 128))
        return GH_EUNSUPPORTED;
    if (begin && !nw) return GH_EUNSUPPORTED;  // the step's start rides on the norm prologue
    const int proj = d_inner + conv_dim + n_heads;
    float* pr = (float*)workspace(WS_MAMBA_PROJ, (size_t)proj * 4);
    float* yb = (float*)workspace(WS_MAMBA_Y, (size_t)d_inner * 4 * 2);
    if (!pr || !yb) return fail(GH_ENOMEM, "mamba: workspace");
    GmFuse f1;
    f1.pro = nw ? GM_PRO_RMSNORM : GM_PRO_NONE;
    f1.pw = nw;
    f1.eps = norm_eps;
    f1.epi = GM_EPI_CONV;
    f1.conv_w = conv_w;
    f1.conv_b = conv_b;
    f1.conv_win = conv_state;
    f1.c0 = d_inner;
    f1.cdim = conv_dim;
    f1.ck = k;
    if (begin) {
        f1.emb = begin->emb;
        f1.emb_out = begin->emb_out;
        f1.bctl = begin->bctl;
        f1.vocab = begin->vocab;
    }
    int rc = gemv_fused(x, w_in, pr, d, proj, kind, f1);
    if (rc) return rc;
    const float* xbc = pr + d_inner;  // conv output, in place of the raw xBC
    const int rows_per_block = 256 / (d_state / 8);
    if (d_state == 128)
        hipLaunchKernelGGL(k_step_scan<128>, dim3(cdiv(d_head, rows_per_block), n_heads), dim3(256), 0, stream(), xbc,
                           pr + d_inner + conv_dim, dt_bias, a_log, D, ssm_state, yb, d_inner, d_head);
    else
        hipLaunchKernelGGL(k_step_scan<64>, dim3(cdiv(d_head, rows_per_block), n_heads), dim3(256), 0, stream(), xbc,
                           pr + d_inner + conv_dim, dt_bias, a_log, D, ssm_state, yb, d_inner, d_head);
    GH_LAUNCHED("k_step_scan");
    GmFuse f3;
    f3.pro = GM_PRO_GATED;
    f3.pz = pr;  // z = in_proj rows [0, d_inner)
    f3.pw = norm_w;
    f3.eps = eps;
    f3.epi = add ? GM_EPI_ADD : GM_EPI_STORE;
    rc = gemv_fused(yb, w_out, out, d_inner, d, kind, f3);
    // GH_EUNSUPPORTED means "nothing launched, take another path" only before the first launch:
    // here the in_proj has already advanced the conv window and the scan the SSM state
    if (rc == GH_EUNSUPPORTED)
        return fail(GH_EINVAL, "mamba step: out_proj (K=%d N=%d kind %d) unsupported after the state advanced",
                    d_inner, d, kind);
    return rc;
}

}  // namespace gh

using namespace gh;

extern "C" {

int gh_ssd_scan(const float* xs, const float* Bm, const float* Cm, const float* dt, const float* A, const float* D,
                float* state, float* y, int T, int H, int P, int N, int chunk) {
    GH_REQUIRE(xs && Bm && Cm && dt && A && D && state && y, "ssd_scan: null pointer");
    if (T <= 0) return GH_OK;
    if (chunk <= 0) chunk = 256;
    // B and C are separate [T][N] arrays here: both use row stride N
    return ssd_run(xs, H * P, Bm, Cm, N, dt, H, nullptr, A, nullptr, D, state, y, H * P, T, H, P, N, chunk);
}

int gh_mamba2_forward_half(const float* x, const void* w_in, const float* conv_w, const float* conv_b,
                           const float* dt_bias, const float* a_log, const float* D, const float* norm_w,
                           const void* w_out, float* state, float* out, int B, int T, int d, int d_inner,
                           int conv_dim, int n_heads, int d_head, int d_state, int k, float eps, int qkind) {
    if (B <= 0 || T <= 0) return GH_OK;
    GH_REQUIRE(x && w_in && conv_w && dt_bias && a_log && D && norm_w && w_out && state && out,
               "mamba2_forward: null pointer");
    GH_REQUIRE(qkind >= -1 && qkind <= 3, "mamba: unknown qkind %d", qkind);
    const int kind = qkind < 0 ? 4 : qkind;  // fp16 weights use the fp16 linear path
    for (int b = 0; b < B; ++b) {
        int rc = mamba_forward_impl(x + (size_t)b * T * d, w_in, conv_w, conv_b, dt_bias, a_log, D, norm_w, w_out,
                                    state + (size_t)b * n_heads * d_head * d_state, nullptr, out + (size_t)b * T * d,
                                    T, d, d_inner, conv_dim, n_heads, d_head, d_state, k, eps, kind, false,
                                    nullptr, 0.0f);
        if (rc) return rc;
    }
    return GH_OK;
}

int gh_mamba2_step_half(const float* x, const void* w_in, const float* conv_w, const float* conv_b,
                        const float* dt_bias, const float* a_log, const float* D, const float* norm_w,
                        const void* w_out, float* conv_state, float* ssm_state, float* out, int d, int d_inner,
                        int conv_dim, int n_heads, int d_head, int d_state, int k, float eps, int qkind) {
    GH_REQUIRE(x && w_in && conv_w && dt_bias && a_log && D && norm_w && w_out && conv_state && ssm_state && out,
               "mamba2_step: null pointer");
    GH_REQUIRE(conv_dim - d_inner == 2 * d_state, "mamba: inconsistent conv_dim / d_state (n_groups must be 1)");
    GH_REQUIRE(n_heads * d_head == d_inner, "mamba: n_heads * d_head != d_inner");
    GH_REQUIRE(d_state == 64 || d_state == 128, "mamba2_step: d_state %d (64 or 128)", d_state);
    GH_REQUIRE(qkind >= -1 && qkind <= 3, "mamba: unknown qkind %d", qkind);
    const int kind = qkind < 0 ? 4 : qkind;
    {
        const int rc = mamba_step_fused(x, nullptr, 0.f, w_in, conv_w, conv_b, dt_bias, a_log, D, norm_w, w_out,
                                        conv_state, ssm_state, out, false, d, d_inner, conv_dim, n_heads, d_head,
                                        d_state, k, eps, kind, nullptr);
        if (rc != GH_EUNSUPPORTED) return rc;
    }
    const int proj = d_inner + conv_dim + n_heads;
    float* pr = (float*)workspace(WS_MAMBA_PROJ, (size_t)proj * 4);
    float* xbc = (float*)workspace(WS_MAMBA_XBC, (size_t)conv_dim * 4);
    float* yb = (float*)workspace(WS_MAMBA_Y, (size_t)d_inner * 4 * 2);
    if (!pr || !xbc || !yb) return fail(GH_ENOMEM, "mamba: workspace");
    float* normed = yb + d_inner;
    int rc = linear_any(x, w_in, pr, 1, d, proj, kind);
    if (rc) return rc;
    hipLaunchKernelGGL(k_step_conv, dim3(cdiv(conv_dim, 256)), dim3(256), 0, stream(), pr + d_inner, conv_w, conv_b,
                       conv_state, xbc, conv_dim, k);
    const int rows_per_block = 256 / (d_state / 8);
    if (d_state == 128)
        hipLaunchKernelGGL(k_step_scan<128>, dim3(cdiv(d_head, rows_per_block), n_heads), dim3(256), 0, stream(), xbc,
                           pr + d_inner + conv_dim, dt_bias, a_log, D, ssm_state, yb, d_inner, d_head);
    else
        hipLaunchKernelGGL(k_step_scan<64>, dim3(cdiv(d_head, rows_per_block), n_heads), dim3(256), 0, stream(), xbc,
                           pr + d_inner + conv_dim, dt_bias, a_log, D, ssm_state, yb, d_inner, d_head);
    hipLaunchKernelGGL(k_gated_norm, dim3(1), dim3(256), 0, stream(), yb, d_inner, pr, proj, norm_w, normed, d_inner,
                       eps);
    GH_LAUNCHED("k_step_*");
    return linear_any(normed, w_out, out, 1, d_inner, d, kind);
}

}  // extern "C"
