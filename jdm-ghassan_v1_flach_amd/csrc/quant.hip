// Quantized weights on the device: block decode (dequantise /
// quant_materialize) and the dequant-fused decode GEMV.
//
// Replaces cuda/kernels.cu:482-598 (k_dequant_quant, k_linear_q4_fused: one
// thread per output walking K with 1-2 byte loads) and the fp16 / fp32
// linear paths used for the lm_head and the router (cuda/kernels.cu:447-633).
//
// GEMV layout (M <= 8, HBM-bound): a wave owns R output rows and walks K in
// "tasks" of 64 values; a task is one contiguous, 4-byte aligned byte run of
// the packed row (Q8_0: 2 blocks = 68 B, Q4_0: 36 B, Q4_1: 40 B, Q4_K: the
// 16 B block header + 32 B of nibbles for 2 sub-blocks, fp16: 128 B, fp32:
// 256 B). Lanes take consecutive tasks, so one wave-wide load instruction
// covers a contiguous stretch of the row and every fetched byte is used. The
// 64 activation values of a task stay in registers and are reused for all R
// rows of the wave, which keeps the activation re-reads off the critical L1
// path. Partial sums are reduced with cross-lane shuffles.
#include <stdlib.h>

#include "gh_common.h"

namespace gh {

// ------------------------------------------------------------ block decode
// Value j of a block, with exactly the reference's arithmetic
// (core/ops.cpp:310-328 for kinds 0-2; GGML block_q4_K for kind 3):
// no multiply-add fusion, so the fp32 result is bit-identical to the CPU's.
__device__ __forceinline__ float deq_value(int kind, const uint8_t* blk, int j) {
#pragma clang fp contract(off)
    const float d = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    if (kind == 2) return (float)(int8_t)blk[2 + j] * d;
    if (kind == 0) {
        const uint8_t b = blk[2 + (j & 15)];
        const int q = (j < 16) ? (b & 0xF) : (b >> 4);
        return (float)(q - 8) * d;
    }
    if (kind == 1) {
        const float mn = f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
        const uint8_t b = blk[4 + (j & 15)];
        const int q = (j < 16) ? (b & 0xF) : (b >> 4);
        return (float)q * d + mn;
    }
    // Q4_K
    const float dmin = f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
    const uint8_t* sc = blk + 4;
    const int s = j >> 5, l = j & 31;
    int scv, mv;
    if (s < 4) {
        scv = sc[s] & 63;
        mv = sc[s + 4] & 63;
    } else {
        scv = (sc[s + 4] & 0xF) | ((sc[s - 4] >> 6) << 4);
        mv = (sc[s + 4] >> 4) | ((sc[s] >> 6) << 4);
    }
    const uint8_t byte = blk[16 + 32 * (s >> 1) + l];
    const int q = (s & 1) ? (byte >> 4) : (byte & 0xF);
    const float d1 = d * (float)scv, m1 = dmin * (float)mv;
    return d1 * (float)q - m1;
}

// One thread per 8 consecutive values (a block is 32 or 256 values).
template <bool TO_F16>
__global__ void __launch_bounds__(256) k_dequant(const uint8_t* __restrict__ p, int kind, int64_t n,
                                                 void* __restrict__ out) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t i0 = g * 8;
    if (i0 >= n) return;
    const int bv = block_values(kind), bb = block_bytes(kind);
    const uint8_t* blk = p + (i0 / bv) * bb;
    const int j0 = (int)(i0 % bv);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        if (i0 + t >= n) break;
        const float v = deq_value(kind, blk, j0 + t);
        if (TO_F16) ((uint16_t*)out)[i0 + t] = f32_to_f16(v);
        else ((float*)out)[i0 + t] = v;
    }
}

}  // namespace gh

#include "gemv_tasks.h"

namespace gh {

// Persistent, software-pipelined GEMV. LPR lanes share one row (LPR | 64),
// 64/LPR rows run side by side and each lane repeats that for R rows, so a
// wave covers R*64/LPR rows per "group". Waves stride over the groups; the
// packed bytes of the next (group, task) step are loaded before the current
// step is decoded and multiplied, so every wave keeps a full set of weight
// loads in flight while it computes.
template <int KIND, int MT, int R>
__global__ void __launch_bounds__(256) k_gemv(const float* __restrict__ x, const uint8_t* __restrict__ W,
                                              float* __restrict__ y, int M, int K, int N, size_t rowb, int LPR) {
    const int lane = threadIdx.x & 63;
    const int RP = 64 / LPR;
    const int sub = lane % LPR, rp = lane / LPR;
    const int T = K / 64;
    const int TI = (T + LPR - 1) / LPR;           // task iterations per row (lane-uniform count)
    const int rows_per_wave = R * RP;
    const int ngroups = (N + rows_per_wave - 1) / rows_per_wave;
    const int wstride = gridDim.x * 4;
    int grp = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (grp >= ngroups) return;
    const int nsteps = ((ngroups - 1 - grp) / wstride + 1) * TI;

    auto step_rows = [&](int g, int* rows) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = g * rows_per_wave + rp + RP * r;
            rows[r] = n < N ? n : N - 1;
        }
    };
    uint32_t wc[R][Task<KIND>::DW], wn[R][Task<KIND>::DW];
    int rows[R];
    step_rows(grp, rows);
    {
        const int t = sub < T ? sub : T - 1;
#pragma unroll
        for (int r = 0; r < R; ++r) load_task<KIND>(W + (size_t)rows[r] * rowb, t, wc[r]);
    }
    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;
    int ti = 0;
    // MT == 1: the activations of the lane's task are loaded BEFORE the next
    // step's weight prefetch is issued (vmcnt waits are in order, so loading
    // them after the prefetch would make every step wait for the prefetch),
    // and only once when the lane keeps the same task for all steps.
    float x1[64], xs1[2];
    auto load_x1 = [&](int t) {
        const float4* xp = (const float4*)(x + (size_t)(t < T ? t : T - 1) * 64);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 v = xp[i];
            x1[4 * i] = v.x; x1[4 * i + 1] = v.y; x1[4 * i + 2] = v.z; x1[4 * i + 3] = v.w;
        }
        task_xsum<KIND>(x1, xs1);
    };
    if (MT == 1) load_x1(sub);
    for (int st = 0; st < nsteps; ++st) {
        const int t = sub + ti * LPR;
        if (MT == 1 && TI > 1 && st > 0) load_x1(t);
        // prefetch the next step
        const bool more = st + 1 < nsteps;
        const int nti = (ti + 1 == TI) ? 0 : ti + 1;
        const int ngrp = (ti + 1 == TI) ? grp + wstride : grp;
        int nrows[R];
        if (more) {
            step_rows(ngrp, nrows);
            int tn = sub + nti * LPR;
            tn = tn < T ? tn : T - 1;
#pragma unroll
            for (int r = 0; r < R; ++r) load_task<KIND>(W + (size_t)nrows[r] * rowb, tn, wn[r]);
        }
        if (t < T) {
            if (MT == 1) {
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r][0] += task_dot<KIND>(wc[r], x1, xs1, t);
            } else {
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    if (m >= M) break;
                    float xv[64];
                    const float4* xp = (const float4*)(x + (size_t)m * K + (size_t)t * 64);
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const float4 v = xp[i];
                        xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
                    }
                    float xs[2];
                    task_xsum<KIND>(xv, xs);
#pragma unroll
                    for (int r = 0; r < R; ++r) acc[r][m] += task_dot<KIND>(wc[r], xv, xs, t);
                }
            }
        }
        if (ti + 1 == TI) {  // group done: reduce and store
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    float v = acc[r][m];
                    v = group_sum(v, LPR);
                    const int n = grp * rows_per_wave + rp + RP * r;
                    if (sub == 0 && m < M && n < N) y[(size_t)m * N + n] = v;
                    acc[r][m] = 0.f;
                }
        }
        grp = ngrp;
        ti = nti;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < Task<KIND>::DW; ++i) wc[r][i] = wn[r][i];
    }
}

// waves per CU of the persistent grid and rows per lane of the single-token GEMV
static int gemv_wpc() { return 8; }
static int gemv_r() { return 2; }

template <int KIND, int MT, int R>
static int launch_gemv_t(const float* x, const void* w, float* y, int M, int K, int N, size_t rowb) {
    const int T = K / 64;
    int LPR = 64;
    while (LPR > 1 && LPR > T) LPR >>= 1;
    const int rows_per_wave = R * (64 / LPR);
    const int groups = cdiv(N, rows_per_wave);
    // persistent grid: at most gemv_wpc() waves per CU, fewer when there is less work
    const int max_waves = gemv_wpc() * num_cus();
    const int waves = groups < max_waves ? groups : max_waves;
    hipLaunchKernelGGL((k_gemv<KIND, MT, R>), dim3(cdiv(waves, 4)), dim3(256), 0, stream(), x,
                       (const uint8_t*)w, y, M, K, N, rowb, LPR);
    GH_LAUNCHED("k_gemv");
    return GH_OK;
}

template <int KIND>
static int launch_gemv(const float* x, const void* w, float* y, int M, int K, int N, size_t rowb) {
    if (M == 1) {
        const int r = gemv_r();
        if (r == 1) return launch_gemv_t<KIND, 1, 1>(x, w, y, M, K, N, rowb);
        if (r == 4) return launch_gemv_t<KIND, 1, 4>(x, w, y, M, K, N, rowb);
        return launch_gemv_t<KIND, 1, 2>(x, w, y, M, K, N, rowb);
    }
    if (M == 2) return launch_gemv_t<KIND, 2, 2>(x, w, y, M, K, N, rowb);
    if (M <= 4) return launch_gemv_t<KIND, 4, 1>(x, w, y, M, K, N, rowb);
    return launch_gemv_t<KIND, 8, 1>(x, w, y, M, K, N, rowb);
}

int gemv1_dispatch(const float* x, const void* w, float* y, int K, int N, int kind, int* rc);  // gemv1.hip

int gemv_mfma_dispatch(const float* x, const void* w, float* y, int M, int K, int N, int kind, int* rc);  // gemv_mfma.hip

int gemv_dispatch(const float* x, const void* w, float* y, int M, int K, int N, int kind) {
    {
        int rc;
        if (gemv_mfma_dispatch(x, w, y, M, K, N, kind, &rc)) return rc;
    }
    if (M == 1) {
        int rc;
        if (gemv1_dispatch(x, w, y, K, N, kind, &rc)) return rc;
    }
    size_t rowb;
    switch (kind) {
        case 0: rowb = row_bytes(0, K); return launch_gemv<0>(x, w, y, M, K, N, rowb);
        case 1: rowb = row_bytes(1, K); return launch_gemv<1>(x, w, y, M, K, N, rowb);
        case 2: rowb = row_bytes(2, K); return launch_gemv<2>(x, w, y, M, K, N, rowb);
        case 3: rowb = row_bytes(3, K); return launch_gemv<3>(x, w, y, M, K, N, rowb);
        case KF16: return launch_gemv<KF16>(x, w, y, M, K, N, (size_t)K * 2);
        case KF32: return launch_gemv<KF32>(x, w, y, M, K, N, (size_t)K * 4);
    }
    return fail(GH_EINVAL, "gemv: bad kind %d", kind);
}

int gemm_dispatch(const float* x, const void* w, float* y, int M, int K, int N, int kind, int accumulate);  // gemm.hip
int launch_add_to(float* y, const float* t, int64_t n);  // gemm.hip

static bool g_fused_q4 = true;
static const int kQuantSlots = 16;

// GEMV path constraint: K a multiple of the 64-value task
static int check_linear(const void* x, const void* w, const void* y, int M, int K, int N, int kind) {
    GH_REQUIRE(x && w && y, "linear_forward: null pointer");
    GH_REQUIRE(M >= 0 && N >= 0 && K > 0, "linear_forward: bad shape M=%d K=%d N=%d", M, K, N);
    GH_REQUIRE(K % 64 == 0 && (kind != 3 || K % 256 == 0),
               "linear_forward: K=%d must be a multiple of %d for kind %d", K, kind == 3 ? 256 : 64, kind);
    GH_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0, "linear_forward: x and W must be 16-byte aligned");
    return GH_OK;
}

int linear_any(const float* x, const void* w, float* y, int M, int K, int N, int kind) {
    int rc = check_linear(x, w, y, M, K, N, kind);
    if (rc) return rc;
    if (M == 0 || N == 0) return GH_OK;
    if (M <= 8) return gemv_dispatch(x, w, y, M, K, N, kind);
    return gemm_dispatch(x, w, y, M, K, N, kind, 0);
}

// y += x W^T (the residual add of a sublayer folded into its output projection)
int linear_acc(const float* x, const void* w, float* y, int M, int K, int N, int kind) {
    int rc = check_linear(x, w, y, M, K, N, kind);
    if (rc) return rc;
    if (M == 0 || N == 0) return GH_OK;
    if (M > 8) return gemm_dispatch(x, w, y, M, K, N, kind, 1);
    float* t = (float*)workspace(WS_GEMM_ACC, (size_t)M * N * 4);
    if (!t) return fail(GH_ENOMEM, "linear: workspace");
    rc = gemv_dispatch(x, w, t, M, K, N, kind);
    return rc ? rc : launch_add_to(y, t, (int64_t)M * N);
}

int dequant_launch(const void* packed, int kind, int64_t n, void* out, bool to_f16) {
    const int64_t threads = (n + 7) / 8;
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (to_f16) hipLaunchKernelGGL(k_dequant<true>, grid, dim3(256), 0, stream(), (const uint8_t*)packed, kind, n, out);
    else hipLaunchKernelGGL(k_dequant<false>, grid, dim3(256), 0, stream(), (const uint8_t*)packed, kind, n, out);
    GH_LAUNCHED("k_dequant");
    return GH_OK;
}

}  // namespace gh

using namespace gh;

extern "C" {

int gh_linear_forward_q4(const float* x, const void* w, float* y, int M, int K, int N, int kind) {
    GH_REQUIRE(valid_kind(kind), "linear_forward_q4: unknown kind %d", kind);
    return linear_any(x, w, y, M, K, N, kind);
}

int gh_linear_forward_fp16(const float* x, const uint16_t* w, float* y, int M, int K, int N) {
    return linear_any(x, w, y, M, K, N, KF16);
}

int gh_linear_forward_f32(const float* x, const float* w, float* y, int M, int K, int N) {
    return linear_any(x, w, y, M, K, N, KF32);
}

int gh_dequantize_f32(const void* packed, int kind, int64_t n, float* out) {
    GH_REQUIRE(valid_kind(kind) && packed && out && n >= 0, "dequantize: bad arguments");
    if (n == 0) return GH_OK;
    return dequant_launch(packed, kind, n, out, false);
}

int gh_quant_materialize(const void* packed, int kind, int64_t n, int slot, const uint16_t** out) {
    // core/ops.cpp:304-347
    GH_REQUIRE(packed != nullptr && n > 0 && out != nullptr, "quant_materialize: bad arguments");
    GH_REQUIRE(valid_kind(kind), "quant_materialize: unknown kind %d", kind);
    if (slot < 0 || slot >= kQuantSlots) slot = 0;
    void* dst = workspace(16 + slot, (size_t)n * 2);
    if (!dst) return fail(GH_ENOMEM, "quant_materialize: scratch allocation of %lld halves failed", (long long)n);
    int rc = dequant_launch(packed, kind, n, dst, true);
    if (rc) return rc;
    *out = (const uint16_t*)dst;
    return GH_OK;
}

int gh_quant_scratch_free(void) {
    free_workspaces();
    return GH_OK;
}

int gh_set_fused_q4(int on) {
    g_fused_q4 = on != 0;
    return GH_OK;
}
int gh_fused_q4_enabled(void) { return g_fused_q4 ? 1 : 0; }

}  // extern "C"
