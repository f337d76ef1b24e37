// Large-M prefill linear layers (M >= 1024 rows): the packed Q4_K / Q8_0 weights are decoded
// once per call into a bf16 copy (k_dequant_fused, hand-written below; k_dequant_bf16 for
// unaligned weights), the activations rounded to bf16 in the same launch, and the product
// runs as a plain bf16 GEMM with fp32 accumulation and fp32 output through hipBLASLt. At
// these sizes the decode costs a few per cent of the product (c2: 33 MB read, 117 MB written, against 240 GFLOP) and the library
// GEMM reaches about half of the bf16 MFMA peak, which the fused decode-in-LDS kernel
// (gemm.hip) does not; smaller M keep the fused kernels, where the extra pass would dominate.
// bf16 operands (not fp16): no range handling is needed for any activation, as the
// reference's fp32 inputs allow; the decoded weight is rounded once (RNE), like the
// reference's fp16 quant_materialize but to bf16 (core/ops.cpp:304-338).
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <tuple>

#include "gemm_tile.h"

namespace gh {

// fp32 -> bf16 pairs by the hardware conversion (v_cvt_pk_bf16_f32: round to nearest even,
// the result of f32_to_bf16 for every finite value)
typedef float lt_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 lt_bf2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((lt_f2){a, b}, lt_bf2));
}
__device__ __forceinline__ uint4 bf16x8(const float4 a, const float4 b) {
    return make_uint4(bf16x2(a.x, a.y), bf16x2(a.z, a.w), bf16x2(b.x, b.y), bf16x2(b.z, b.w));
}

// Row-major [N][K] packed rows (K a multiple of 256 for Q4_K, 32 for Q8_0) -> bf16 [N][K].
// One thread per 8 consecutive values of one sub-block: the block header once, one 8-byte
// code load, one 16-byte store. The value is the reference decode (d sc) q - dmin m / q d
// in fp32 without fused multiply-add, then rounded to bf16.
template <int KIND>
__global__ void __launch_bounds__(256) k_dequant_bf16(const uint8_t* __restrict__ W, uint16_t* __restrict__ out,
                                                      int64_t n8, int K, size_t rowb) {
#pragma clang fp contract(off)
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= n8) return;
    const int k8 = K / 8;
    const int64_t row = g / k8;
    const int c8 = (int)(g - row * k8);  // 8-value group within the row
    const uint8_t* rp = W + (size_t)row * rowb;
    float v[8];
    if constexpr (KIND == 3) {
        const uint8_t* blk = rp + (size_t)(c8 >> 5) * 144;
        const int j0 = (c8 & 31) * 8, s = j0 >> 5, l0 = j0 & 31;
        const uint32_t hd = *(const uint32_t*)blk;
        const float d = f16_to_f32((uint16_t)hd), dmin = f16_to_f32((uint16_t)(hd >> 16));
        const uint8_t* sc = blk + 4;
        int scv, mv;
        if (s < 4) {
            scv = sc[s] & 63;
            mv = sc[s + 4] & 63;
        } else {
            scv = (sc[s + 4] & 0xF) | ((sc[s - 4] >> 6) << 4);
            mv = (sc[s + 4] >> 4) | ((sc[s] >> 6) << 4);
        }
        const float d1 = d * (float)scv, m1 = dmin * (float)mv;
        const uint2 q8 = *(const uint2*)(blk + 16 + 32 * (s >> 1) + l0);
        const uint32_t qs[2] = {q8.x, q8.y};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t b = (qs[i >> 2] >> (8 * (i & 3))) & 0xFF;
            const int q = (s & 1) ? (int)(b >> 4) : (int)(b & 0xF);
            v[i] = d1 * (float)q - m1;
        }
    } else {  // Q8_0
        const uint8_t* blk = rp + (size_t)(c8 >> 2) * 34;
        const float d = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        const int j0 = (c8 & 3) * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (float)(int8_t)blk[2 + j0 + i] * d;
    }
    ((uint4*)out)[g] = make_uint4(bf16x2(v[0], v[1]), bf16x2(v[2], v[3]), bf16x2(v[4], v[5]), bf16x2(v[6], v[7]));
}


// Packed rows -> bf16 with the activations' conversion in the same launch. Blocks below
// `wblocks` decode weights, one thread per item of 64 consecutive values of a row:
//  - Q4_K (KIND 3): a super-block's sub-block pair p: the 16-byte header (d, dmin, 12 scale
//    bytes) and the pair's 32 code bytes in three 16-byte loads (low nibbles: sub-block 2p,
//    high: 2p + 1); value (d sc) q - dmin m (the k_dequant_bf16<3> arithmetic);
//  - Q8_0 (KIND 2): two 34-byte blocks as 17 dwords (rows of K % 256 == 0 are 4-byte
//    aligned), codes realigned with alignbyte; value q d.
// fp32 without fused multiply-add, rounded to bf16. A wave's 64 items are 64 consecutive
// 128-byte runs of the output (rows are contiguous): the lanes leave their 8 pieces in LDS
// (XOR-swizzled against bank conflicts) and the wave stores its 8 KB as eight 1 KB-contiguous
// instructions (a lane writing its own 128 bytes ran at 3.2 TB/s). The other blocks convert x.
template <int KIND>
__device__ __forceinline__ void dq_item(const uint8_t* __restrict__ W, uint32_t i, uint32_t ipr, size_t rowb,
                                        uint4* piece, int lane) {
#pragma clang fp contract(off)
    const uint32_t row = i / ipr, r = i - row * ipr;
    if constexpr (KIND == 3) {
        const int sb = (int)(r >> 2), pr = (int)(r & 3);
        const uint8_t* blk = W + (size_t)row * rowb + (size_t)sb * 144;
        const uint4 h = *(const uint4*)blk;
        const uint4 c0 = *(const uint4*)(blk + 16 + 32 * pr), c1 = *(const uint4*)(blk + 32 + 32 * pr);
        const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
        auto sbyte = [&](int j) -> int { return (int)((hw[(4 + j) >> 2] >> (8 * ((4 + j) & 3))) & 0xFF); };
        const float d = f16_to_f32((uint16_t)h.x), dmin = f16_to_f32((uint16_t)(h.x >> 16));
        float d1[2], m1[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int s = 2 * pr + k;
            int scv, mv;
            if (s < 4) {
                scv = sbyte(s) & 63;
                mv = sbyte(s + 4) & 63;
            } else {
                scv = (sbyte(s + 4) & 0xF) | ((sbyte(s - 4) >> 6) << 4);
                mv = (sbyte(s + 4) >> 4) | ((sbyte(s) >> 6) << 4);
            }
            d1[k] = d * (float)scv;
            m1[k] = dmin * (float)mv;
        }
        const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
            for (int q8 = 0; q8 < 4; ++q8) {  // values 8 q8 .. 8 q8 + 7 of sub-block 2 pr + k: piece 4k + q8
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int l = 8 * q8 + e;
                    const uint32_t b = (cw[l >> 2] >> (8 * (l & 3))) & 0xFF;
                    const int q = k ? (int)(b >> 4) : (int)(b & 0xF);
                    v[e] = d1[k] * (float)q - m1[k];
                }
                piece[(4 * k + q8) ^ (lane & 7)] =
                    bf16x8(make_float4(v[0], v[1], v[2], v[3]), make_float4(v[4], v[5], v[6], v[7]));
            }
    } else {
        const uint32_t* bp = (const uint32_t*)(W + (size_t)row * rowb + (size_t)r * 68);
        uint32_t w[17];
#pragma unroll
        for (int k = 0; k < 17; ++k) w[k] = bp[k];
        // block 0: d in bytes 0-1, codes 2-33; block 1: d in 34-35, codes 36-67
        uint32_t c[16];
#pragma unroll
        for (int k = 0; k < 8; ++k) c[k] = __builtin_amdgcn_alignbyte(w[k + 1], w[k], 2);
#pragma unroll
        for (int k = 0; k < 8; ++k) c[8 + k] = w[9 + k];
        const float d0 = f16_to_f32((uint16_t)(w[0] & 0xFFFF)), d1 = f16_to_f32((uint16_t)(w[8] >> 16));
#pragma unroll
        for (int p = 0; p < 8; ++p) {  // piece p: values 8p .. 8p + 7 (block p / 4)
            const float d = p < 4 ? d0 : d1;
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t dw = c[2 * p + (e >> 2)];
                v[e] = (float)(int8_t)((dw >> (8 * (e & 3))) & 0xFF) * d;
            }
            piece[p ^ (lane & 7)] = bf16x8(make_float4(v[0], v[1], v[2], v[3]), make_float4(v[4], v[5], v[6], v[7]));
        }
    }
}

template <int KIND>
__global__ void __launch_bounds__(256) k_dequant_fused(const uint8_t* __restrict__ W, uint16_t* __restrict__ out,
                                                       uint32_t nitems, uint32_t items_per_row, size_t rowb,
                                                       uint32_t wblocks, const float* __restrict__ x,
                                                       uint16_t* __restrict__ x16, int64_t n8x) {
    if (blockIdx.x >= wblocks) {  // activations: 4 groups of 8 per thread, all loads first
        const int64_t i0 = (int64_t)(blockIdx.x - wblocks) * 1024 + threadIdx.x;
        float4 a[4], b[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t i = i0 + 256 * u;
            if (i < n8x) {
                a[u] = ((const float4*)x)[2 * i];
                b[u] = ((const float4*)x)[2 * i + 1];
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (i0 + 256 * u < n8x) ((uint4*)x16)[i0 + 256 * u] = bf16x8(a[u], b[u]);
        return;
    }
    __shared__ uint4 stg[4][512];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    const uint32_t i0 = blockIdx.x * 256u + 64u * wave;  // the wave's first item
    if (i0 >= nitems) return;                            // whole wave past the end
    if (i < nitems) dq_item<KIND>(W, i, items_per_row, rowb, &stg[wave][8 * lane], lane);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    uint4* o = (uint4*)out + (size_t)8 * i0;  // item i starts at value 64 i
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int e = 64 * j + lane, t = e >> 3;  // piece e of the wave: item t, piece e & 7
        if (i0 + (uint32_t)t < nitems) o[e] = stg[wave][8 * t + ((e & 7) ^ (t & 7))];
    }
}

// fp32 -> bf16 (round to nearest even), 8 values per thread
__global__ void __launch_bounds__(256) k_to_bf16(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t n8) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
        ((uint4*)y)[i] = bf16x8(((const float4*)x)[2 * i], ((const float4*)x)[2 * i + 1]);
    }
}

namespace {
struct LtPlan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t ws = 0;
};
hipblasLtHandle_t g_lt = nullptr;
int g_lt_dev = -1;
std::map<std::tuple<int, int, int>, LtPlan> g_plans;
constexpr size_t LT_WS = (size_t)64 << 20;

#define LTC(call)                                                                              \
    do {                                                                                       \
        const hipblasStatus_t st_ = (call);                                                    \
        if (st_ != HIPBLAS_STATUS_SUCCESS) return fail(GH_EHIP, "hipBLASLt: %s -> %d", #call, (int)st_); \
    } while (0)

// y [M][N] row-major (fp32) = x16 [M][K] . w16 [N][K]^T, as the column-major product
// D (N x M) = op_T(A = w16, K x N) . B (= x16, K x M); beta selects y += (1) or y = (0).
int lt_plan(int M, int N, int K, LtPlan** out) {
    int dev = 0;
    GH_HIP(hipGetDevice(&dev));
    if (!g_lt || g_lt_dev != dev) {
        if (g_lt) {
            for (auto& kv : g_plans) {
                hipblasLtMatrixLayoutDestroy(kv.second.la);
                hipblasLtMatrixLayoutDestroy(kv.second.lb);
                hipblasLtMatrixLayoutDestroy(kv.second.lc);
                hipblasLtMatmulDescDestroy(kv.second.desc);
            }
            g_plans.clear();
            hipblasLtDestroy(g_lt);
            g_lt = nullptr;
        }
        LTC(hipblasLtCreate(&g_lt));
        g_lt_dev = dev;
    }
    auto key = std::make_tuple(M, N, K);
    auto it = g_plans.find(key);
    if (it != g_plans.end()) {
        *out = &it->second;
        return GH_OK;
    }
    LtPlan p;
    LTC(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    LTC(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta));
    LTC(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb));
    LTC(hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, K, N, K));
    LTC(hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, K, M, K));
    LTC(hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, N, M, N));
    hipblasLtMatmulPreference_t pref = nullptr;
    LTC(hipblasLtMatmulPreferenceCreate(&pref));
    const uint64_t wsmax = LT_WS;
    LTC(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsmax, sizeof wsmax));
    hipblasLtMatmulHeuristicResult_t res[1];
    int nres = 0;
    const hipblasStatus_t st =
        hipblasLtMatmulAlgoGetHeuristic(g_lt, p.desc, p.la, p.lb, p.lc, p.lc, pref, 1, res, &nres);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || nres < 1) {
        hipblasLtMatrixLayoutDestroy(p.la);
        hipblasLtMatrixLayoutDestroy(p.lb);
        hipblasLtMatrixLayoutDestroy(p.lc);
        hipblasLtMatmulDescDestroy(p.desc);
        return GH_EUNSUPPORTED;
    }
    p.algo = res[0].algo;
    p.ws = res[0].workspaceSize;
    *out = &(g_plans[key] = p);
    return GH_OK;
}
}  // namespace

// Returns GH_EUNSUPPORTED (nothing launched) when the shape or kind is not taken here.
int gemm_lib(const float* x, const void* w, float* y, int M, int K, int N, int kind, int accumulate) {
    if ((kind != 2 && kind != 3) || M < 1024 || N < 256 || K % 256 != 0 || N % 8 != 0) return GH_EUNSUPPORTED;
    if (((uintptr_t)x | (uintptr_t)y) & 15) return GH_EUNSUPPORTED;
    LtPlan* plan = nullptr;
    const int rc = lt_plan(M, N, K, &plan);
    if (rc) return rc;
    const size_t xb = ((size_t)M * K * 2 + 255) & ~(size_t)255, wb = (size_t)N * K * 2;
    uint16_t* x16 = (uint16_t*)workspace(WS_GEMM_X, xb);
    uint16_t* w16 = (uint16_t*)workspace(WS_GEMM_W16, wb);
    void* ws = plan->ws ? workspace(WS_BLASLT, plan->ws) : nullptr;
    if (!x16 || !w16 || (plan->ws && !ws)) return fail(GH_ENOMEM, "gemm: workspace");
    const int64_t n8w = (int64_t)N * K / 8, n8x = (int64_t)M * K / 8;
    const size_t rowb = row_bytes(kind, K);
    // rows of K % 256 == 0 values stay 16-byte (Q4_K) / 4-byte (Q8_0) aligned from an aligned base
    const bool fused_ok = ((uintptr_t)w & (kind == 3 ? 15 : 3)) == 0 && (int64_t)N * (K / 64) < ((int64_t)1 << 31);
    if (fused_ok) {
        const uint32_t ipr = (uint32_t)(K / 64), nitems = (uint32_t)N * ipr;
        const uint32_t wblocks = (nitems + 255) / 256, xblocks = (uint32_t)cdiv64(n8x, 1024);
        if (kind == 3)
            hipLaunchKernelGGL(k_dequant_fused<3>, dim3(wblocks + xblocks), dim3(256), 0, stream(), (const uint8_t*)w,
                               w16, nitems, ipr, rowb, wblocks, x, x16, n8x);
        else
            hipLaunchKernelGGL(k_dequant_fused<2>, dim3(wblocks + xblocks), dim3(256), 0, stream(), (const uint8_t*)w,
                               w16, nitems, ipr, rowb, wblocks, x, x16, n8x);
        GH_LAUNCHED("k_dequant_fused");
    } else {
        if (kind == 3)
            hipLaunchKernelGGL(k_dequant_bf16<3>, dim3((unsigned)cdiv64(n8w, 256)), dim3(256), 0, stream(),
                               (const uint8_t*)w, w16, n8w, K, rowb);
        else
            hipLaunchKernelGGL(k_dequant_bf16<2>, dim3((unsigned)cdiv64(n8w, 256)), dim3(256), 0, stream(),
                               (const uint8_t*)w, w16, n8w, K, rowb);
        hipLaunchKernelGGL(k_to_bf16, dim3((unsigned)std::min<int64_t>(cdiv64(n8x, 256), 8192)), dim3(256), 0,
                           stream(), x, x16, n8x);
        GH_LAUNCHED("k_dequant_bf16 / k_to_bf16");
    }
    const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
    LTC(hipblasLtMatmul(g_lt, plan->desc, &alpha, w16, plan->la, x16, plan->lb, &beta, y, plan->lc, y, plan->lc,
                        &plan->algo, ws, plan->ws, stream()));
    return GH_OK;
}

}  // namespace gh
