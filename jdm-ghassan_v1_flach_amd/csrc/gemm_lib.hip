// Large-M prefill linear layers (M >= 1024 rows): the packed Q4_K / Q8_0 weights are decoded
// once per call into a bf16 copy (k_dequant_bf16, hand-written below), the activations are
// rounded to bf16 (k_to_bf16), and the product runs as a plain bf16 GEMM with fp32
// accumulation and fp32 output through hipBLASLt. At these sizes the decode costs a few
// per cent of the product (c2: 33 MB read, 117 MB written, against 240 GFLOP) and the library
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
    uint4 o;
    o.x = f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
    o.y = f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
    o.z = f32_to_bf16(v[4]) | ((uint32_t)f32_to_bf16(v[5]) << 16);
    o.w = f32_to_bf16(v[6]) | ((uint32_t)f32_to_bf16(v[7]) << 16);
    ((uint4*)out)[g] = o;
}

// fp32 -> bf16 (round to nearest even), 8 values per thread
__global__ void __launch_bounds__(256) k_to_bf16(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t n8) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
        const float4 a = ((const float4*)x)[2 * i], b = ((const float4*)x)[2 * i + 1];
        uint4 o;
        o.x = f32_to_bf16(a.x) | ((uint32_t)f32_to_bf16(a.y) << 16);
        o.y = f32_to_bf16(a.z) | ((uint32_t)f32_to_bf16(a.w) << 16);
        o.z = f32_to_bf16(b.x) | ((uint32_t)f32_to_bf16(b.y) << 16);
        o.w = f32_to_bf16(b.z) | ((uint32_t)f32_to_bf16(b.w) << 16);
        ((uint4*)y)[i] = o;
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
    if (kind == 3)
        hipLaunchKernelGGL(k_dequant_bf16<3>, dim3((unsigned)cdiv64(n8w, 256)), dim3(256), 0, stream(),
                           (const uint8_t*)w, w16, n8w, K, rowb);
    else
        hipLaunchKernelGGL(k_dequant_bf16<2>, dim3((unsigned)cdiv64(n8w, 256)), dim3(256), 0, stream(),
                           (const uint8_t*)w, w16, n8w, K, rowb);
    hipLaunchKernelGGL(k_to_bf16, dim3((unsigned)std::min<int64_t>(cdiv64(n8x, 256), 8192)), dim3(256), 0, stream(), x,
                       x16, n8x);
    GH_LAUNCHED("k_dequant_bf16 / k_to_bf16");
    const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
    LTC(hipblasLtMatmul(g_lt, plan->desc, &alpha, w16, plan->la, x16, plan->lb, &beta, y, plan->lc, y, plan->lc,
                        &plan->algo, ws, plan->ws, stream()));
    return GH_OK;
}

}  // namespace gh
