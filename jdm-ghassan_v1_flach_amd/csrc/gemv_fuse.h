// Fusion hooks of the single-token GEMV (decode): how the activation vector
// is formed before the product (prologue) and where each output goes
// (epilogue). They let one decode sub-layer run as one launch instead of
// norm + GEMV(s) + scatter + residual add.
#pragma once
#include "gh_common.h"

namespace gh {

enum GmPro {
    GM_PRO_NONE = 0,
    GM_PRO_RMSNORM = 1,  // x * rrms(x) * w       (core/ops.h:134 rmsnorm_forward)
    GM_PRO_GATED = 2,    // rmsnorm(y * silu(z)) * w (Mamba-2 gated norm)
    GM_PRO_ATTN = 3,     // merge of the split-K attention partials, all heads
};
enum GmEpi {
    GM_EPI_STORE = 0,    // y[n] = v
    GM_EPI_ADD = 1,      // y[n] += v                      (residual)
    GM_EPI_QKV = 2,      // rows [0,n0): y; then K and V rows as fp16 into the cache slot
    GM_EPI_CONV = 3,     // rows [c0, c0+cdim): causal conv step + SiLU (window shift); others stored
};

struct GmFuse {
    int pro = GM_PRO_NONE;
    const float* pw = nullptr;      // norm weight [K]
    const float* pz = nullptr;      // gated norm: z [K]
    float eps = 0.f;
    const float* o_part = nullptr;  // attention partials [KV][splits][G][hd]
    const float* ml = nullptr;      // [KV][splits][G][2] (running max, sum)
    int H = 0, KV = 0, G = 0, splits = 0, hd = 0;
    // weight segments: output rows [0,n0) from W, [n0,n0+n1) from w1, the rest from w2
    const void* w1 = nullptr;
    const void* w2 = nullptr;
    int n0 = 0, n1 = 0;
    int epi = GM_EPI_STORE;
    uint16_t* kc = nullptr;         // QKV: caches [cap][kvd] fp16, slot index at *slot
    uint16_t* vc = nullptr;
    const int32_t* slot = nullptr;
    int kvd = 0;
    const float* conv_w = nullptr;  // CONV: [cdim][ck], bias [cdim], window [cdim][ck-1]
    const float* conv_b = nullptr;
    float* conv_win = nullptr;
    int c0 = 0, cdim = 0, ck = 0;
};

// y = f(x) . W^T for ONE token, K-quant (kind 3) or Q8_0 (kind 2) weights,
// K a multiple of 256. Returns GH_EUNSUPPORTED if the shape is not handled.
int gemv_fused(const float* x, const void* w, float* y, int K, int N, int kind, const GmFuse& f);

}  // namespace gh
