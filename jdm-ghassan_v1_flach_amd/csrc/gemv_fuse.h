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
    // start of a decode step folded into the first layer's norm prologue: the activation is the
    // fp16 embedding row of token bctl[0] (zero if out of range), block 0 also stores it to
    // emb_out and takes the step's cache slot (decode_alloc_slot). Nothing else in that launch
    // may read the slot: layer 0 must be a Mamba layer (its in_proj takes the fold).
    const uint16_t* emb = nullptr;
    float* emb_out = nullptr;
    int32_t* bctl = nullptr;
    int vocab = 0;
};

// The decode control block: [0] token, [1] cache length, [2] ring start, [3] pinned prefix,
// [4] capacity, [5] slot of the new token. A slot of the ring cache with a pinned prefix
// (inference/kv_cache.h:75-92): append while there is room, else overwrite the oldest
// unpinned position and advance the ring start. One thread.
__device__ inline void decode_alloc_slot(int32_t* ctl) {
    const int cap = ctl[4], pin = ctl[3];
    int len = ctl[1], start = ctl[2], slot;
    if (len < cap) {
        slot = len;
        if (len >= pin) slot = pin + ((start + (len - pin)) % (cap - pin));
        ++len;
    } else {
        slot = pin + (start % (cap - pin));
        start = (start + 1) % (cap - pin);
    }
    ctl[1] = len;
    ctl[2] = start;
    ctl[5] = slot;
}

// y = f(x) . W^T for ONE token, K-quant (kind 3) or Q8_0 (kind 2) weights,
// K a multiple of 256. Returns GH_EUNSUPPORTED if the shape is not handled.
int gemv_fused(const float* x, const void* w, float* y, int K, int N, int kind, const GmFuse& f);

}  // namespace gh
