// core/hip_ops.h — the reference-side C++ shim over the backend's C ABI
// (include/ghassan_hip.h), as a maintainer would add it to the reference
// engine: one inline wrapper per hot-path function of core/ops.h /
// core/device.h, with that function's argument list less the Device, turning
// a non-zero status into gai::Error (GAI_FAIL, core/common.h:29) with the
// backend's message. Compiled against the reference headers by
// tests/test_binding_cpu.py (syntax only: no reference code is linked).
#pragma once
#include <string>

#include "core/common.h"
#include "core/tensor.h"
#include "ghassan_hip.h"

namespace gai {
namespace hip_ops {

inline void check(int rc, const char* what) {
    if (rc != GH_OK) GAI_FAIL(std::string("hip ") + what + ": " + gh_last_error());
}

// core/device.h:40-46
inline void* device_alloc(size_t nbytes) {
    void* p = nullptr;
    check(gh_device_alloc(&p, nbytes), "device_alloc");
    return p;
}
inline void device_free(void* p) { check(gh_device_free(p), "device_free"); }
inline void device_memset_zero(void* p, size_t nbytes) { check(gh_device_memset_zero(p, nbytes), "device_memset_zero"); }
inline void device_copy(void* dst, Device dst_dev, const void* src, Device src_dev, size_t nbytes) {
    check(gh_device_copy(dst, (int)dst_dev, src, (int)src_dev, nbytes), "device_copy");
}

// core/ops.h:78-99
inline void linear_forward(const float* x, const float* w, float* y, int M, int K, int N) {
    check(gh_linear_forward_f32(x, w, y, M, K, N), "linear_forward");
}
inline void linear_forward_fp16(const float* x, const u16* w, float* y, int M, int K, int N) {
    check(gh_linear_forward_fp16(x, w, y, M, K, N), "linear_forward_fp16");
}
inline void convert_f32_to_f16(const float* src, u16* dst, i64 n) {
    check(gh_convert_f32_to_f16(src, dst, n), "convert_f32_to_f16");
}
inline void convert_f16_to_f32(const u16* src, float* dst, i64 n) {
    check(gh_convert_f16_to_f32(src, dst, n), "convert_f16_to_f32");
}
inline const u16* quant_materialize(const void* packed, int kind, i64 n, int slot) {
    const uint16_t* out = nullptr;
    check(gh_quant_materialize(packed, kind, n, slot, &out), "quant_materialize");
    return out;
}
inline void quant_scratch_free() { check(gh_quant_scratch_free(), "quant_scratch_free"); }
inline void set_fused_q4(bool on) { check(gh_set_fused_q4(on ? 1 : 0), "set_fused_q4"); }
inline bool fused_q4_enabled() { return gh_fused_q4_enabled() != 0; }
inline void linear_forward_q4(const float* x, const void* w, float* y, int M, int K, int N, int kind) {
    check(gh_linear_forward_q4(x, w, y, M, K, N, kind), "linear_forward_q4");
}

// core/ops.h:111-156
inline void embedding_forward_half(const i32* ids, const u16* table, float* out, i64 ntok, int dim, int vocab) {
    check(gh_embedding_forward_half(ids, table, out, ntok, dim, vocab), "embedding_forward_half");
}
inline void add(const float* a, const float* b, float* out, i64 n) { check(gh_add(a, b, out, n), "add"); }
inline void add_inplace(float* a, const float* b, i64 n) { check(gh_add_inplace(a, b, n), "add_inplace"); }
inline void scale_inplace(float* a, float s, i64 n) { check(gh_scale_inplace(a, s, n), "scale_inplace"); }
inline void zero(float* a, i64 n) { check(gh_zero(a, n), "zero"); }
inline void copy(float* dst, const float* src, i64 n) { check(gh_copy(dst, src, n), "copy"); }
inline void rmsnorm_forward(const float* x, const float* weight, float* out, float* rrms, i64 rows, int dim,
                            float eps) {
    check(gh_rmsnorm_forward(x, weight, out, rrms, rows, dim, eps), "rmsnorm_forward");
}
inline void swiglu_forward(const float* g, const float* u, float* out, i64 n) {
    check(gh_swiglu_forward(g, u, out, n), "swiglu_forward");
}

// core/ops.h:182-197: packed expert weights arrive as u16 byte streams (core/quant.h:53-64)
inline void moe_forward_bias_half(const float* x, const float* router_w, const float* router_bias, const u16* gates,
                                  const u16* ups, const u16* downs, const u16* sh_g, const u16* sh_u, const u16* sh_d,
                                  float* out, float* probs_cache, i32* idx_cache, float* w_cache, float* s_gate,
                                  float* s_up, float* s_act, i64 N, int d, int E, int ne, int K, int SH, int qkind) {
    check(gh_moe_forward_bias_half(x, router_w, router_bias, gates, ups, downs, sh_g, sh_u, sh_d, out, probs_cache,
                                   idx_cache, w_cache, s_gate, s_up, s_act, N, d, E, ne, K, SH, qkind),
          "moe_forward_bias_half");
}
inline void moe_forward_half(const float* x, const float* router_w, const u16* gates, const u16* ups,
                             const u16* downs, const u16* sh_g, const u16* sh_u, const u16* sh_d, float* out,
                             float* probs_cache, i32* idx_cache, float* w_cache, float* s_gate, float* s_up,
                             float* s_act, i64 N, int d, int E, int ne, int K, int SH, int qkind) {
    moe_forward_bias_half(x, router_w, nullptr, gates, ups, downs, sh_g, sh_u, sh_d, out, probs_cache, idx_cache,
                          w_cache, s_gate, s_up, s_act, N, d, E, ne, K, SH, qkind);
}

// core/ops.h:256-288
inline void mamba2_forward_half(const float* x, const u16* w_in, const float* conv_w, const float* conv_b,
                                const float* dt_bias, const float* a_log, const float* D, const float* norm_w,
                                const u16* w_out, float* state, float* out, int B, int T, int d, int d_inner,
                                int conv_dim, int n_heads, int d_head, int d_state, int k, float eps, int qkind) {
    check(gh_mamba2_forward_half(x, w_in, conv_w, conv_b, dt_bias, a_log, D, norm_w, w_out, state, out, B, T, d,
                                 d_inner, conv_dim, n_heads, d_head, d_state, k, eps, qkind),
          "mamba2_forward_half");
}
inline void mamba2_step_half(const float* x, const u16* w_in, const float* conv_w, const float* conv_b,
                             const float* dt_bias, const float* a_log, const float* D, const float* norm_w,
                             const u16* w_out, float* conv_state, float* ssm_state, float* out, int d, int d_inner,
                             int conv_dim, int n_heads, int d_head, int d_state, int k, float eps, int qkind) {
    check(gh_mamba2_step_half(x, w_in, conv_w, conv_b, dt_bias, a_log, D, norm_w, w_out, conv_state, ssm_state, out,
                              d, d_inner, conv_dim, n_heads, d_head, d_state, k, eps, qkind),
          "mamba2_step_half");
}

// core/ops.h:343-367
inline void attention_forward_ex(const float* q, const float* k, const float* v, float* out, float* probs, int B,
                                 int T, int H, int KV, int hd, float scale, int window, const i32* segment_ids) {
    check(gh_attention_forward_ex(q, k, v, out, probs, B, T, H, KV, hd, scale, window, segment_ids),
          "attention_forward_ex");
}
inline void attention_decode_ring_fp16(const float* q, const u16* kcache, const u16* vcache, float* out, int H,
                                       int KV, int hd, int ring_start, int pinned_prefix, int cur_len, int cache_max,
                                       float scale, float* scratch, int window) {
    check(gh_attention_decode_ring_fp16(q, kcache, vcache, out, H, KV, hd, ring_start, pinned_prefix, cur_len,
                                        cache_max, scale, scratch, window),
          "attention_decode_ring_fp16");
}

// core/ops.h:397-404
inline void topk_select(const float* logits, int V, int K, float* out_vals, i32* out_ids) {
    check(gh_topk_select(logits, V, K, out_vals, out_ids), "topk_select");
}
inline i32 argmax_token(const float* logits, int V) {
    int32_t id = 0;
    check(gh_argmax_token(logits, V, &id), "argmax_token");
    return id;
}
inline void apply_rep_penalties(float* logits, int V, const i32* hist, int hist_n, float rep, float freq,
                                float pres) {
    check(gh_apply_rep_penalties(logits, V, hist, hist_n, rep, freq, pres), "apply_rep_penalties");
}

}  // namespace hip_ops
}  // namespace gai
