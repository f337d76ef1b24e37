/* CPU oracle: a restatement of the reference engine's CPU forward path for
 * the quantized Granite-hybrid model. TEST INFRASTRUCTURE ONLY: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker. The product path (libghassan_hip.so) never links it.
 *
 * Every function cites the reference file:line it follows. Parity status of
 * each function is listed in the header comment of oracle.cpp. */
#pragma once
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- number formats (core/dtype.h:61-126) ---- */
void orc_f32_to_f16(const float* src, uint16_t* dst, int64_t n);
void orc_f16_to_f32(const uint16_t* src, float* dst, int64_t n);
void orc_f32_to_bf16(const float* src, uint16_t* dst, int64_t n);
void orc_bf16_to_f32(const uint16_t* src, float* dst, int64_t n);

/* ---- seeded inputs (core/rng.h:8-92) ---- */
void orc_rng_normal(uint64_t seed, float mean, float stddev, float* out, int64_t n);
void orc_rng_uniform(uint64_t seed, float lo, float hi, float* out, int64_t n);
void orc_rng_below(uint64_t seed, uint64_t bound, int32_t* out, int64_t n);
uint64_t orc_fnv1a64(const void* data, int64_t n);

/* ---- codecs: kind 0=Q4_0 1=Q4_1 2=Q8_0 3=Q4_K (core/quant.h:13-18 + new Q4_K) ---- */
int64_t orc_quant_row_bytes(int kind, int64_t k);
int  orc_quantize(int kind, const float* src, void* dst, int64_t n);
int  orc_dequantize(int kind, const void* src, float* dst, int64_t n);
int  orc_quant_materialize(int kind, const void* packed, uint16_t* dst, int64_t n);

/* ---- linear ops ---- */
int  orc_linear_forward_q4(const float* x, const void* w, float* y, int M, int K, int N, int kind);
void orc_linear_forward_fp16(const float* x, const uint16_t* w, float* y, int M, int K, int N);
void orc_linear_forward_f32(const float* x, const float* w, float* y, int M, int K, int N);
float orc_dot_f32(const float* a, const float* b, int n);

/* ---- elementwise ---- */
void orc_rmsnorm_forward(const float* x, const float* w, float* out, float* rrms,
                         int64_t rows, int dim, float eps);
void orc_swiglu_forward(const float* g, const float* u, float* out, int64_t n);
void orc_softmax_row(float* x, int n);
int32_t orc_argmax_token(const float* logits, int V);
int  orc_topk_select(const float* logits, int V, int K, float* out_vals, int32_t* out_ids);
void orc_apply_rep_penalties(float* logits, int V, const int32_t* hist, int hist_n, float rep, float freq,
                             float pres);
void orc_embedding_forward_half(const int32_t* ids, const uint16_t* table, float* out,
                                int64_t ntok, int dim, int vocab);

/* ---- attention ---- */
void orc_attention_forward_ex(const float* q, const float* k, const float* v, float* out,
                              int B, int T, int H, int KV, int hd, float scale, int window);
int  orc_attention_decode_ring_fp16(const float* q, const uint16_t* kc, const uint16_t* vc,
                                    float* out, int H, int KV, int hd, int ring_start,
                                    int pinned, int cur_len, int cache_max, float scale,
                                    int window);
/* Paged bf16 extension: per sequence, widen bf16 -> f32 and run the ring
 * kernel on the gathered logical sequence (exact widening). */
int  orc_attention_decode_paged_bf16(const float* q, const uint16_t* kpages,
                                     const uint16_t* vpages, const int32_t* page_table,
                                     const int32_t* seq_lens, int n_seqs, int max_pages,
                                     int page_size, float* out, int H, int KV, int hd,
                                     float scale);

/* ---- Mamba-2 ---- */
int  orc_mamba2_forward_q(const float* x, const void* w_in, const float* conv_w,
                          const float* conv_b, const float* dt_bias, const float* a_log,
                          const float* D, const float* norm_w, const void* w_out,
                          float* state, float* out, int B, int T, int d, int d_inner,
                          int conv_dim, int n_heads, int d_head, int d_state, int k,
                          float eps, int qkind);
/* the scan core only: (x,B,C,dt already formed) sequential recurrence */
void orc_ssd_scan_sequential(const float* xs, const float* Bm, const float* Cm,
                             const float* dt, const float* A, const float* D,
                             float* state, float* y, int T, int H, int P, int N);
int  orc_mamba2_step_q(const float* x, const void* w_in, const float* conv_w,
                       const float* conv_b, const float* dt_bias, const float* a_log,
                       const float* D, const float* norm_w, const void* w_out,
                       float* conv_state, float* ssm_state, float* out, int d,
                       int d_inner, int conv_dim, int n_heads, int d_head, int d_state,
                       int k, float eps, int qkind);

/* ---- MoE ---- */
int  orc_moe_route(const float* x, const float* router_w, const float* bias,
                   float* probs, int32_t* idx, float* w, int64_t N, int d, int ne, int K);
void orc_moe_permute(const int32_t* idx, int64_t N, int K, int ne, int32_t* grouped,
                     int32_t* offsets);
int  orc_moe_forward_q(const float* x, const float* router_w, const float* bias,
                       const void* gates, const void* ups, const void* downs,
                       const void* sh_g, const void* sh_u, const void* sh_d, float* out,
                       int32_t* idx_out, float* w_out, int64_t N, int d, int E, int ne,
                       int K, int SH, int qkind);

/* ---- synthetic Granite weights + the tiny-model generator ---- */
void orc_synth_param_f32(const char* name, uint64_t seed, float* out, int64_t n);
int  orc_granite_generate(const int32_t* cfg, const float* fcfg, const char** names,
                          const void** ptrs, int nparams, const int32_t* prompt, int P,
                          int n_new, int max_ctx, int32_t* out_ids, float* out_margins);
int  orc_granite_generate_timed(const int32_t* cfg, const float* fcfg, const char** names,
                                const void** ptrs, int nparams, const int32_t* prompt, int P,
                                int n_new, int max_ctx, int32_t* out_ids, float* out_margins,
                                double* seconds);
/* General form: optional Granite fields past cfg[16+L] / fcfg[2] (tie_embeddings, moe_aux_free;
 * embedding_multiplier, residual_multiplier, logits_scaling), teacher forcing (forced: the id fed
 * at each step, NULL = greedy) and the per-step logits (out_logits [n_new x V], may be NULL). */
int  orc_granite_generate_ex(const int32_t* cfg, int ncfg, const float* fcfg, int nfcfg, const char** names,
                             const void** ptrs, int nparams, const int32_t* prompt, int P, int n_new,
                             int max_ctx, const int32_t* forced, int32_t* out_ids, float* out_margins,
                             float* out_logits, double* seconds);

#ifdef __cplusplus
}
#endif
