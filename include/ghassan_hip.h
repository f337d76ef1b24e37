/* ghassan_hip.h — C ABI of the MI355X (gfx950) backend for the quantized
 * Granite-hybrid forward path.
 *
 * Each entry point replaces one function of the reference engine's dispatch
 * surface, core/ops.h (namespace gai::ops) and core/device.h, on the
 * Device::CUDA branch of GAI_DISPATCH (core/ops.cpp:28-40). The cited
 * file:line is the reference declaration it stands in for. Conventions
 * (core/ops.h, core/ops.cpp):
 *   - every pointer is a raw, caller-owned, row-major DEVICE pointer unless
 *     the comment says "host";
 *   - weights are W[N_out, K] with y = x W^T (core/math_cpu.cpp:117-119);
 *     packed weights are GGML blocks, `kind` 0=Q4_0 1=Q4_1 2=Q8_0 (as in
 *     core/quant.h:13-18) and 3=Q4_K (new: the reference has no K-quants);
 *   - the return value is a status (GH_OK = 0); the message of the last
 *     failure on the calling host thread is gh_last_error(). The reference
 *     throws gai::Error (core/common.h:22-31); its C++ shim rethrows on != 0;
 *   - work is enqueued on the backend stream (gh_set_stream; default: the
 *     null stream), in order, like the reference's stream-0 ordering.
 *     Calls are single-host-thread and not re-entrant (core/ops.h:52-55).
 */
#ifndef GHASSAN_HIP_H
#define GHASSAN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { GH_OK = 0, GH_EINVAL = 1, GH_EHIP = 2, GH_ENOMEM = 3, GH_EUNSUPPORTED = 4 };
/* Device numbering of core/tensor.h:11 (the HIP GPU takes CUDA's slot). */
enum { GH_DEV_CPU = 0, GH_DEV_GPU = 1 };
/* Packed weight kinds. */
enum { GH_Q4_0 = 0, GH_Q4_1 = 1, GH_Q8_0 = 2, GH_Q4_K = 3 };

typedef struct {
    char name[256];
    int arch_major, arch_minor; /* gfx9.5 for MI355X */
    int compute_units;
    size_t total_mem, free_mem;
} gh_device_info_t;

/* ---------------------------------------------------------------- runtime */
const char* gh_last_error(void);
/* core/device.h:26 device_info(). Selects `device` and initialises the backend. */
int gh_init(int device);
int gh_device_info(gh_device_info_t* out);
/* core/device.h:40-46 (core/device.cpp:253-333) */
int gh_device_alloc(void** out, size_t bytes);
int gh_device_free(void* p);
int gh_device_memset_zero(void* p, size_t bytes);
/* Synchronous copy like device_copy (core/device.cpp:315-333); dst_dev /
 * src_dev are GH_DEV_CPU or GH_DEV_GPU. */
int gh_device_copy(void* dst, int dst_dev, const void* src, int src_dev, size_t bytes);
/* Stream / event helpers (cuda/cuda_utils.cu:200-265 phase timers). */
int gh_set_stream(void* hip_stream);
void* gh_get_stream(void);
int gh_synchronize(void);
int gh_event_create(void** ev);
int gh_event_record(void* ev);
int gh_event_elapsed_ms(void* start, void* stop, float* ms);
int gh_event_destroy(void* ev);
/* Frees the backend's grow-only workspaces (cuda/kernels.cu:31-70). */
int gh_free_workspace(void);

/* ------------------------------------------------------- quantized linear */
/* core/ops.h:98-99 linear_forward_q4: y[M,N] = x[M,K] dequant(W)^T.
 * K must be a multiple of the block size (32, or 256 for Q4_K). M <= 8 runs
 * the decode GEMV; larger M the dequant-to-LDS bf16 MFMA GEMM. */
int gh_linear_forward_q4(const float* x, const void* w, float* y, int M, int K, int N, int kind);
/* core/ops.h:81 linear_forward_fp16: fp16 weights (lm_head / tied embedding). */
int gh_linear_forward_fp16(const float* x, const uint16_t* w, float* y, int M, int K, int N);
/* core/ops.h:78 linear_forward: fp32 weights (the router logits). */
int gh_linear_forward_f32(const float* x, const float* w, float* y, int M, int K, int N);
/* core/ops.h:91 quant_materialize: packed -> fp16 scratch slot (0..15);
 * *out stays valid until the next call on the same slot. */
int gh_quant_materialize(const void* packed, int kind, int64_t n, int slot, const uint16_t** out);
/* core/ops.h:92 quant_scratch_free */
int gh_quant_scratch_free(void);
/* Dequantise to fp32 (quantization/quantize.cpp:114-133 dequantize_* on the
 * device; used to check bit-exactness of the decode). */
int gh_dequantize_f32(const void* packed, int kind, int64_t n, float* out);
/* core/ops.h:96-97 */
int gh_set_fused_q4(int on);
int gh_fused_q4_enabled(void);

/* ------------------------------------------------------------ elementwise */
int gh_convert_f32_to_f16(const float* src, uint16_t* dst, int64_t n);   /* core/ops.h:82 */
int gh_convert_f16_to_f32(const uint16_t* src, float* dst, int64_t n);   /* core/ops.h:83 */
int gh_embedding_forward_half(const int32_t* ids, const uint16_t* table, float* out, int64_t ntok,
                              int dim, int vocab);                      /* core/ops.h:111 */
int gh_add(const float* a, const float* b, float* out, int64_t n);     /* core/ops.h:121 */
int gh_add_inplace(float* a, const float* b, int64_t n);               /* core/ops.h:122 */
int gh_scale_inplace(float* a, float s, int64_t n);                    /* core/ops.h:125 */
int gh_zero(float* a, int64_t n);                                      /* core/ops.h:126 */
int gh_copy(float* dst, const float* src, int64_t n);                  /* core/ops.h:127 */
/* Measurement helper, no counterpart in the reference: reads `bytes` (a multiple of 16) once with
 * 16-byte loads from `blocks` blocks of 256 lanes and writes one XOR word per block to sink[blocks].
 * Its time is the HBM read ceiling the weight-streaming kernels are compared with. */
int gh_stream_read(const void* src, int64_t bytes, uint32_t* sink, int blocks);
/* core/ops.h:134 rmsnorm_forward (rrms may be NULL) */
int gh_rmsnorm_forward(const float* x, const float* w, float* out, float* rrms, int64_t rows, int dim,
                       float eps);
int gh_swiglu_forward(const float* g, const float* u, float* out, int64_t n); /* core/ops.h:156 */
/* core/ops.h:400 argmax_token: writes the id to *out_host (host int). */
int gh_argmax_token(const float* logits, int V, int32_t* out_host);
/* Device-resident variant for graph-captured decode: writes the id to a
 * device int. No reference counterpart (the reference copies it back). */
int gh_argmax_token_dev(const float* logits, int V, int32_t* out_dev);
/* core/ops.h:397 topk_select (device logits / outputs): the K largest logits, larger value first,
 * lower index first among equal values (core/math_cpu.cpp:695-707); NaN ranks below -inf.
 * Limits of the CUDA branch (cuda/kernels.cu:1474-1476): 1 <= K <= 128, K <= V <= 262144. */
int gh_topk_select(const float* logits, int V, int K, float* out_vals, int32_t* out_ids);
/* core/ops.h:402 apply_rep_penalties: logits on the device, hist a HOST array of hist_n ids
 * (as Generator passes its history, inference/generator.cpp:1042); semantics of
 * core/math_cpu.cpp:725-752. */
int gh_apply_rep_penalties(float* logits, int V, const int32_t* hist, int hist_n, float rep, float freq,
                           float pres);
/* The tail of a decode step in one launch: final rmsnorm (core/ops.h:134) of x[d],
 * the tied fp16 lm head (model/model.cpp:1087-1160, logits[V] written) and
 * argmax_token (core/ops.h:400) into a device int. d % 8 == 0, d <= 2048. */
int gh_lm_head_greedy_dev(const float* x, const float* norm_w, float eps, const uint16_t* tab_f16, float* logits,
                          int d, int V, int32_t* out_dev);

/* ----------------------------------------------------------------- Mamba-2 */
/* core/ops.h:256-269 mamba2_forward_half: one Mamba-2 layer over B x T
 * tokens; `state` [B, H, P, N] is carried in and out; the conv window starts
 * at zero (core/mamba_cpu.cpp:99). qkind -1: fp16 projections, else packed.
 * The scan is the chunked SSD (chunk 256, MFMA intra-chunk). */
int gh_mamba2_forward_half(const float* x, const void* w_in, const float* conv_w, const float* conv_b,
                           const float* dt_bias, const float* a_log, const float* D, const float* norm_w,
                           const void* w_out, float* state, float* out, int B, int T, int d, int d_inner,
                           int conv_dim, int n_heads, int d_head, int d_state, int k, float eps,
                           int qkind);
/* core/ops.h:281-288 mamba2_step_half: one decode token. conv_state
 * [conv_dim, k-1] and ssm_state [H, P, N] are carried on the device. */
int gh_mamba2_step_half(const float* x, const void* w_in, const float* conv_w, const float* conv_b,
                        const float* dt_bias, const float* a_log, const float* D, const float* norm_w,
                        const void* w_out, float* conv_state, float* ssm_state, float* out, int d,
                        int d_inner, int conv_dim, int n_heads, int d_head, int d_state, int k, float eps,
                        int qkind);
/* The scan core alone (x/B/C/dt formed, dt already softplus'ed, A = -exp(A_log)):
 * xs [T, H*P], Bm/Cm [T, N], dt [T, H], y [T, H*P]; state [H,P,N] in/out.
 * Component of mamba2_forward (core/mamba_cpu.cpp:120-170). */
int gh_ssd_scan(const float* xs, const float* Bm, const float* Cm, const float* dt, const float* A,
                const float* D, float* state, float* y, int T, int H, int P, int N, int chunk);

/* --------------------------------------------------------------- attention */
/* core/ops.h:343-347 attention_forward_ex (B, T causal; probs must be NULL,
 * segment_ids must be NULL: the inference path passes neither). */
int gh_attention_forward_ex(const float* q, const float* k, const float* v, float* out, float* probs, int B,
                            int T, int H, int KV, int hd, float scale, int window, const int32_t* segment_ids);
/* core/ops.h:363-367 attention_decode_ring_fp16. `scratch` may be NULL (the
 * backend keeps its own split-K partials). */
int gh_attention_decode_ring_fp16(const float* q, const uint16_t* kcache, const uint16_t* vcache, float* out,
                                  int H, int KV, int hd, int ring_start, int pinned_prefix, int cur_len,
                                  int cache_max, float scale, float* scratch, int window);
/* No counterpart in the reference. attention_decode_ring_fp16 for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops): the same kernels
 * and result, with the split-K partials in a static 4 MiB device array per GPU instead of the
 * backend's grow-only workspace; it calls no hipMalloc / hipFree. Returns GH_EINVAL when the
 * partials (H * splits * (hd + 2) floats, splits ~ cur_len / chunk) would exceed 4 MiB.
 * Calls that overlap on one GPU (several streams or host threads) race on that array. */
int gh_attention_decode_ring_fp16_noalloc(const float* q, const uint16_t* kcache, const uint16_t* vcache,
                                          float* out, int H, int KV, int hd, int ring_start, int pinned_prefix,
                                          int cur_len, int cache_max, float scale, int window);
/* Extension (no reference counterpart; benchmark configuration c4): ragged batched
 * decode over a paged bf16 KV cache. q [S, H, hd]; pages [n_pages, page_size,
 * KV, hd] bf16; page_table [S, max_pages] (device int32); seq_lens [S]
 * (device int32); out [S, H, hd]. */
int gh_attention_decode_paged_bf16(const float* q, const uint16_t* kpages, const uint16_t* vpages,
                                   const int32_t* page_table, const int32_t* seq_lens, int n_seqs,
                                   int max_pages, int page_size, int max_len, float* out, int H, int KV,
                                   int hd, float scale);

/* --------------------------------------------------------------------- MoE */
/* core/ops.h:191-197 moe_forward_bias_half (router_bias may be NULL, which
 * is core/ops.h:182 moe_forward_half). qkind -1: fp16 experts, else packed.
 * probs/idx/w caches may be NULL; s_gate/s_up/s_act are ignored (the
 * backend keeps its own grouped scratch). */
int gh_moe_forward_bias_half(const float* x, const float* router_w, const float* router_bias,
                             const void* gates, const void* ups, const void* downs, const void* sh_g,
                             const void* sh_u, const void* sh_d, float* out, float* probs_cache,
                             int32_t* idx_cache, float* w_cache, float* s_gate, float* s_up, float* s_act,
                             int64_t N, int d, int E, int ne, int K, int SH, int qkind);
/* Router top-k alone (core/moe_cpu.cpp:218-256): probs [N,ne], idx [N,K], w [N,K]. */
int gh_moe_route(const float* x, const float* router_w, const float* router_bias, float* probs,
                 int32_t* idx, float* w, int64_t N, int d, int ne, int K);
/* Deterministic token permutation (replaces the atomic grouping of
 * cuda/moe.cu:623-651): stable order of slot s = t*K+k by expert.
 * grouped [N*K], offsets [ne+1] (device). */
int gh_moe_permute(const int32_t* idx, int64_t N, int K, int ne, int32_t* grouped, int32_t* offsets);

/* ------------------------------------------------------------------ GGUF */
/* format/gguf_codec.h:150-205 GGUFReader (open / tensors / find_tensor / get_* /
 * read_tensor_quant / read_tensor_f32), widened: GGML Q4_K (type 12) is accepted
 * next to F32, F16, Q4_0, Q4_1 and Q8_0, and packed blocks go from the mapped
 * file straight into device memory (dst_dev = GH_DEV_GPU) or host memory.
 * Errors use the reference's "gguf_format: ..." messages. */
typedef struct gh_gguf gh_gguf;
int gh_gguf_open(const char* path, gh_gguf** out);
int gh_gguf_close(gh_gguf* f);
int64_t gh_gguf_tensor_count(const gh_gguf* f);
/* dims8: up to 8 dimensions, innermost (row length) first, as stored. */
int gh_gguf_tensor_info(const gh_gguf* f, int64_t i, const char** name, uint32_t* ggml_type, int* ndims,
                        uint64_t* dims8, uint64_t* nbytes);
/* index of a tensor by the backend (= reference internal) name, or by the
 * llama.cpp alias GGUFReader::find_weight also tries (gguf_codec.cpp:1216-1258); -1 if absent */
int64_t gh_gguf_find_tensor(const gh_gguf* f, const char* name);
int gh_gguf_get_u64(const gh_gguf* f, const char* key, uint64_t* out);
int gh_gguf_get_f32(const gh_gguf* f, const char* key, float* out);
int gh_gguf_get_str(const gh_gguf* f, const char* key, char* buf, size_t cap);
/* GGUFReader::model_config (gguf_codec.cpp:1083-1180) for the Granite hybrid: the native
 * ghassan.* keys to the gh_granite_create_ex arrays (cfg with cfg[15] = qkind, then the L layer
 * kinds, tie_embeddings, moe_aux_free: *ncfg = 18 + L ints; fcfg: 5 floats). Missing keys take
 * the ModelConfig defaults; a file that is not a hybrid, or asks for what this backend does not
 * run (dense FFN, no shared expert, n_groups != 1, qk-norm, qkv / Mamba projection bias, a conv
 * without bias, positional embeddings, a sliding window), returns GH_EUNSUPPORTED. */
int gh_gguf_granite_config(const gh_gguf* f, int qkind, int32_t* cfg, int cfg_cap, float* fcfg, int fcfg_cap,
                           int* ncfg);
/* read_tensor_quant (gguf_codec.cpp:1450-1501): kind 0 Q4_0, 1 Q4_1, 2 Q8_0, 3 Q4_K. A file
 * tensor of that GGML type is copied verbatim; any other decodable type (F32, F16, Q4_0,
 * Q4_1, Q8_0, Q4_K, Q5_K, Q6_K) is decoded to fp32 and quantised on the host. */
int gh_gguf_read_packed(const gh_gguf* f, const char* name, int kind, void* dst, int dst_dev, size_t cap_bytes);
/* read_tensor_f32 (F32 / F16 in the reference), here for every decodable type above;
 * read_f16: the same rounded to fp16 (F16 verbatim). */
int gh_gguf_read_f32(const gh_gguf* f, const char* name, float* dst, int dst_dev, size_t cap_elems);
int gh_gguf_read_f16(const gh_gguf* f, const char* name, uint16_t* dst, int dst_dev, size_t cap_elems);
/* GGUFWriter (gguf_codec.h:64-130) for already-packed host data: GGUF v3, types as above,
 * metadata scalars (GGUF value types 0-7, 10-12) or strings (8), general.alignment honoured. */
int gh_gguf_write(const char* path, int n_tensors, const char* const* names, const uint32_t* ggml_types,
                  const int* ndims, const uint64_t* dims8, const void* const* data, int n_kv,
                  const char* const* keys, const uint32_t* kv_types, const void* const* kv_values);

/* -------------------------------------------------- host codec / synthetic */
/* quantization/quantize.cpp:322-341 quantize (host pointers): kinds 0-2 as
 * the reference; kind 3 (Q4_K) our own quantizer. n % block == 0 except Q8_0. */
int gh_quantize_host(int kind, const float* src, void* dst, int64_t n);
/* Synthetic parameter values by name (host): seed ^ fnv1a64(name) streams of
 * core/rng.h; norms/conv bias/D/dt_bias = 1, A_log[h] = log(h+1), else N(0,0.02). */
int gh_synth_param_f32(const char* name, uint64_t seed, float* out_host, int64_t n);
/* core/rng.h Rng(seed).normal / uniform / below streams (host). */
int gh_rng_normal_host(uint64_t seed, float mean, float sd, float* out_host, int64_t n);
int gh_rng_uniform_host(uint64_t seed, float lo, float hi, float* out_host, int64_t n);
int gh_rng_below_host(uint64_t seed, uint64_t bound, int32_t* out_host, int64_t n);

/* ------------------------------------------------ Granite-hybrid generator */
/* The caller side of the boundary (model/model.cpp forward +
 * inference/generator.cpp prefill/decode + inference/kv_cache.cpp), built on
 * the entry points above. cfg ints: V d L H KV hd E ne K SH d_inner m_heads
 * m_dhead m_dstate conv_k qkind, then L layer types (0 mamba, 1 attention);
 * fcfg: eps, attention scale. */
typedef struct gh_granite gh_granite;
int gh_granite_create(const int32_t* cfg, const float* fcfg, int max_ctx, gh_granite** out);
/* The same with the optional Granite fields: cfg[16 + L] tie_embeddings (default 1; 0 adds an fp16
 * "lm_head" [V, d], model/model.cpp:1160), cfg[17 + L] moe_aux_free (default 0; 1 adds fp32
 * "layers.N.moe_bias" [ne] router biases, model/model.cpp:179-199); fcfg[2] embedding_multiplier,
 * fcfg[3] residual_multiplier, fcfg[4] logits_scaling (default 1; inference/generator.cpp:248,
 * 266, 440, model/model.cpp:2431, 2531). Entries past ncfg / nfcfg take their defaults. */
int gh_granite_create_ex(const int32_t* cfg, int ncfg, const float* fcfg, int nfcfg, int max_ctx,
                         gh_granite** out);
int gh_granite_destroy(gh_granite* g);
/* Parameter storage bytes by reference name (host buffer, nbytes must match). */
int gh_granite_set_param(gh_granite* g, const char* name, const void* host, size_t nbytes);
int gh_granite_init_synthetic(gh_granite* g, uint64_t seed);
int gh_granite_param_count(gh_granite* g);
int gh_granite_param_name(gh_granite* g, int i, const char** name, size_t* nbytes);
int gh_granite_get_param(gh_granite* g, const char* name, void* host, size_t nbytes);
int gh_granite_reset(gh_granite* g);
/* load_model_from_gguf (gguf_codec.cpp:1507-1564) for a created model: every
 * parameter by its name (or llama.cpp alias) from the file, packed weights in
 * the model's kind (verbatim when the file holds that kind, including Q4_K),
 * fp16 / fp32 vectors decoded. Shapes must match the model's configuration. */
int gh_granite_load_gguf(gh_granite* g, const gh_gguf* f);
/* The reference's load path in one call (gguf_codec.cpp:1083-1180 model_config, then Model
 * construction and load_model_from_gguf, 1507-1564): open the file, build the model from its
 * metadata with weights packed as qkind, load every parameter, close the file. */
int gh_granite_open_gguf(const char* path, int qkind, int max_ctx, gh_granite** out);
/* Generator::prefill + first logits (inference/generator.cpp:917-983).
 * logits_host may be NULL. mamba_mode: 0 token-by-token state updates
 * (the reference's order), 1 chunked SSD scan. */
int gh_granite_prefill(gh_granite* g, const int32_t* ids_host, int P, float* logits_host, int mamba_mode);
/* One decode step (inference/generator.cpp:221-443) for `token`. */
int gh_granite_decode(gh_granite* g, int32_t token, float* logits_host);
/* Greedy generation of n_new ids from the current logits
 * (inference/generator.cpp:985-1098, greedy branch). use_graph: 0 launches the decode
 * step's kernels one by one; 1 captures the step (embedding .. argmax) in a hipGraph
 * and replays it; 2 runs the whole loop as one persistent cooperative launch (falls back
 * to 1 when the model's shapes or the context do not fit that kernel). */
int gh_granite_generate_greedy(gh_granite* g, int n_new, int32_t* ids_host, int use_graph);
/* When a persistent launch (use_graph 2) aborts (a bounded hand-over wait ran out), the
 * recurrent state, KV cache and ids are partly advanced: generate returns GH_EHIP and the
 * model refuses prefill / decode / generate until gh_granite_reset. Test hook, no reference
 * counterpart: makes the next persistent launch start with its abort flag raised (every
 * kernel still runs to its end), to exercise that contract. */
int gh_granite_test_force_abort(gh_granite* g);

#ifdef __cplusplus
}
#endif
#endif /* GHASSAN_HIP_H */
