// extern "C" shim over the genuine reference engine's CPU path, compiled
// from /root/reference by oracle/ref.mk into oracle/_ref/libgai_ref.so.
// TEST INFRASTRUCTURE ONLY: tests/golden/make_golden.py loads it in the build
// container to write golden fixtures, and bench.py's cpu_baseline leg times
// the reference CPU Generator through it (the built .so travels with the
// tree; no reference source does). The product never links it.
//
// The Generator's per-token host path is private in the reference; the shim
// reaches it by opening the class (test code only), so the greedy loop below
// is the reference's own prefill + decode_step + greedy argmax
// (inference/generator.cpp:917-1098 with the greedy branch of
// inference/sampler.cpp:129-141).
#include "core/ops.h"
#include "core/ops_cpu.h"
#include "core/rng.h"
#include "core/dtype.h"
#include "quantization/quantize.h"
#include "model/model.h"
#include "format/gguf_codec.h"
#define private public
#include "inference/generator.h"
#undef private

#include <cmath>
#include <cstring>
#include <limits>
#include <map>
#include <string>
#include <vector>

using namespace gai;

extern "C" {

void ref_f32_to_f16(const float* s, u16* d, i64 n) { for (i64 i = 0; i < n; ++i) d[i] = fp32_to_fp16(s[i]); }
void ref_f16_to_f32(const u16* s, float* d, i64 n) { for (i64 i = 0; i < n; ++i) d[i] = fp16_to_fp32(s[i]); }
void ref_f32_to_bf16(const float* s, u16* d, i64 n) { for (i64 i = 0; i < n; ++i) d[i] = fp32_to_bf16(s[i]); }

void ref_rng_normal(u64 seed, float mean, float sd, float* out, i64 n) {
    Rng r(seed);
    for (i64 i = 0; i < n; ++i) out[i] = r.normal(mean, sd);
}
void ref_rng_uniform(u64 seed, float lo, float hi, float* out, i64 n) {
    Rng r(seed);
    for (i64 i = 0; i < n; ++i) out[i] = r.uniform(lo, hi);
}
void ref_rng_below(u64 seed, u64 bound, i32* out, i64 n) {
    Rng r(seed);
    for (i64 i = 0; i < n; ++i) out[i] = (i32)r.below(bound);
}

int ref_quantize(int kind, const float* src, void* dst, i64 n) {
    try {
        if (kind == 0) quant::quantize_q4_0(src, dst, n);
        else if (kind == 1) quant::quantize_q4_1(src, dst, n);
        else if (kind == 2) quant::quantize_q8_0(src, dst, n);
        else return -1;
    } catch (...) { return -2; }
    return 0;
}
int ref_dequantize(int kind, const void* src, float* dst, i64 n) {
    try {
        if (kind == 0) quant::dequantize_q4_0(src, dst, n);
        else if (kind == 1) quant::dequantize_q4_1(src, dst, n);
        else if (kind == 2) quant::dequantize_q8_0(src, dst, n);
        else return -1;
    } catch (...) { return -2; }
    return 0;
}
int ref_quant_materialize(int kind, const void* packed, u16* out, i64 n) {
    try {
        const u16* p = ops::quant_materialize(Device::CPU, packed, kind, n, 0);
        std::memcpy(out, p, (size_t)n * 2);
    } catch (...) { return -2; }
    return 0;
}
int ref_linear_forward_q4(const float* x, const void* w, float* y, int M, int K, int N, int kind) {
    try { ops::linear_forward_q4(Device::CPU, x, w, y, M, K, N, kind); } catch (...) { return -2; }
    return 0;
}
void ref_linear_forward_fp16(const float* x, const u16* w, float* y, int M, int K, int N) {
    ops::linear_forward_fp16(Device::CPU, x, w, y, M, K, N);
}
void ref_linear_forward_f32(const float* x, const float* w, float* y, int M, int K, int N) {
    ops::linear_forward(Device::CPU, x, w, y, M, K, N);
}
void ref_rmsnorm_forward(const float* x, const float* w, float* out, float* rrms, i64 rows, int dim, float eps) {
    ops::rmsnorm_forward(Device::CPU, x, w, out, rrms, rows, dim, eps);
}
void ref_swiglu_forward(const float* g, const float* u, float* out, i64 n) {
    ops::swiglu_forward(Device::CPU, g, u, out, n);
}
void ref_softmax_row(float* x, int n) { cpu::softmax_row(x, n); }
i32 ref_argmax_token(const float* l, int V) { return ops::argmax_token(Device::CPU, l, V); }
void ref_topk_select(const float* l, int V, int K, float* vals, i32* ids) {
    ops::topk_select(Device::CPU, l, V, K, vals, ids);
}
void ref_apply_rep_penalties(float* l, int V, const i32* hist, int n, float rep, float freq, float pres) {
    ops::apply_rep_penalties(Device::CPU, l, V, hist, n, rep, freq, pres);
}
void ref_embedding_forward_half(const i32* ids, const u16* table, float* out, i64 ntok, int dim, int vocab) {
    ops::embedding_forward_half(Device::CPU, ids, table, out, ntok, dim, vocab);
}
void ref_attention_forward_ex(const float* q, const float* k, const float* v, float* out, int B, int T, int H,
                              int KV, int hd, float scale, int window) {
    ops::attention_forward_ex(Device::CPU, q, k, v, out, nullptr, B, T, H, KV, hd, scale, window, nullptr);
}
int ref_attention_decode_ring_fp16(const float* q, const u16* kc, const u16* vc, float* out, int H, int KV, int hd,
                                   int ring_start, int pinned, int cur_len, int cache_max, float scale,
                                   int window) {
    std::vector<float> scratch((size_t)H * (size_t)(cur_len > 0 ? cur_len : 1));
    try {
        ops::attention_decode_ring_fp16(Device::CPU, q, kc, vc, out, H, KV, hd, ring_start, pinned, cur_len,
                                        cache_max, scale, scratch.data(), window);
    } catch (...) { return -2; }
    return 0;
}
int ref_mamba2_forward_half(const float* x, const void* w_in, const float* conv_w, const float* conv_b,
                            const float* dt_bias, const float* a_log, const float* D, const float* norm_w,
                            const void* w_out, float* state, float* out, int B, int T, int d, int d_inner,
                            int conv_dim, int n_heads, int d_head, int d_state, int k, float eps, int qkind) {
    try {
        ops::mamba2_forward_half(Device::CPU, x, (const u16*)w_in, conv_w, conv_b, dt_bias, a_log, D, norm_w,
                                 (const u16*)w_out, state, out, B, T, d, d_inner, conv_dim, n_heads, d_head,
                                 d_state, k, eps, qkind);
    } catch (...) { return -2; }
    return 0;
}
int ref_moe_forward_bias_half(const float* x, const float* rw, const float* bias, const void* g, const void* u,
                              const void* dn, const void* sg, const void* su, const void* sd, float* out,
                              float* probs, i32* idx, float* w, i64 N, int d, int E, int ne, int K, int SH,
                              int qkind) {
    std::vector<float> s_gate((size_t)N * K * E), s_up(s_gate.size()), s_act(s_gate.size());
    try {
        ops::moe_forward_bias_half(Device::CPU, x, rw, bias, (const u16*)g, (const u16*)u, (const u16*)dn,
                                   (const u16*)sg, (const u16*)su, (const u16*)sd, out, probs, idx, w,
                                   s_gate.data(), s_up.data(), s_act.data(), N, d, E, ne, K, SH, qkind);
    } catch (...) { return -2; }
    return 0;
}

// Tiny Granite-hybrid greedy run through the reference Model + Generator.
// cfg / fcfg use the same layout as orc_granite_generate (oracle/oracle.h).
// Parameters are set by name from caller buffers holding the storage bytes
// (Q-kind blocks for matrices, fp16 for tok_embeddings, fp32 for vectors).
int ref_granite_generate_timed(const i32* cfg, const float* fcfg, const char** names, const void** ptrs, int nparams,
                               const i32* prompt, int P, int n_new, int max_ctx, i32* out_ids, float* out_margins,
                               double* seconds);

int ref_granite_generate(const i32* cfg, const float* fcfg, const char** names, const void** ptrs, int nparams,
                         const i32* prompt, int P, int n_new, int max_ctx, i32* out_ids, float* out_margins) {
    return ref_granite_generate_timed(cfg, fcfg, names, ptrs, nparams, prompt, P, n_new, max_ctx, out_ids,
                                      out_margins, nullptr);
}

int ref_granite_generate_ex(const i32* cfg, int ncfg, const float* fcfg, int nfcfg, const char** names,
                            const void** ptrs, int nparams, const i32* prompt, int P, int n_new, int max_ctx,
                            const i32* forced, i32* out_ids, float* out_margins, float* out_logits, double* seconds);

// seconds (optional): [0] prefill wall time, [1] wall time of the n_new-1
// decode steps (Generator::decode_step on the host path).
int ref_granite_generate_timed(const i32* cfg, const float* fcfg, const char** names, const void** ptrs, int nparams,
                               const i32* prompt, int P, int n_new, int max_ctx, i32* out_ids, float* out_margins,
                               double* seconds) {
    return ref_granite_generate_ex(cfg, 16 + cfg[2], fcfg, 2, names, ptrs, nparams, prompt, P, n_new, max_ctx,
                                   nullptr, out_ids, out_margins, nullptr, seconds);
}

// The optional Granite fields of orc_granite_generate_ex (oracle/oracle.h) set on the
// reference ModelConfig: tie_embeddings, moe_aux_free (router biases from parameters named
// "layers.N.moe_bias" through Model::set_moe_bias, as load_model_from_gguf does), and the
// embedding / residual multipliers and logits scaling.
static void granite_options(ModelConfig& c, const i32* cfg, int ncfg, const float* fcfg, int nfcfg) {
    const int L = cfg[2];
    c.tie_embeddings = ncfg > 16 + L ? cfg[16 + L] != 0 : true;
    c.moe_aux_free = ncfg > 17 + L ? cfg[17 + L] != 0 : false;
    if (c.moe_aux_free) c.moe_aux_scale = 0.0f;  // model/model.cpp:388 (no aux-loss term with the bias)
    if (nfcfg > 2) c.embedding_multiplier = fcfg[2];
    if (nfcfg > 3) c.residual_multiplier = fcfg[3];
    if (nfcfg > 4) c.logits_scaling = fcfg[4];
}

// forced (optional): the id fed at each step instead of the greedy one (out_ids
// keeps the greedy id); out_logits (optional, n_new x V): the host logits of each step.
int ref_granite_generate_ex(const i32* cfg, int ncfg, const float* fcfg, int nfcfg, const char** names,
                            const void** ptrs, int nparams, const i32* prompt, int P, int n_new, int max_ctx,
                            const i32* forced, i32* out_ids, float* out_margins, float* out_logits, double* seconds) {
    try {
        ModelConfig c;
        c.arch = ModelConfig::ArchGranite;
        c.vocab_size = cfg[0];
        c.hidden_size = cfg[1];
        c.num_layers = cfg[2];
        c.num_heads = cfg[3];
        c.num_kv_heads = cfg[4];
        c.head_dim_override = cfg[5];
        c.moe_expert_dim = cfg[6];
        c.num_experts = cfg[7];
        c.moe_top_k = cfg[8];
        c.shared_expert_intermediate_size = cfg[9];
        c.use_moe = true;
        c.moe_shared = true;
        c.mamba_expand = cfg[10] / cfg[1];
        c.mamba_n_heads = cfg[11];
        c.mamba_d_head = cfg[12];
        c.mamba_d_state = cfg[13];
        c.mamba_n_groups = 1;
        c.mamba_d_conv = cfg[14];
        c.layer_types.assign(cfg + 16, cfg + 16 + cfg[2]);
        c.position_embedding = 1;  // NoPE
        c.rms_eps = fcfg[0];
        c.attention_multiplier = fcfg[1];
        c.intermediate_size = cfg[6];
        c.max_seq_len = max_ctx;
        c.tie_embeddings = true;
        granite_options(c, cfg, ncfg, fcfg, nfcfg);
        const int qkind = cfg[15];
        Model m(c, Device::CPU, false, qkind);
        std::map<std::string, const void*> pm;
        for (int i = 0; i < nparams; ++i) pm[names[i]] = ptrs[i];
        for (Parameter* p : m.parameters()) {
            auto it = pm.find(p->name);
            if (it == pm.end()) return -3;
            std::memcpy(p->w.data_ptr(), it->second, p->w.nbytes());
        }
        if (c.moe_aux_free) {
            for (int l = 0; l < c.num_layers; ++l) {
                auto it = pm.find("layers." + std::to_string(l) + ".moe_bias");
                if (it != pm.end()) m.set_moe_bias(l, (const float*)it->second, (size_t)c.num_experts);
            }
        }
        ops::set_fused_q4(true);
        Tokenizer tok;
        Generator g(m, tok, max_ctx);
        std::vector<i32> pr(prompt, prompt + P);
        Timer tp;
        g.prefill(pr);
        if (seconds) seconds[0] = tp.seconds();
        Timer td;
        const int V = c.vocab_size;
        for (int step = 0; step < n_new; ++step) {
            const float* lg = g.logits_host_.data();
            const i32 next = ops::argmax_token(Device::CPU, lg, V);
            float best = -std::numeric_limits<float>::infinity(), second = best;
            for (int i = 0; i < V; ++i) {
                if (!std::isfinite(lg[i])) continue;
                if (lg[i] > best) { second = best; best = lg[i]; }
                else if (lg[i] > second) second = lg[i];
            }
            out_ids[step] = next;
            out_margins[step] = best - second;
            if (out_logits) std::memcpy(out_logits + (size_t)step * V, lg, sizeof(float) * (size_t)V);
            if (step == n_new - 1) break;
            const i32 fed = forced ? forced[step] : next;
            g.push_history(fed);
            g.decode_step(fed, (int)g.absolute_pos_);
            ++g.absolute_pos_;
        }
        if (seconds) seconds[1] = td.seconds();
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_granite_generate: %s\n", e.what());
        return -2;
    }
    return 0;
}

// The parameter table the reference Model allocates for a config: names,
// element counts and storage dtypes (core/dtype.h:9-21 numbering), so the
// fixture writer fills exactly the tensors the reference expects.
int ref_granite_param_table_ex(const i32* cfg, int ncfg, const float* fcfg, int nfcfg, int max_ctx,
                               char* names_out, int names_cap, i64* numel_out, i32* dtype_out, int cap);
int ref_granite_param_table(const i32* cfg, const float* fcfg, int max_ctx, char* names_out, int names_cap,
                            i64* numel_out, i32* dtype_out, int cap) {
    return ref_granite_param_table_ex(cfg, 16 + cfg[2], fcfg, 2, max_ctx, names_out, names_cap, numel_out, dtype_out,
                                      cap);
}
int ref_granite_param_table_ex(const i32* cfg, int ncfg, const float* fcfg, int nfcfg, int max_ctx,
                               char* names_out, int names_cap, i64* numel_out, i32* dtype_out, int cap) {
    ModelConfig c;
    c.arch = ModelConfig::ArchGranite;
    c.vocab_size = cfg[0]; c.hidden_size = cfg[1]; c.num_layers = cfg[2]; c.num_heads = cfg[3];
    c.num_kv_heads = cfg[4]; c.head_dim_override = cfg[5]; c.moe_expert_dim = cfg[6]; c.num_experts = cfg[7];
    c.moe_top_k = cfg[8]; c.shared_expert_intermediate_size = cfg[9]; c.use_moe = true; c.moe_shared = true;
    c.mamba_expand = cfg[10] / cfg[1]; c.mamba_n_heads = cfg[11]; c.mamba_d_head = cfg[12];
    c.mamba_d_state = cfg[13]; c.mamba_n_groups = 1; c.mamba_d_conv = cfg[14];
    c.layer_types.assign(cfg + 16, cfg + 16 + cfg[2]); c.position_embedding = 1; c.rms_eps = fcfg[0];
    c.attention_multiplier = fcfg[1]; c.intermediate_size = cfg[6]; c.max_seq_len = max_ctx;
    c.tie_embeddings = true;
    granite_options(c, cfg, ncfg, fcfg, nfcfg);
    Model m(c, Device::CPU, false, cfg[15]);
    int i = 0, off = 0;
    for (Parameter* p : m.parameters()) {
        if (i >= cap) return -1;
        const int l = (int)p->name.size() + 1;
        if (off + l > names_cap) return -1;
        std::memcpy(names_out + off, p->name.c_str(), (size_t)l);
        off += l;
        numel_out[i] = p->w.numel();
        dtype_out[i] = (i32)p->w.dtype();
        ++i;
    }
    return i;
}


// GGUF through the reference's own writer and reader (format/gguf_codec.cpp):
// three tensors of the given f32 values -- F32 [r0][64], Q8_0 [r1][64] and
// F16 [r2][64] -- plus a few metadata keys.
int ref_gguf_write(const char* path, const float* a, int r0, const float* b, int r1, const float* c, int r2) {
    auto mk = [](const float* v, int rows) {
        Tensor t({(i64)rows, 64}, DType::F32, Device::CPU);
        std::memcpy(t.data_ptr(), v, sizeof(float) * (size_t)rows * 64);
        return t;
    };
    GGUFWriter w(path);
    w.set_arch("ghassan");
    w.set_hidden_size(64);
    w.set_num_layers(2);
    w.set_rms_eps(1e-5f);
    w.add_tensor("layers.0.attn_norm", mk(a, r0), GGMLType::F32);
    w.add_tensor("layers.0.wq", mk(b, r1), GGMLType::Q8_0);
    w.add_tensor("tok_embeddings", mk(c, r2), GGMLType::F16);
    w.write();
    return 0;
}
// packed bytes of a Q8_0 tensor as the reference's loader returns them
long ref_gguf_read_q8(const char* path, const char* name, void* out, long cap) {
    GGUFReader r;
    if (!r.open(path)) return -1;
    Tensor t = r.read_tensor_quant(name, DType::Q8_0);
    if ((long)t.nbytes() > cap) return -2;
    std::memcpy(out, t.data_ptr(), t.nbytes());
    return (long)t.nbytes();
}
long ref_gguf_read_f32(const char* path, const char* name, float* out, long cap) {
    GGUFReader r;
    if (!r.open(path)) return -1;
    Tensor t = r.read_tensor_f32(name);
    if ((long)t.numel() > cap) return -2;
    std::memcpy(out, t.data_ptr(), sizeof(float) * (size_t)t.numel());
    return (long)t.numel();
}
// The model of ref_granite_generate_ex written by the reference's own exporter
// (format/gguf_codec.cpp:1672 export_model_gguf: native ghassan.* keys, the "q8_k" profile with
// the hybrid precision policy), with an empty tokenizer.
int ref_granite_export_gguf(const i32* cfg, int ncfg, const float* fcfg, int nfcfg, const char** names,
                            const void** ptrs, int nparams, int max_ctx, const char* path) {
    try {
        ModelConfig c;
        c.arch = ModelConfig::ArchGranite;
        c.vocab_size = cfg[0]; c.hidden_size = cfg[1]; c.num_layers = cfg[2]; c.num_heads = cfg[3];
        c.num_kv_heads = cfg[4]; c.head_dim_override = cfg[5]; c.moe_expert_dim = cfg[6]; c.num_experts = cfg[7];
        c.moe_top_k = cfg[8]; c.shared_expert_intermediate_size = cfg[9]; c.use_moe = true; c.moe_shared = true;
        c.mamba_expand = cfg[10] / cfg[1]; c.mamba_n_heads = cfg[11]; c.mamba_d_head = cfg[12];
        c.mamba_d_state = cfg[13]; c.mamba_n_groups = 1; c.mamba_d_conv = cfg[14];
        c.layer_types.assign(cfg + 16, cfg + 16 + cfg[2]); c.position_embedding = 1; c.rms_eps = fcfg[0];
        c.attention_multiplier = fcfg[1]; c.intermediate_size = cfg[6]; c.max_seq_len = max_ctx;
        c.tie_embeddings = true;
        granite_options(c, cfg, ncfg, fcfg, nfcfg);
        Model m(c, Device::CPU, false, cfg[15]);
        std::map<std::string, const void*> pm;
        for (int i = 0; i < nparams; ++i) pm[names[i]] = ptrs[i];
        for (Parameter* p : m.parameters()) {
            auto it = pm.find(p->name);
            if (it == pm.end()) return -3;
            std::memcpy(p->w.data_ptr(), it->second, p->w.nbytes());
        }
        if (c.moe_aux_free) {
            for (int l = 0; l < c.num_layers; ++l) {
                auto it = pm.find("layers." + std::to_string(l) + ".moe_bias");
                if (it != pm.end()) m.set_moe_bias(l, (const float*)it->second, (size_t)c.num_experts);
            }
        }
        ExportProfileGGUF prof = gguf_profile_for("q8_k");
        prof.hybrid = true;
        Tokenizer tok;
        export_model_gguf(path, m, tok, prof, {}, "native");
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_granite_export_gguf: %s\n", e.what());
        return -2;
    }
    return 0;
}

// A model file as the reference loads it -- GGUFReader::model_config(), then
// load_model_from_gguf with storage kind qkind (format/gguf_codec.cpp:1083-1180, 1507-1563) --
// and its greedy run (the loop of ref_granite_generate_ex). cfg_out (16 + L + 2 ints) and
// fcfg_out (5 floats) receive the parsed configuration in the layout of
// orc_granite_generate_ex.
int ref_granite_generate_gguf(const char* path, int qkind, const i32* prompt, int P, int n_new, int max_ctx,
                              i32* out_ids, float* out_margins, i32* cfg_out, int cfg_cap, float* fcfg_out) {
    try {
        GGUFReader r;
        if (!r.open(path)) return -4;
        const ModelConfig c = r.model_config();
        if (cfg_out) {
            if (cfg_cap < 18 + c.num_layers) return -5;
            const i32 v[16] = {c.vocab_size, c.hidden_size, c.num_layers, c.num_heads, c.num_kv_heads, c.head_dim(),
                               c.moe_expert_dim, c.num_experts, c.moe_top_k, c.shared_expert_intermediate_size,
                               c.mamba_expand * c.hidden_size, c.mamba_n_heads, c.mamba_d_head, c.mamba_d_state,
                               c.mamba_d_conv, qkind};
            std::memcpy(cfg_out, v, sizeof v);
            for (int l = 0; l < c.num_layers; ++l) cfg_out[16 + l] = c.layer_types[l];
            cfg_out[16 + c.num_layers] = c.tie_embeddings ? 1 : 0;
            cfg_out[17 + c.num_layers] = c.moe_aux_free ? 1 : 0;
        }
        if (fcfg_out) {
            fcfg_out[0] = c.rms_eps;
            fcfg_out[1] = c.attention_multiplier;
            fcfg_out[2] = c.embedding_multiplier;
            fcfg_out[3] = c.residual_multiplier;
            fcfg_out[4] = c.logits_scaling;
        }
        Model m(c, Device::CPU, false, qkind);
        if (!load_model_from_gguf(path, m, qkind)) return -6;
        ops::set_fused_q4(true);
        Tokenizer tok;
        Generator g(m, tok, max_ctx);
        std::vector<i32> pr(prompt, prompt + P);
        g.prefill(pr);
        const int V = c.vocab_size;
        for (int step = 0; step < n_new; ++step) {
            const float* lg = g.logits_host_.data();
            const i32 next = ops::argmax_token(Device::CPU, lg, V);
            float best = -std::numeric_limits<float>::infinity(), second = best;
            for (int i = 0; i < V; ++i) {
                if (!std::isfinite(lg[i])) continue;
                if (lg[i] > best) { second = best; best = lg[i]; }
                else if (lg[i] > second) second = lg[i];
            }
            out_ids[step] = next;
            out_margins[step] = best - second;
            if (step == n_new - 1) break;
            g.push_history(next);
            g.decode_step(next, (int)g.absolute_pos_);
            ++g.absolute_pos_;
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_granite_generate_gguf: %s\n", e.what());
        return -2;
    }
    return 0;
}
}  // extern "C"
