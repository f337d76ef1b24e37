// GGUF v2/v3 reader and writer for the weight formats of the path, with the
// K-quant passthrough the reference's loader lacks (format/gguf_codec.cpp:
// GGUFReader::open :697-731, read_tensor_info :862-909, read_tensor_quant
// :1450-1501; it accepts F32/F16/Q4_0/Q4_1/Q8_0 only).
//
// The file is memory-mapped once; tensor infos are parsed into a table and
// packed blocks are copied straight from the mapping into device memory (one
// hipMemcpy per tensor, no host staging) when the file's GGML type is the
// backend kind asked for. Otherwise F32/F16 tensors are decoded and quantised
// on the host like the reference's slow path (quant::quantize). Layout facts
// kept alike with the reference: little-endian fields, dimensions innermost
// first, the data section at the end of the tensor infos rounded up to the
// alignment (general.alignment when present, else 32 -- the reference always
// uses 32, which is the same for files without the key), tensor offsets
// relative to the data section.
#include <fcntl.h>
#include <math.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <map>
#include <string>
#include <vector>

#include "../../include/ghassan_hip.h"
#include "gh_common.h"

namespace {

enum : uint32_t { GT_F32 = 0, GT_F16 = 1, GT_Q4_0 = 2, GT_Q4_1 = 3, GT_Q8_0 = 8, GT_Q4_K = 12, GT_Q5_K = 13, GT_Q6_K = 14 };
enum : uint32_t {
    KV_U8 = 0, KV_I8 = 1, KV_U16 = 2, KV_I16 = 3, KV_U32 = 4, KV_I32 = 5, KV_F32 = 6, KV_BOOL = 7,
    KV_STR = 8, KV_ARR = 9, KV_U64 = 10, KV_I64 = 11, KV_F64 = 12
};
constexpr uint32_t GGUF_MAGIC = 0x46554747u;  // "GGUF"

// block values / bytes of a GGML type (0 bytes = unsupported)
void ggml_block(uint32_t t, uint64_t& vals, uint64_t& bytes) {
    vals = 1;
    bytes = 0;
    switch (t) {
        case GT_F32: bytes = 4; break;
        case GT_F16: bytes = 2; break;
        case GT_Q4_0: vals = 32; bytes = 18; break;
        case GT_Q4_1: vals = 32; bytes = 20; break;
        case GT_Q8_0: vals = 32; bytes = 34; break;
        case GT_Q4_K: vals = 256; bytes = 144; break;
        case GT_Q5_K: vals = 256; bytes = 176; break;
        case GT_Q6_K: vals = 256; bytes = 210; break;
        default: break;
    }
}

// backend kind (0 Q4_0, 1 Q4_1, 2 Q8_0, 3 Q4_K) -> GGML type
uint32_t kind_type(int kind) {
    static const uint32_t t[4] = {GT_Q4_0, GT_Q4_1, GT_Q8_0, GT_Q4_K};
    return kind >= 0 && kind < 4 ? t[kind] : 0xFFFFFFFFu;
}

size_t kv_scalar_size(uint32_t t) {
    switch (t) {
        case KV_U8: case KV_I8: case KV_BOOL: return 1;
        case KV_U16: case KV_I16: return 2;
        case KV_U32: case KV_I32: case KV_F32: return 4;
        case KV_U64: case KV_I64: case KV_F64: return 8;
        default: return 0;
    }
}

struct Cursor {
    const uint8_t* p;
    size_t n, at = 0;
    bool ok = true;
    template <typename T>
    T pod() {
        T v{};
        if (at + sizeof(T) > n) { ok = false; return v; }
        memcpy(&v, p + at, sizeof(T));
        at += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t len = pod<uint64_t>();
        if (!ok || len > n - at) { ok = false; return {}; }
        std::string s((const char*)p + at, (size_t)len);
        at += (size_t)len;
        return s;
    }
    bool skip(uint64_t b) {
        if (b > n - at) return ok = false;
        at += (size_t)b;
        return true;
    }
};

struct KV {
    uint32_t type;
    size_t off;  // value bytes in the mapping
    uint32_t arr_type = 0;
    uint64_t arr_n = 0;
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type;
    uint64_t offset, numel, nbytes;
};

uint16_t f32_to_half_bits(float f) { return gh::f32_to_f16(f); }
float half_bits_to_f32(uint16_t h) { return gh::f16_to_f32(h); }

}  // namespace

struct gh_gguf {
    int fd = -1;
    const uint8_t* map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t data_start = 0;
    std::map<std::string, KV> kv;
    std::vector<Tensor> tensors;
    std::map<std::string, size_t> by_name;
};

namespace {

void close_file(gh_gguf* g) {
    if (g->map) munmap((void*)g->map, g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

// The reference's naming of llama.cpp-style files (format/gguf_codec.cpp:1216-1245)
// for the parameters both know; the backend's own names are tried first.
std::string llama_alias(const std::string& internal) {
    if (internal == "tok_embeddings") return "token_embd.weight";
    if (internal == "final_norm") return "output_norm.weight";
    if (internal == "lm_head") return "output.weight";
    const std::string pre = "layers.";
    if (internal.compare(0, pre.size(), pre) != 0) return {};
    const size_t dot = internal.find('.', pre.size());
    if (dot == std::string::npos) return {};
    const std::string blk = "blk." + internal.substr(pre.size(), dot - pre.size()) + ".";
    static const std::map<std::string, std::string> rest = {
        {"attn_norm", "attn_norm.weight"}, {"wq", "attn_q.weight"},        {"wk", "attn_k.weight"},
        {"wv", "attn_v.weight"},           {"wo", "attn_output.weight"},  {"ffn_norm", "ffn_norm.weight"},
    };
    auto it = rest.find(internal.substr(dot + 1));
    return it == rest.end() ? std::string() : blk + it->second;
}

const Tensor* find(const gh_gguf* g, const std::string& name) {
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) {
        const std::string alt = llama_alias(name);
        if (!alt.empty()) it = g->by_name.find(alt);
    }
    return it == g->by_name.end() ? nullptr : &g->tensors[it->second];
}

int copy_out(void* dst, int dst_dev, const void* src, size_t bytes) {
    if (dst_dev == GH_DEV_GPU) {
        GH_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    } else {
        memcpy(dst, src, bytes);
    }
    return GH_OK;
}

// ---- block decoders (host), fp32 arithmetic without fused multiply-add. Q4_0 / Q4_1 /
// Q8_0 as quantization/quantize.cpp:114-133 dequantizes them; the K-quants (absent from the
// reference) by the GGML block layouts: 256 values per super-block, fp16 d (and dmin), 32- or
// 16-value sub-blocks with their own scales.
#pragma clang fp contract(off)
float h16(const uint8_t* p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return half_bits_to_f32(h);
}
// the 6-bit (scale, min) pair j of a Q4_K / Q5_K header's 12 scale bytes
void k_scale_min(const uint8_t* sc, int j, int& s, int& m) {
    if (j < 4) {
        s = sc[j] & 63;
        m = sc[j + 4] & 63;
    } else {
        s = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4);
        m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}
// Q4_K (144 B): d, dmin, scales[12], qs[128]; byte 32 i + l holds value l of sub-block 2 i
// (low nibble) and of sub-block 2 i + 1 (high nibble); v = (d s_j) q - dmin m_j.
void dec_q4_k(const uint8_t* b, float* y) {
    const float d = h16(b), dmin = h16(b + 2);
    for (int j = 0; j < 8; ++j) {
        int s, m;
        k_scale_min(b + 4, j, s, m);
        const float d1 = d * (float)s, m1 = dmin * (float)m;
        for (int l = 0; l < 32; ++l) {
            const uint8_t q = b[16 + 32 * (j >> 1) + l];
            y[32 * j + l] = d1 * (float)((j & 1) ? (q >> 4) : (q & 0xF)) - m1;
        }
    }
}
// Q5_K (176 B): d, dmin, scales[12], qh[32], qs[128]: as Q4_K, the fifth bit of value l of
// sub-block j is bit j of qh[l].
void dec_q5_k(const uint8_t* b, float* y) {
    const float d = h16(b), dmin = h16(b + 2);
    const uint8_t* qh = b + 16;
    const uint8_t* qs = b + 48;
    for (int j = 0; j < 8; ++j) {
        int s, m;
        k_scale_min(b + 4, j, s, m);
        const float d1 = d * (float)s, m1 = dmin * (float)m;
        for (int l = 0; l < 32; ++l) {
            const uint8_t q = qs[32 * (j >> 1) + l];
            const int v = ((j & 1) ? (q >> 4) : (q & 0xF)) | (((qh[l] >> j) & 1) << 4);
            y[32 * j + l] = d1 * (float)v - m1;
        }
    }
}
// Q6_K (210 B): ql[128], qh[64], scales[16] (int8), d. In each half (128 values) h, value
// 32 r + l (r = 0..3) takes the low nibble of ql[64 h + l] (r = 0), of ql[64 h + 32 + l]
// (r = 1), the high nibbles of the same bytes (r = 2, 3), and bits 2 r, 2 r + 1 of
// qh[32 h + l] above them; v = (d sc) (q - 32) with sc = scales[8 h + 2 r + l / 16].
void dec_q6_k(const uint8_t* b, float* y) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    const float d = h16(b + 208);
    for (int h = 0; h < 2; ++h)
        for (int r = 0; r < 4; ++r)
            for (int l = 0; l < 32; ++l) {
                const uint8_t lb = ql[64 * h + 32 * (r & 1) + l];
                const int lo = (r < 2) ? (lb & 0xF) : (lb >> 4);
                const int q = lo | (((qh[32 * h + l] >> (2 * r)) & 3) << 4);
                y[128 * h + 32 * r + l] = (d * (float)sc[8 * h + 2 * r + l / 16]) * (float)(q - 32);
            }
}
void dec_q8_0(const uint8_t* b, float* y) {
    const float d = h16(b);
    for (int i = 0; i < 32; ++i) y[i] = (float)(int8_t)b[2 + i] * d;
}
void dec_q4_0(const uint8_t* b, float* y) {
    const float d = h16(b);
    for (int i = 0; i < 16; ++i) {
        y[i] = (float)((b[2 + i] & 0xF) - 8) * d;
        y[i + 16] = (float)((b[2 + i] >> 4) - 8) * d;
    }
}
void dec_q4_1(const uint8_t* b, float* y) {
    const float d = h16(b), m = h16(b + 2);
    for (int i = 0; i < 16; ++i) {
        y[i] = (float)(b[4 + i] & 0xF) * d + m;
        y[i + 16] = (float)(b[4 + i] >> 4) * d + m;
    }
}
#pragma clang fp contract(on)

// any supported tensor -> fp32 host values (the reference's read_tensor_f32 / the decode step
// of read_tensor_quant's slow path, gguf_codec.cpp:1495-1500)
int decode_f32(const gh_gguf* g, const Tensor& t, std::vector<float>& out) {
    const uint8_t* src = g->map + g->data_start + t.offset;
    out.resize((size_t)t.numel);
    if (t.type == GT_F32) {
        memcpy(out.data(), src, (size_t)t.numel * 4);
        return GH_OK;
    }
    if (t.type == GT_F16) {
        for (uint64_t i = 0; i < t.numel; ++i) out[(size_t)i] = h16(src + 2 * i);
        return GH_OK;
    }
    void (*dec)(const uint8_t*, float*) = nullptr;
    switch (t.type) {
        case GT_Q4_0: dec = dec_q4_0; break;
        case GT_Q4_1: dec = dec_q4_1; break;
        case GT_Q8_0: dec = dec_q8_0; break;
        case GT_Q4_K: dec = dec_q4_k; break;
        case GT_Q5_K: dec = dec_q5_k; break;
        case GT_Q6_K: dec = dec_q6_k; break;
        default:
            return gh::fail(GH_EUNSUPPORTED, "gguf: tensor '%s' has GGML type %u, which cannot be decoded",
                            t.name.c_str(), t.type);
    }
    uint64_t bv, bb;
    ggml_block(t.type, bv, bb);
    const uint64_t nb = t.numel / bv;
    for (uint64_t i = 0; i < nb; ++i) dec(src + i * bb, out.data() + i * bv);
    return GH_OK;
}

}  // namespace

using gh::fail;

extern "C" {

int gh_gguf_open(const char* path, gh_gguf** out) {
    GH_REQUIRE(path && out, "gguf_open: null argument");
    *out = nullptr;
    gh_gguf* g = new gh_gguf();
    g->fd = open(path, O_RDONLY);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0 || st.st_size <= 0) {
        close_file(g);
        return fail(GH_EINVAL, "gguf_open: cannot open %s", path);
    }
    g->size = (size_t)st.st_size;
    void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        g->map = nullptr;
        close_file(g);
        return fail(GH_EINVAL, "gguf_open: cannot map %s", path);
    }
    g->map = (const uint8_t*)m;
    Cursor c{g->map, g->size};
    auto bad = [&](const char* what) {
        close_file(g);
        return fail(GH_EINVAL, "gguf_format: %s (%s)", what, path);
    };
    if (c.pod<uint32_t>() != GGUF_MAGIC || !c.ok) return bad("not a GGUF file");
    g->version = c.pod<uint32_t>();
    if (!c.ok || g->version < 2 || g->version > 3) return bad("unsupported version");
    const uint64_t nt = c.pod<uint64_t>(), nkv = c.pod<uint64_t>();
    if (!c.ok) return bad("truncated header");
    if (nt > 100000 || nkv > 100000) return bad("absurd header counts (tensors/metadata); refusing file");
    for (uint64_t i = 0; i < nkv; ++i) {
        const std::string key = c.str();
        KV v{};
        v.type = c.pod<uint32_t>();
        if (!c.ok) return bad("truncated metadata");
        v.off = c.at;
        if (v.type == KV_STR) {
            c.str();
        } else if (v.type == KV_ARR) {
            v.arr_type = c.pod<uint32_t>();
            v.arr_n = c.pod<uint64_t>();
            if (!c.ok) return bad("truncated metadata array");
            if (v.arr_type == KV_STR) {
                for (uint64_t j = 0; j < v.arr_n && c.ok; ++j) c.str();
            } else {
                const size_t es = kv_scalar_size(v.arr_type);
                if (!es || v.arr_n > (c.n - c.at) / es) return bad("bad metadata array");
                c.skip(v.arr_n * es);
            }
        } else {
            const size_t es = kv_scalar_size(v.type);
            if (!es) return bad("unknown metadata type");
            c.skip(es);
        }
        if (!c.ok) return bad("truncated metadata");
        g->kv[key] = v;
    }
    for (uint64_t i = 0; i < nt; ++i) {
        Tensor t;
        t.name = c.str();
        const uint32_t nd = c.pod<uint32_t>();
        if (!c.ok || nd == 0 || nd > 8) return bad("bad tensor info");
        t.numel = 1;
        for (uint32_t d = 0; d < nd; ++d) {
            const uint64_t v = c.pod<uint64_t>();
            if (v == 0 || v > (1ull << 40) || t.numel > (1ull << 40) / v) return bad("invalid element count");
            t.dims.push_back(v);
            t.numel *= v;
        }
        t.type = c.pod<uint32_t>();
        t.offset = c.pod<uint64_t>();
        if (!c.ok) return bad("truncated tensor info");
        uint64_t bv, bb;
        ggml_block(t.type, bv, bb);
        if (!bb) {
            close_file(g);
            return fail(GH_EUNSUPPORTED, "gguf_format: tensor '%s' uses unsupported GGML type %u", t.name.c_str(),
                        t.type);
        }
        if (t.dims[0] % bv) return bad("row length not a whole number of blocks");
        t.nbytes = t.numel / bv * bb;
        g->by_name[t.name] = g->tensors.size();
        g->tensors.push_back(std::move(t));
    }
    uint64_t align = 32;
    auto ai = g->kv.find("general.alignment");
    if (ai != g->kv.end() && ai->second.type == KV_U32) {
        uint32_t a;
        memcpy(&a, g->map + ai->second.off, 4);
        if (a == 0 || (a & (a - 1))) return bad("general.alignment is not a power of two");
        align = a;
    }
    g->data_start = (c.at + align - 1) / align * align;
    if (g->data_start > g->size) return bad("bad data section");
    for (const Tensor& t : g->tensors)
        if (t.offset > g->size - g->data_start || t.nbytes > g->size - g->data_start - t.offset) {
            const std::string name = t.name;  // t lives in g
            close_file(g);
            return fail(GH_EINVAL, "gguf_format: tensor overruns file: %s", name.c_str());
        }
    *out = g;
    return GH_OK;
}

int gh_gguf_close(gh_gguf* g) {
    if (g) close_file(g);
    return GH_OK;
}

int64_t gh_gguf_tensor_count(const gh_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }

int gh_gguf_tensor_info(const gh_gguf* g, int64_t i, const char** name, uint32_t* ggml_type, int* ndims,
                        uint64_t* dims8, uint64_t* nbytes) {
    GH_REQUIRE(g && i >= 0 && i < (int64_t)g->tensors.size(), "gguf_tensor_info: bad index");
    const Tensor& t = g->tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    if (ggml_type) *ggml_type = t.type;
    if (ndims) *ndims = (int)t.dims.size();
    if (dims8)
        for (int d = 0; d < 8; ++d) dims8[d] = d < (int)t.dims.size() ? t.dims[(size_t)d] : 0;
    if (nbytes) *nbytes = t.nbytes;
    return GH_OK;
}

int64_t gh_gguf_find_tensor(const gh_gguf* g, const char* name) {
    if (!g || !name) return -1;
    const Tensor* t = find(g, name);
    return t ? (int64_t)(t - g->tensors.data()) : -1;
}

int gh_gguf_get_u64(const gh_gguf* g, const char* key, uint64_t* out) {
    GH_REQUIRE(g && key && out, "gguf_get_u64: null argument");
    auto it = g->kv.find(key);
    GH_REQUIRE(it != g->kv.end(), "gguf: no metadata key %s", key);
    const KV& v = it->second;
    const uint8_t* p = g->map + v.off;
    switch (v.type) {
        case KV_U8: case KV_BOOL: *out = p[0]; break;
        case KV_U16: { uint16_t x; memcpy(&x, p, 2); *out = x; break; }
        case KV_U32: { uint32_t x; memcpy(&x, p, 4); *out = x; break; }
        case KV_I32: { int32_t x; memcpy(&x, p, 4); GH_REQUIRE(x >= 0, "gguf: %s is negative", key); *out = (uint64_t)x; break; }
        case KV_U64: memcpy(out, p, 8); break;
        case KV_I64: { int64_t x; memcpy(&x, p, 8); GH_REQUIRE(x >= 0, "gguf: %s is negative", key); *out = (uint64_t)x; break; }
        default: return fail(GH_EINVAL, "gguf: %s is not an unsigned integer (type %u)", key, v.type);
    }
    return GH_OK;
}

int gh_gguf_get_f32(const gh_gguf* g, const char* key, float* out) {
    GH_REQUIRE(g && key && out, "gguf_get_f32: null argument");
    auto it = g->kv.find(key);
    GH_REQUIRE(it != g->kv.end(), "gguf: no metadata key %s", key);
    const KV& v = it->second;
    if (v.type == KV_F32) {
        memcpy(out, g->map + v.off, 4);
    } else if (v.type == KV_F64) {
        double x;
        memcpy(&x, g->map + v.off, 8);
        *out = (float)x;
    } else {
        return fail(GH_EINVAL, "gguf: %s is not a float (type %u)", key, v.type);
    }
    return GH_OK;
}

int gh_gguf_get_str(const gh_gguf* g, const char* key, char* buf, size_t cap) {
    GH_REQUIRE(g && key && buf && cap > 0, "gguf_get_str: bad arguments");
    auto it = g->kv.find(key);
    GH_REQUIRE(it != g->kv.end(), "gguf: no metadata key %s", key);
    GH_REQUIRE(it->second.type == KV_STR, "gguf: %s is not a string", key);
    uint64_t len;
    memcpy(&len, g->map + it->second.off, 8);
    GH_REQUIRE(len < cap, "gguf: %s needs %llu bytes", key, (unsigned long long)(len + 1));
    memcpy(buf, g->map + it->second.off + 8, (size_t)len);
    buf[len] = 0;
    return GH_OK;
}

int gh_gguf_read_packed(const gh_gguf* g, const char* name, int kind, void* dst, int dst_dev, size_t cap) {
    GH_REQUIRE(g && name && dst, "gguf_read_packed: null argument");
    GH_REQUIRE(kind >= 0 && kind <= 3, "gguf_read_packed: kind %d (0 Q4_0, 1 Q4_1, 2 Q8_0, 3 Q4_K)", kind);
    const Tensor* t = find(g, name);
    GH_REQUIRE(t != nullptr, "gguf_format: tensor not found: %s", name);
    uint64_t bv, bb;
    ggml_block(kind_type(kind), bv, bb);
    GH_REQUIRE(t->dims[0] % bv == 0, "gguf_read_packed: %s rows of %llu values are not whole blocks", name,
               (unsigned long long)t->dims[0]);
    const size_t need = (size_t)(t->numel / bv * bb);
    GH_REQUIRE(cap >= need, "gguf_read_packed: %s needs %zu bytes, buffer has %zu", name, need, cap);
    if (t->type == kind_type(kind))  // packed blocks verbatim
        return copy_out(dst, dst_dev, g->map + g->data_start + t->offset, need);
    std::vector<float> f;
    int rc = decode_f32(g, *t, f);
    if (rc) return rc;
    std::vector<uint8_t> q(need);
    rc = gh_quantize_host(kind, f.data(), q.data(), (int64_t)t->numel);
    if (rc) return rc;
    return copy_out(dst, dst_dev, q.data(), need);
}

int gh_gguf_read_f32(const gh_gguf* g, const char* name, float* dst, int dst_dev, size_t cap_elems) {
    GH_REQUIRE(g && name && dst, "gguf_read_f32: null argument");
    const Tensor* t = find(g, name);
    GH_REQUIRE(t != nullptr, "gguf_format: tensor not found: %s", name);
    GH_REQUIRE(cap_elems >= t->numel, "gguf_read_f32: %s has %llu values", name, (unsigned long long)t->numel);
    std::vector<float> f;
    const int rc = decode_f32(g, *t, f);
    if (rc) return rc;
    return copy_out(dst, dst_dev, f.data(), f.size() * 4);
}

int gh_gguf_read_f16(const gh_gguf* g, const char* name, uint16_t* dst, int dst_dev, size_t cap_elems) {
    GH_REQUIRE(g && name && dst, "gguf_read_f16: null argument");
    const Tensor* t = find(g, name);
    GH_REQUIRE(t != nullptr, "gguf_format: tensor not found: %s", name);
    GH_REQUIRE(cap_elems >= t->numel, "gguf_read_f16: %s has %llu values", name, (unsigned long long)t->numel);
    if (t->type == GT_F16) return copy_out(dst, dst_dev, g->map + g->data_start + t->offset, (size_t)t->numel * 2);
    std::vector<float> f;
    const int rc = decode_f32(g, *t, f);
    if (rc) return rc;
    std::vector<uint16_t> h(f.size());
    for (size_t i = 0; i < f.size(); ++i) h[i] = f32_to_half_bits(f[i]);
    return copy_out(dst, dst_dev, h.data(), h.size() * 2);
}

int gh_gguf_write(const char* path, int n_tensors, const char* const* names, const uint32_t* types,
                  const int* ndims, const uint64_t* dims8, const void* const* data, int n_kv,
                  const char* const* keys, const uint32_t* kv_types, const void* const* kv_values) {
    GH_REQUIRE(path && n_tensors >= 0 && n_kv >= 0, "gguf_write: bad arguments");
    std::vector<uint8_t> head;
    auto put = [&](const void* p, size_t n) { head.insert(head.end(), (const uint8_t*)p, (const uint8_t*)p + n); };
    auto put_str = [&](const char* s) {
        const uint64_t n = strlen(s);
        put(&n, 8);
        put(s, (size_t)n);
    };
    const uint32_t magic = GGUF_MAGIC, version = 3;
    const uint64_t nt = (uint64_t)n_tensors, nk = (uint64_t)n_kv;
    put(&magic, 4);
    put(&version, 4);
    put(&nt, 8);
    put(&nk, 8);
    uint64_t align = 32;
    for (int i = 0; i < n_kv; ++i) {
        GH_REQUIRE(keys[i] && kv_values[i], "gguf_write: metadata %d is null", i);
        put_str(keys[i]);
        put(&kv_types[i], 4);
        if (kv_types[i] == KV_STR) {
            put_str((const char*)kv_values[i]);
        } else {
            const size_t es = kv_scalar_size(kv_types[i]);
            GH_REQUIRE(es > 0, "gguf_write: metadata %s has unsupported type %u", keys[i], kv_types[i]);
            put(kv_values[i], es);
            if (!strcmp(keys[i], "general.alignment") && kv_types[i] == KV_U32) {
                uint32_t a;
                memcpy(&a, kv_values[i], 4);
                GH_REQUIRE(a && !(a & (a - 1)), "gguf_write: alignment %u", a);
                align = a;
            }
        }
    }
    std::vector<uint64_t> offs((size_t)n_tensors), sizes((size_t)n_tensors);
    uint64_t off = 0;
    for (int i = 0; i < n_tensors; ++i) {
        uint64_t bv, bb, numel = 1;
        ggml_block(types[i], bv, bb);
        GH_REQUIRE(bb > 0, "gguf_write: tensor %s has unsupported GGML type %u", names[i], types[i]);
        GH_REQUIRE(ndims[i] >= 1 && ndims[i] <= 8, "gguf_write: tensor %s has %d dimensions", names[i], ndims[i]);
        for (int d = 0; d < ndims[i]; ++d) numel *= dims8[8 * i + d];
        GH_REQUIRE(numel > 0 && dims8[8 * i] % bv == 0, "gguf_write: tensor %s is not whole blocks", names[i]);
        sizes[(size_t)i] = numel / bv * bb;
        offs[(size_t)i] = off;
        off = (off + sizes[(size_t)i] + align - 1) / align * align;
        put_str(names[i]);
        const uint32_t nd = (uint32_t)ndims[i];
        put(&nd, 4);
        put(dims8 + 8 * i, 8 * (size_t)nd);
        put(&types[i], 4);
        put(&offs[(size_t)i], 8);
    }
    FILE* f = fopen(path, "wb");
    GH_REQUIRE(f != nullptr, "gguf_write: cannot create %s", path);
    const size_t pad_head = (size_t)((head.size() + align - 1) / align * align - head.size());
    head.insert(head.end(), pad_head, 0);
    bool ok = fwrite(head.data(), 1, head.size(), f) == head.size();
    uint64_t at = 0;
    for (int i = 0; i < n_tensors && ok; ++i) {
        if (offs[(size_t)i] > at) {
            const std::vector<uint8_t> z((size_t)(offs[(size_t)i] - at), 0);
            ok = fwrite(z.data(), 1, z.size(), f) == z.size();
        }
        ok = ok && fwrite(data[i], 1, (size_t)sizes[(size_t)i], f) == sizes[(size_t)i];
        at = offs[(size_t)i] + sizes[(size_t)i];
    }
    ok = (fclose(f) == 0) && ok;
    GH_REQUIRE(ok, "gguf_write: short write to %s", path);
    return GH_OK;
}


// GGUFReader::model_config (format/gguf_codec.cpp:1083-1180) for the Granite hybrid this backend
// runs, from the native ghassan.* keys the reference's exporter writes (gguf_codec.cpp:1749-1824):
// the gh_granite_create_ex arrays. A key the file lacks takes the ModelConfig default
// (model/model.h), as the reference's get_uint / get_float / get_bool do; features the backend
// does not implement are refused by name. The shared expert width falls back to the routed width
// (model.h:126-129); the attention scale 0 means 1 / sqrt(head_dim) (model.h:103).
int gh_gguf_granite_config(const gh_gguf* g, int qkind, int32_t* cfg, int cfg_cap, float* fcfg, int fcfg_cap,
                           int* ncfg) {
    GH_REQUIRE(g && cfg && fcfg && ncfg && fcfg_cap >= 5, "gguf_granite_config: bad arguments");
    auto has = [&](const char* k) { return g->kv.count(k) != 0; };
    GH_REQUIRE(has("ghassan.block_count"),
               "GGUF has no architecture keys (ghassan.block_count / llama.block_count): not a Ghassan model file");
    auto u = [&](const char* k, uint64_t def) -> int64_t {
        uint64_t v = def;
        if (has(k) && gh_gguf_get_u64(g, k, &v) != GH_OK) v = def;
        return (int64_t)v;
    };
    auto f32 = [&](const char* k, float def) -> float {
        float v = def;
        if (has(k) && gh_gguf_get_f32(g, k, &v) != GH_OK) v = def;
        return v;
    };
    auto b = [&](const char* k, bool def) -> bool {
        auto it = g->kv.find(k);
        if (it == g->kv.end() || it->second.type != KV_BOOL) return def;
        return g->map[it->second.off] != 0;
    };
    const bool hybrid = b("ghassan.hybrid", b("ghassan.granite", false));
    if (!hybrid) return fail(GH_EUNSUPPORTED, "gguf_granite_config: not a Granite hybrid file (ghassan.hybrid)");
    // defaults of ModelConfig (model/model.h:14-48, 100-113) for keys the file lacks
    const int64_t V = u("ghassan.vocab_size", 16000), d = u("ghassan.embedding_length", 768),
                  L = u("ghassan.block_count", 26);
    const int64_t H = u("ghassan.attention.head_count", 12), KV = u("ghassan.attention.head_count_kv", 4);
    GH_REQUIRE(V > 0 && d > 0 && L > 0 && L <= 1024 && H > 0 && KV > 0, "gguf_granite_config: bad model dimensions");
    GH_REQUIRE(cfg_cap >= 18 + L, "gguf_granite_config: %lld layers need %lld ints", (long long)L,
               (long long)(18 + L));
    const int64_t hd_o = u("ghassan.attention.head_dim", 0), hd = hd_o > 0 ? hd_o : d / H;
    // the parts of ModelConfig this backend does not implement
    const struct {
        bool bad;
        const char* what;
    } refuse[] = {
        {!b("ghassan.use_moe", false), "a dense FFN (ghassan.use_moe false)"},
        {!b("ghassan.moe.shared_expert", true), "MoE without the shared expert"},
        {u("ghassan.mamba.n_groups", 1) != 1, "mamba.n_groups != 1"},
        {b("ghassan.use_qk_norm", false), "use_qk_norm"},
        {b("ghassan.use_qkv_bias", false), "use_qkv_bias"},
        {b("ghassan.mamba.proj_bias", false), "mamba.proj_bias"},
        {!b("ghassan.mamba.conv_bias", true), "a Mamba conv without bias"},
        {u("ghassan.position_embedding", 0) != 1, "positional embeddings (the Granite hybrid is NoPE: position_embedding 1)"},
        {u("ghassan.sliding_window", 0) != 0, "a sliding window"},
    };
    for (const auto& r : refuse)
        if (r.bad) return fail(GH_EUNSUPPORTED, "gguf_granite_config: %s is not supported", r.what);
    // model.cpp:407-420 requires one kind per layer for the hybrid: the list is mandatory here
    GH_REQUIRE(has("ghassan.layer_types"), "GGUF has no ghassan.layer_types: a Granite hybrid needs one kind per layer");
    std::vector<int32_t> lt;
    {
        char buf[8192];
        const int rc = gh_gguf_get_str(g, "ghassan.layer_types", buf, sizeof buf);
        if (rc != GH_OK) return rc;
        // comma separated "0" (mamba) / "1" (attention); each item is read by its first character
        for (const char* p = buf; *p;) {
            GH_REQUIRE(*p == '0' || *p == '1', "GGUF ghassan.layer_types: expected '0' or '1', got '%c'", *p);
            lt.push_back(*p == '1');
            const char* comma = strchr(p, ',');
            if (!comma) break;
            p = comma + 1;
        }
        GH_REQUIRE(lt.size() == (size_t)L, "GGUF ghassan.layer_types: length does not match num_layers");
    }
    const int64_t ffe = u("ghassan.moe.expert_feed_forward_length", 768), sh = u("ghassan.moe.shared_intermediate_size", 0);
    const int32_t v[16] = {(int32_t)V, (int32_t)d, (int32_t)L, (int32_t)H, (int32_t)KV, (int32_t)hd,
                           (int32_t)ffe,
                           (int32_t)u("ghassan.moe.expert_count", 8), (int32_t)u("ghassan.moe.experts_used_count", 2),
                           (int32_t)(sh > 0 ? sh : ffe),
                           (int32_t)(u("ghassan.mamba.expand", 2) * d), (int32_t)u("ghassan.mamba.n_heads", 48),
                           (int32_t)u("ghassan.mamba.d_head", 64), (int32_t)u("ghassan.mamba.d_state", 128),
                           (int32_t)u("ghassan.mamba.d_conv", 4), (int32_t)qkind};
    memcpy(cfg, v, sizeof v);
    for (int64_t l = 0; l < L; ++l) cfg[16 + l] = lt[(size_t)l];
    cfg[16 + L] = b("ghassan.tie_word_embeddings", true) ? 1 : 0;
    cfg[17 + L] = b("ghassan.moe.aux_free", false) ? 1 : 0;
    const float am = f32("ghassan.attention_multiplier", 0.0f);  // 0: 1 / sqrt(head_dim)
    fcfg[0] = f32("ghassan.attention.layer_norm_rms_epsilon", 1e-5f);
    fcfg[1] = am != 0.0f ? am : 1.0f / sqrtf((float)hd);
    fcfg[2] = f32("ghassan.embedding_multiplier", 1.0f);
    fcfg[3] = f32("ghassan.residual_multiplier", 1.0f);
    fcfg[4] = f32("ghassan.logits_scaling", 1.0f);
    *ncfg = (int)(18 + L);
    return GH_OK;
}

}  // extern "C"
