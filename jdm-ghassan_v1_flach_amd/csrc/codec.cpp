// Host side of the weight formats: the block quantisers (load time, like
// quantization/quantize.cpp:58-341), the seeded generator of core/rng.h and
// the synthetic-parameter recipe used for random-init Granite models.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <string>

#include "../../include/ghassan_hip.h"
#include "gh_common.h"

namespace gh {

// core/rng.h:8-92 (xoshiro256** seeded by splitmix64, Marsaglia polar normal)
class Rng {
public:
    explicit Rng(uint64_t seed) {
        for (int i = 0; i < 4; ++i) {
            seed += 0x9E3779B97F4A7C15ULL;
            uint64_t z = seed;
            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
            z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
            s_[i] = z ^ (z >> 31);
        }
    }
    uint64_t next() {
        const uint64_t r = rotl(s_[1] * 5, 7) * 9, t = s_[1] << 17;
        s_[2] ^= s_[0];
        s_[3] ^= s_[1];
        s_[1] ^= s_[2];
        s_[0] ^= s_[3];
        s_[2] ^= t;
        s_[3] = rotl(s_[3], 45);
        return r;
    }
    float uniform() { return (float)((next() >> 40) * (1.0 / 16777216.0)); }
    uint64_t below(uint64_t n) {
        const uint64_t t = (0u - n) % n;
        uint64_t v;
        do v = next(); while (v < t);
        return v % n;
    }
    float normal(float mean, float sd) {
        if (spare_ok_) {
            spare_ok_ = false;
            return mean + sd * spare_;
        }
        float u, v, q;
        do {
            u = uniform() * 2.0f - 1.0f;
            v = uniform() * 2.0f - 1.0f;
            q = u * u + v * v;
        } while (q >= 1.0f || q == 0.0f);
        const float m = sqrtf(-2.0f * logf(q) / q);
        spare_ = v * m;
        spare_ok_ = true;
        return mean + sd * (u * m);
    }

private:
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t s_[4];
    float spare_ = 0.f;
    bool spare_ok_ = false;
};

static uint64_t fnv1a64(const char* s, size_t n) {
    uint64_t h = 1469598103934665603ULL;
    for (size_t i = 0; i < n; ++i) {
        h ^= (uint8_t)s[i];
        h *= 1099511628211ULL;
    }
    return h;
}

static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }
static inline void put16(uint8_t* p, uint16_t v) { memcpy(p, &v, 2); }

// Q8_0 (quantization/quantize.cpp:58-112): scale = amax/127 as fp16, q =
// clamp(lround(x/scale)), a block with a non-finite value is all zero.
static void q8_0_block(const float* x, int cnt, uint8_t* b) {
    memset(b, 0, 34);
    float amax = 0.f;
    for (int i = 0; i < cnt; ++i) {
        if (!isfinite(x[i])) return;
        amax = std::max(amax, fabsf(x[i]));
    }
    const float scale = amax / 127.0f, inv = scale > 0.f ? 1.0f / scale : 0.f;
    put16(b, f32_to_f16(scale));
    for (int i = 0; i < cnt; ++i) b[2 + i] = (uint8_t)(int8_t)clampi((int)lroundf(x[i] * inv), -127, 127);
}
// Q4_0 (quantization/quantize.cpp:114-156): scale = amax/8, q+8 in [0,15],
// low nibble value j, high nibble value j+16; bad block -> 0x88 nibbles.
static void q4_0_block(const float* x, uint8_t* b) {
    memset(b, 0, 18);
    float amax = 0.f;
    for (int i = 0; i < 32; ++i) {
        if (!isfinite(x[i])) {
            memset(b + 2, 0x88, 16);
            return;
        }
        amax = std::max(amax, fabsf(x[i]));
    }
    const float scale = amax / 8.0f, inv = scale > 0.f ? 1.0f / scale : 0.f;
    put16(b, f32_to_f16(scale));
    for (int j = 0; j < 16; ++j) {
        const int a = clampi((int)lroundf(x[j] * inv), -8, 7) + 8;
        const int c = clampi((int)lroundf(x[j + 16] * inv), -8, 7) + 8;
        b[2 + j] = (uint8_t)((c << 4) | a);
    }
}
// Q4_1 (quantization/quantize.cpp:183-220): scale = (max-min)/15, min as fp16.
static void q4_1_block(const float* x, uint8_t* b) {
    memset(b, 0, 20);
    for (int i = 0; i < 32; ++i)
        if (!isfinite(x[i])) return;
    float mn = x[0], mx = x[0];
    for (int i = 1; i < 32; ++i) {
        mn = std::min(mn, x[i]);
        mx = std::max(mx, x[i]);
    }
    const float scale = (mx - mn) / 15.0f, inv = scale > 0.f ? 1.0f / scale : 0.f;
    put16(b, f32_to_f16(scale));
    put16(b + 2, f32_to_f16(mn));
    for (int i = 0; i < 16; ++i) {
        const int a = clampi((int)lroundf((x[i] - mn) * inv), 0, 15);
        const int c = clampi((int)lroundf((x[i + 16] - mn) * inv), 0, 15);
        b[4 + i] = (uint8_t)((c << 4) | a);
    }
}
// Q4_K (GGML block_q4_K layout; the reference has no K-quants, this
// quantiser is our own): per 32-value sub-block an affine range
// [min(0,lo), hi] over 15 steps; 6-bit scale/min codes against fp16 super
// scales d = max scale/63 and dmin = max min/63; nibbles rounded against
// the decoded (d*sc, dmin*m). A non-finite value zeroes the block.
static void q4_k_block(const float* x, uint8_t* b) {
    memset(b, 0, 144);
    for (int i = 0; i < 256; ++i)
        if (!isfinite(x[i])) return;
    float scl[8], mn[8], maxs = 0.f, maxm = 0.f;
    for (int s = 0; s < 8; ++s) {
        float lo = 0.f, hi = x[32 * s];
        for (int l = 0; l < 32; ++l) {
            lo = std::min(lo, x[32 * s + l]);
            hi = std::max(hi, x[32 * s + l]);
        }
        scl[s] = (hi - lo) / 15.0f;
        mn[s] = -lo;
        maxs = std::max(maxs, scl[s]);
        maxm = std::max(maxm, mn[s]);
    }
    const uint16_t hd = f32_to_f16(maxs / 63.0f), hm = f32_to_f16(maxm / 63.0f);
    put16(b, hd);
    put16(b + 2, hm);
    const float d = f16_to_f32(hd), dmin = f16_to_f32(hm);
    int sc[8], m[8];
    for (int s = 0; s < 8; ++s) {
        sc[s] = d > 0.f ? clampi((int)lroundf(scl[s] / d), 0, 63) : 0;
        m[s] = dmin > 0.f ? clampi((int)lroundf(mn[s] / dmin), 0, 63) : 0;
    }
    uint8_t* S = b + 4;
    for (int s = 0; s < 4; ++s) {
        S[s] = (uint8_t)(sc[s] | ((sc[s + 4] >> 4) << 6));
        S[s + 4] = (uint8_t)(m[s] | ((m[s + 4] >> 4) << 6));
        S[s + 8] = (uint8_t)((sc[s + 4] & 0xF) | ((m[s + 4] & 0xF) << 4));
    }
    uint8_t* qs = b + 16;
    for (int s = 0; s < 8; ++s) {
        const float d1 = d * (float)sc[s], m1 = dmin * (float)m[s];
        for (int l = 0; l < 32; ++l) {
            const int q = d1 > 0.f ? clampi((int)lroundf((x[32 * s + l] + m1) / d1), 0, 15) : 0;
            qs[32 * (s >> 1) + l] |= (uint8_t)((s & 1) ? (q << 4) : q);
        }
    }
}

}  // namespace gh

using namespace gh;

extern "C" {

int gh_quantize_host(int kind, const float* src, void* dst, int64_t n) {
    GH_REQUIRE(src && dst && n >= 0, "quantize: bad arguments");
    uint8_t* o = (uint8_t*)dst;
    if (kind == GH_Q8_0) {
        const int64_t full = n / 32;
        for (int64_t i = 0; i < full; ++i) q8_0_block(src + i * 32, 32, o + i * 34);
        if (n % 32) q8_0_block(src + full * 32, (int)(n % 32), o + full * 34);
        return GH_OK;
    }
    GH_REQUIRE(kind >= 0 && kind <= 3, "quantize: unknown kind %d", kind);
    const int bv = block_values(kind), bb = block_bytes(kind);
    GH_REQUIRE(n % bv == 0, "quantize: n=%lld is not a multiple of the %d-value block", (long long)n, bv);
    for (int64_t i = 0; i < n / bv; ++i) {
        if (kind == GH_Q4_0) q4_0_block(src + i * bv, o + i * bb);
        else if (kind == GH_Q4_1) q4_1_block(src + i * bv, o + i * bb);
        else q4_k_block(src + i * bv, o + i * bb);
    }
    return GH_OK;
}

int gh_rng_normal_host(uint64_t seed, float mean, float sd, float* out, int64_t n) {
    GH_REQUIRE(out || n == 0, "rng: null output");
    Rng r(seed);
    for (int64_t i = 0; i < n; ++i) out[i] = r.normal(mean, sd);
    return GH_OK;
}
int gh_rng_uniform_host(uint64_t seed, float lo, float hi, float* out, int64_t n) {
    GH_REQUIRE(out || n == 0, "rng: null output");
    Rng r(seed);
    for (int64_t i = 0; i < n; ++i) out[i] = lo + (hi - lo) * r.uniform();
    return GH_OK;
}
int gh_rng_below_host(uint64_t seed, uint64_t bound, int32_t* out, int64_t n) {
    GH_REQUIRE((out || n == 0) && bound > 0, "rng: bad arguments");
    Rng r(seed);
    for (int64_t i = 0; i < n; ++i) out[i] = (int32_t)r.below(bound);
    return GH_OK;
}

int gh_synth_param_f32(const char* name, uint64_t seed, float* out, int64_t n) {
    GH_REQUIRE(name && (out || n == 0), "synth_param: bad arguments");
    const std::string s(name);
    auto ends = [&](const char* suf) {
        const size_t l = strlen(suf);
        return s.size() >= l && s.compare(s.size() - l, l, suf) == 0;
    };
    if (ends("norm") || ends("norm.weight") || ends("conv1d.bias") || ends("mamba.D") || ends("dt_bias")) {
        for (int64_t i = 0; i < n; ++i) out[i] = 1.0f;
        return GH_OK;
    }
    if (ends("moe_bias")) {  // model/model.cpp:179-191: the aux-free router bias starts at zero
        for (int64_t i = 0; i < n; ++i) out[i] = 0.0f;
        return GH_OK;
    }
    if (ends("A_log")) {  // model/model.cpp:1597-1600
        for (int64_t i = 0; i < n; ++i) out[i] = logf((float)(i + 1));
        return GH_OK;
    }
    return gh_rng_normal_host(seed ^ fnv1a64(name, s.size()), 0.0f, 0.02f, out, n);
}

}  // extern "C"
