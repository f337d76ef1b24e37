// Small ops of the forward path: conversions, embedding gather, residual
// adds, RMSNorm, SwiGLU and greedy argmax (core/math_cpu.cpp:173-316,
// 522-529, 710-723; cuda/kernels.cu:451-461, 727-895, 1076, 1310-1334).
#include "gh_common.h"

namespace gh {

static dim3 grid1d(int64_t n, int per_thread = 1) {
    int64_t t = (n + per_thread - 1) / per_thread;
    int64_t b = (t + 255) / 256;
    if (b > 65535LL * 8) b = 65535LL * 8;
    return dim3((unsigned)(b < 1 ? 1 : b));
}

#define GRID_STRIDE(i, n) \
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (n); i += (int64_t)gridDim.x * blockDim.x)

__global__ void k_f32_to_f16(const float* __restrict__ s, uint16_t* __restrict__ d, int64_t n) {
    GRID_STRIDE(i, n) d[i] = f32_to_f16(s[i]);
}
__global__ void k_f16_to_f32(const uint16_t* __restrict__ s, float* __restrict__ d, int64_t n) {
    GRID_STRIDE(i, n) d[i] = f16_to_f32(s[i]);
}
__global__ void k_add(const float* a, const float* b, float* o, int64_t n) { GRID_STRIDE(i, n) o[i] = a[i] + b[i]; }
__global__ void k_scale(float* a, float s, int64_t n) { GRID_STRIDE(i, n) a[i] *= s; }
__global__ void k_fill0(float* a, int64_t n) { GRID_STRIDE(i, n) a[i] = 0.f; }
__global__ void k_copy(float* d, const float* s, int64_t n) { GRID_STRIDE(i, n) d[i] = s[i]; }

// Read-only streaming probe: every lane reads 16-byte pieces, four requests in
// flight per lane, grid-strided so that consecutive lanes read consecutive
// pieces; the XOR of everything read leaves one word per block (so nothing is
// elided). The measured time of one pass is the HBM read ceiling that the
// weight-streaming GEMVs are compared with.
__global__ void __launch_bounds__(256) k_stream_read(const uint4* __restrict__ src, int64_t n16,
                                                     uint32_t* __restrict__ sink) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = src[i];
        const uint4 b = src[i + stride];
        const uint4 c = src[i + 2 * stride];
        const uint4 d = src[i + 3 * stride];
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n16; i += stride) {
        const uint4 a = src[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    __shared__ uint32_t red[4];
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

// core/math_cpu.cpp:522-529 (silu(g) * u)
__global__ void k_swiglu(const float* g, const float* u, float* o, int64_t n) {
    GRID_STRIDE(i, n) {
        const float gv = g[i];
        o[i] = gv / (1.0f + expf(-gv)) * u[i];
    }
}

// core/math_cpu.cpp:227-241: out-of-range ids give a zero row.
__global__ void k_embed_half(const int32_t* __restrict__ ids, const uint16_t* __restrict__ tab,
                             float* __restrict__ out, int64_t ntok, int dim, int vocab) {
    const int64_t t = blockIdx.x;
    if (t >= ntok) return;
    const int id = ids[t];
    for (int i = threadIdx.x; i < dim; i += blockDim.x)
        out[t * dim + i] = (id < 0 || id >= vocab) ? 0.f : f16_to_f32(tab[(size_t)id * dim + i]);
}

// core/math_cpu.cpp:299-316: sum of squares in double, inv in double then
// fp32, out = x * inv * w. One block per row.
__global__ void __launch_bounds__(256) k_rmsnorm(const float* __restrict__ x, const float* __restrict__ w,
                                                 float* __restrict__ out, float* __restrict__ rrms, int dim,
                                                 float eps) {
    const int64_t r = blockIdx.x;
    const float* xr = x + r * dim;
    double ss = 0.0;
    for (int i = threadIdx.x; i < dim; i += 256) ss += (double)xr[i] * xr[i];
    __shared__ double red[4];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const double tot = red[0] + red[1] + red[2] + red[3];
    const double invd = 1.0 / sqrt(tot / (double)dim + (double)eps);
    const float inv = isfinite(invd) ? (float)invd : 0.0f;
    if (rrms && threadIdx.x == 0) rrms[r] = inv;
    float* o = out + r * dim;
    for (int i = threadIdx.x; i < dim; i += 256) o[i] = xr[i] * inv * w[i];
}

// core/math_cpu.cpp:710-723: the first finite maximum (strict '>', lowest
// index on ties); if no value is finite, the reference's serial fallback.
// With `step` set, the winner is also appended to ids[*step] (if *step <
// cap) and *step advances: the greedy-decode record of one token.
__global__ void __launch_bounds__(1024) k_argmax(const float* __restrict__ l, int V, int32_t* __restrict__ out,
                                                 int32_t* __restrict__ step, int32_t* __restrict__ ids, int cap) {
    float bv = 0.f;
    int bi = -1;
    for (int i = threadIdx.x; i < V; i += 1024) {
        const float v = l[i];
        if (isfinite(v) && (bi < 0 || v > bv)) { bv = v; bi = i; }
    }
    __shared__ float sv[16];
    __shared__ int si[16];
    {
        // the wave's best as an unsigned key (value in an order-preserving form, then ~index so
        // the lower index wins ties; 0 = none) reduced on the DPP path into lane 63
        const uint32_t u = __builtin_bit_cast(uint32_t, bv == 0.f ? 0.f : bv);  // -0 ties with +0
        uint32_t hi = bi >= 0 ? ((u & 0x80000000u) ? ~u : (u | 0x80000000u)) : 0u;
        uint32_t lo = bi >= 0 ? ~(uint32_t)bi : 0u;
        auto step = [&](uint32_t oh, uint32_t ol) {
            if (oh > hi || (oh == hi && ol > lo)) { hi = oh; lo = ol; }
        };
        step((uint32_t)dpp_i32<0xB1>((int)hi, (int)hi), (uint32_t)dpp_i32<0xB1>((int)lo, (int)lo));
        step((uint32_t)dpp_i32<0x4E>((int)hi, (int)hi), (uint32_t)dpp_i32<0x4E>((int)lo, (int)lo));
        step((uint32_t)dpp_i32<0x124>((int)hi, (int)hi), (uint32_t)dpp_i32<0x124>((int)lo, (int)lo));
        step((uint32_t)dpp_i32<0x128>((int)hi, (int)hi), (uint32_t)dpp_i32<0x128>((int)lo, (int)lo));
        step((uint32_t)dpp_i32<0x142, 0xA>((int)hi, (int)hi), (uint32_t)dpp_i32<0x142, 0xA>((int)lo, (int)lo));
        step((uint32_t)dpp_i32<0x143, 0xC>((int)hi, (int)hi), (uint32_t)dpp_i32<0x143, 0xC>((int)lo, (int)lo));
        const uint32_t bh = (uint32_t)__builtin_amdgcn_readlane((int)hi, 63);
        const uint32_t bl = (uint32_t)__builtin_amdgcn_readlane((int)lo, 63);
        bi = bh ? (int)~bl : -1;
        bv = bh ? ((bh & 0x80000000u) ? __builtin_bit_cast(float, bh & 0x7FFFFFFFu) : __builtin_bit_cast(float, ~bh)) : 0.f;
    }
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w) {
            const float ov = sv[w];
            const int oi = si[w];
            if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
        }
        if (bi < 0) {
            bi = 0;
            for (int i = 1; i < V; ++i) if (l[i] > l[bi]) bi = i;
        }
        *out = bi;
        if (step) {
            const int s = *step;
            if (s < cap) ids[s] = bi;
            *step = s + 1;
        }
    }
}

int launch_f32_to_f16(const float* s, uint16_t* d, int64_t n) {
    hipLaunchKernelGGL(k_f32_to_f16, grid1d(n), dim3(256), 0, stream(), s, d, n);
    GH_LAUNCHED("k_f32_to_f16");
    return GH_OK;
}

int launch_argmax(const float* l, int V, int32_t* out_dev) {
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, stream(), l, V, out_dev, nullptr, nullptr, 0);
    GH_LAUNCHED("k_argmax");
    return GH_OK;
}

int launch_argmax_record(const float* l, int V, int32_t* out_dev, int32_t* step, int32_t* ids, int cap) {
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, stream(), l, V, out_dev, step, ids, cap);
    GH_LAUNCHED("k_argmax");
    return GH_OK;
}

}  // namespace gh

using namespace gh;

extern "C" {

int gh_convert_f32_to_f16(const float* s, uint16_t* d, int64_t n) {
    if (n <= 0) return GH_OK;
    GH_REQUIRE(s && d, "convert_f32_to_f16: null pointer");
    return launch_f32_to_f16(s, d, n);
}
int gh_convert_f16_to_f32(const uint16_t* s, float* d, int64_t n) {
    if (n <= 0) return GH_OK;
    GH_REQUIRE(s && d, "convert_f16_to_f32: null pointer");
    hipLaunchKernelGGL(k_f16_to_f32, grid1d(n), dim3(256), 0, stream(), s, d, n);
    GH_LAUNCHED("k_f16_to_f32");
    return GH_OK;
}
int gh_embedding_forward_half(const int32_t* ids, const uint16_t* table, float* out, int64_t ntok, int dim,
                              int vocab) {
    if (ntok <= 0) return GH_OK;
    GH_REQUIRE(ids && table && out && dim > 0, "embedding_forward_half: bad arguments");
    hipLaunchKernelGGL(k_embed_half, dim3((unsigned)ntok), dim3(256), 0, stream(), ids, table, out, ntok, dim, vocab);
    GH_LAUNCHED("k_embed_half");
    return GH_OK;
}
int gh_add(const float* a, const float* b, float* out, int64_t n) {
    if (n <= 0) return GH_OK;
    GH_REQUIRE(a && b && out, "add: null pointer");
    hipLaunchKernelGGL(k_add, grid1d(n), dim3(256), 0, stream(), a, b, out, n);
    GH_LAUNCHED("k_add");
    return GH_OK;
}
int gh_add_inplace(float* a, const float* b, int64_t n) { return gh_add(a, b, a, n); }
int gh_scale_inplace(float* a, float s, int64_t n) {
    if (n <= 0) return GH_OK;
    GH_REQUIRE(a, "scale_inplace: null pointer");
    hipLaunchKernelGGL(k_scale, grid1d(n), dim3(256), 0, stream(), a, s, n);
    GH_LAUNCHED("k_scale");
    return GH_OK;
}
int gh_zero(float* a, int64_t n) {
    if (n <= 0) return GH_OK;
    GH_REQUIRE(a, "ops::zero on null pointer");
    hipLaunchKernelGGL(k_fill0, grid1d(n), dim3(256), 0, stream(), a, n);
    GH_LAUNCHED("k_fill0");
    return GH_OK;
}
int gh_copy(float* d, const float* s, int64_t n) {
    if (n <= 0) return GH_OK;
    GH_REQUIRE(d && s, "ops::copy on null pointer");
    hipLaunchKernelGGL(k_copy, grid1d(n), dim3(256), 0, stream(), d, s, n);
    GH_LAUNCHED("k_copy");
    return GH_OK;
}
int gh_stream_read(const void* src, int64_t bytes, uint32_t* sink, int blocks) {
    GH_REQUIRE(src && sink && bytes > 0 && bytes % 16 == 0 && blocks > 0 && blocks <= 65536,
               "stream_read: bad arguments (bytes must be a positive multiple of 16, 1 <= blocks <= 65536)");
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)blocks), dim3(256), 0, stream(), (const uint4*)src, bytes / 16,
                       sink);
    GH_LAUNCHED("k_stream_read");
    return GH_OK;
}
int gh_rmsnorm_forward(const float* x, const float* w, float* out, float* rrms, int64_t rows, int dim, float eps) {
    if (rows <= 0) return GH_OK;
    GH_REQUIRE(x && w && out && dim > 0, "rmsnorm_forward: bad arguments");
    hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)rows), dim3(256), 0, stream(), x, w, out, rrms, dim, eps);
    GH_LAUNCHED("k_rmsnorm");
    return GH_OK;
}
int gh_swiglu_forward(const float* g, const float* u, float* out, int64_t n) {
    if (n <= 0) return GH_OK;
    GH_REQUIRE(g && u && out, "swiglu_forward: null pointer");
    hipLaunchKernelGGL(k_swiglu, grid1d(n), dim3(256), 0, stream(), g, u, out, n);
    GH_LAUNCHED("k_swiglu");
    return GH_OK;
}
int gh_argmax_token_dev(const float* logits, int V, int32_t* out_dev) {
    GH_REQUIRE(logits && out_dev && V > 0, "argmax_token: empty vocabulary");
    return launch_argmax(logits, V, out_dev);
}
int gh_argmax_token(const float* logits, int V, int32_t* out_host) {
    GH_REQUIRE(logits && out_host && V > 0, "argmax_token: empty vocabulary");
    int32_t* d = (int32_t*)workspace(0, sizeof(int32_t));
    if (!d) return fail(GH_ENOMEM, "argmax_token: workspace");
    int rc = launch_argmax(logits, V, d);
    if (rc) return rc;
    GH_HIP(hipMemcpyAsync(out_host, d, sizeof(int32_t), hipMemcpyDeviceToHost, stream()));
    GH_HIP(hipStreamSynchronize(stream()));
    return GH_OK;
}

}  // extern "C"
