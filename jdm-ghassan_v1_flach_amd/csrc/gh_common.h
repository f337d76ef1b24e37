// Shared definitions of the MI355X (gfx950) backend: status handling, the
// stream the backend launches on, number formats and the packed weight
// blocks. Device code is written for wave64 CDNA4 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <string>

#include "../../include/ghassan_hip.h"

namespace gh {

// ------------------------------------------------------------------ status
// The C ABI returns an int status and keeps the message of the last failure
// per host thread (core/common.h:22-31 throws gai::Error; a C caller cannot
// catch that, so the C++ shim on the caller's side turns status != 0 back
// into an exception).
void set_error(int code, const std::string& msg);
int  fail(int code, const char* fmt, ...);

#define GH_REQUIRE(cond, ...)                                         \
    do {                                                              \
        if (!(cond)) return ::gh::fail(GH_EINVAL, __VA_ARGS__);       \
    } while (0)

#define GH_HIP(call)                                                                   \
    do {                                                                               \
        hipError_t e_ = (call);                                                        \
        if (e_ != hipSuccess)                                                          \
            return ::gh::fail(GH_EHIP, "%s failed: %s (%s:%d)", #call,                 \
                              hipGetErrorString(e_), __FILE__, __LINE__);              \
    } while (0)

// Checks the launch that was just issued (a bad configuration surfaces here;
// asynchronous faults surface at the next synchronising call).
#define GH_LAUNCHED(name)                                                              \
    do {                                                                               \
        hipError_t e_ = hipGetLastError();                                             \
        if (e_ != hipSuccess)                                                          \
            return ::gh::fail(GH_EHIP, "launch of %s failed: %s", name,                \
                              hipGetErrorString(e_));                                  \
    } while (0)

// The stream every entry point launches on (settable, default: the null
// stream, matching the reference's implicit stream-0 ordering).
hipStream_t stream();

// Grow-only device workspace owned by the backend (like the reference's
// free_workspace()-managed buffers, cuda/kernels.cu:31-70). `slot` keeps
// buffers that are live at the same time apart.
void* workspace(int slot, size_t bytes);
void  free_workspaces();

// Device count of compute units (for grid sizing).
int num_cus();

// ----------------------------------------------------------- block formats
// kind: 0=Q4_0 (32 vals, 18 B), 1=Q4_1 (32, 20), 2=Q8_0 (32, 34),
//       3=Q4_K (256, 144). Same numbering as core/quant.h:13-18 plus Q4_K.
__host__ __device__ constexpr int block_values(int kind) { return kind == 3 ? 256 : 32; }
__host__ __device__ constexpr int block_bytes(int kind) {
    return kind == 0 ? 18 : kind == 1 ? 20 : kind == 2 ? 34 : kind == 3 ? 144 : 0;
}
inline bool valid_kind(int kind) { return kind >= 0 && kind <= 3; }
inline size_t row_bytes(int kind, int K) { return (size_t)(K / block_values(kind)) * block_bytes(kind); }

// ------------------------------------------------------------ conversions
// fp16 <-> fp32 with the exact rounding of core/dtype.h:61-111 (RNE, NaN
// keeps sign and a quiet bit), usable on host and device.
__host__ __device__ inline uint16_t f32_to_f16(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t eb = (x >> 23) & 0xFFu;
    uint32_t mant = x & 0x7FFFFFu;
    if (eb == 0xFFu) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    const int e = (int)eb - 112;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        const uint32_t sh = (uint32_t)(14 - e);
        uint32_t q = mant >> sh;
        const uint32_t rem = mant & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t low = mant & 0x1FFFu;
    if (low > 0x1000u || (low == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)h;
}

__host__ __device__ inline float f16_to_f32(uint16_t h) {
    // Every finite fp16 (normal or subnormal) is exactly representable in
    // fp32; the hardware conversion is exact and maps Inf/NaN like the
    // reference (payload shifted into the fp32 mantissa).
#if defined(__HIP_DEVICE_COMPILE__)
    return (float)__builtin_bit_cast(_Float16, h);
#else
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, out;
    if (e == 0) {
        if (m == 0) out = sign;
        else {
            int s = -1;
            do { m <<= 1; ++s; } while (!(m & 0x400u));
            out = sign | ((uint32_t)(112 - s) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 0x1F) out = sign | 0x7F800000u | (m << 13);
    else out = sign | ((e + 112u) << 23) | (m << 13);
    return __builtin_bit_cast(float, out);
#endif
}

__host__ __device__ inline float bf16_to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
    const uint32_t x = __builtin_bit_cast(uint32_t, f);
    if (((x >> 23) & 0xFF) == 0xFF) return (uint16_t)(x >> 16);
    return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

// ------------------------------------------------------------ wave helpers
__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__host__ __device__ inline int cdiv(int a, int b) { return (a + b - 1) / b; }

}  // namespace gh

namespace gh {
// Workspace slot map (grow-only device buffers owned by the backend).
enum WsSlot {
    WS_ARGMAX = 0,
    WS_ATTN_O = 1,
    WS_ATTN_ML = 2,
    WS_MOE_ROUTE = 3,   // probs/idx/w when the caller passes none
    WS_MOE_PERM = 4,    // grouped slot ids, offsets, counters
    WS_MOE_ACT = 5,     // gate/up activations of the grouped experts
    WS_MOE_OUT = 6,     // per-slot expert outputs before the combine
    WS_MOE_SHARED = 7,  // shared-expert activation
    WS_MAMBA_PROJ = 8,
    WS_MAMBA_XBC = 9,
    WS_MAMBA_Y = 10,
    WS_MAMBA_CHUNK = 11,
    WS_MAMBA_XF = 12,
    WS_GEMM_X = 13,
    WS_ATTN_KV16 = 14,  // prefill: K and V^T as fp16, per kv head
    WS_MOE_X16 = 15,    // prefill: fp16 copy of the MoE input rows
    WS_QUANT0 = 16,     // 16 quant_materialize slots: 16..31
    WS_MOE_XG = 32,     // gathered rows for the grouped prefill GEMM
    WS_MOE_H = 33,
    WS_MOE_TERMS = 34,  // router group terms (large routers, few tokens)
};
}  // namespace gh
