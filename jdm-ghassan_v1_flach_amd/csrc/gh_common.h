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
// Changes whenever a workspace buffer is replaced or freed: work captured into a graph
// holds the buffer addresses of its capture and is stale once this moves on.
uint64_t workspace_generation();

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
// Cross-lane moves on the DPP path (no LDS round trip): quad_perm 0xB1 /
// 0x4E = lane xor 1 / 2, row_ror 4 / 8 rotate inside a row of 16 lanes,
// row_shl 4 / 8 read lane + 4 / + 8 of the row, row_bcast 15 / 31 pass a
// row's last lane to the next row(s) selected by the row mask. A lane without
// a source (or in an unselected row) gets `old`.
template <int CTRL, int RM = 0xF>
__device__ __forceinline__ int dpp_i32(int v, int old) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, RM, 0xF, false);
}
template <int CTRL, int RM = 0xF>
__device__ __forceinline__ float dpp_f32(float v, float old = 0.f) {
    return __builtin_bit_cast(float, dpp_i32<CTRL, RM>(__builtin_bit_cast(int, v), __builtin_bit_cast(int, old)));
}
template <int CTRL, int RM = 0xF>
__device__ __forceinline__ double dpp_f64(double v) {  // old = 0
    typedef int i2 __attribute__((ext_vector_type(2)));
    const i2 p = __builtin_bit_cast(i2, v);
    i2 r;
    r.x = dpp_i32<CTRL, RM>(p.x, 0);
    r.y = dpp_i32<CTRL, RM>(p.y, 0);
    return __builtin_bit_cast(double, r);
}
// Sum over a whole wave (every lane active): the total ends in lane 63.
template <typename T>
__device__ __forceinline__ T wave_total63(T v) {
    if constexpr (sizeof(T) == 8) {
        v += dpp_f64<0xB1>(v);
        v += dpp_f64<0x4E>(v);
        v += dpp_f64<0x124>(v);
        v += dpp_f64<0x128>(v);       // every lane: its row of 16
        v += dpp_f64<0x142, 0xA>(v);  // rows 1, 3 += rows 0, 2
        v += dpp_f64<0x143, 0xC>(v);  // rows 2, 3 += lane 31 (rows 0 + 1)
    } else {
        v += dpp_f32<0xB1>(v);
        v += dpp_f32<0x4E>(v);
        v += dpp_f32<0x124>(v);
        v += dpp_f32<0x128>(v);
        v += dpp_f32<0x142, 0xA>(v);
        v += dpp_f32<0x143, 0xC>(v);
    }
    return v;
}
__device__ __forceinline__ float lane63(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ double lane63(double v) {
    typedef int i2 __attribute__((ext_vector_type(2)));
    const i2 p = __builtin_bit_cast(i2, v);
    i2 r;
    r.x = __builtin_amdgcn_readlane(p.x, 63);
    r.y = __builtin_amdgcn_readlane(p.y, 63);
    return __builtin_bit_cast(double, r);
}
// Sum / max over a whole wave (every lane active); every lane gets the result.
__device__ inline float wave_sum(float v) { return lane63(wave_total63(v)); }
__device__ inline double wave_sum(double v) { return lane63(wave_total63(v)); }
// Sum over groups of lpr consecutive lanes (lpr a power of two <= 64); every
// lane of a group gets its total. Inside a row by mirrors (row_mirror: lane i
// <-> 15 - i, row_half_mirror: i <-> 7 - i, each lane then holds a pair) and
// the two quad xors; across rows by lane permutes.
__device__ __forceinline__ float group_sum(float v, int lpr) {
    if (lpr >= 16) v += dpp_f32<0x140>(v);
    if (lpr >= 8) v += dpp_f32<0x141>(v);
    if (lpr >= 4) v += dpp_f32<0x4E>(v);
    if (lpr >= 2) v += dpp_f32<0xB1>(v);
    if (lpr >= 32) v += __shfl_xor(v, 16, 64);
    if (lpr >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}
__device__ inline float wave_max(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v, v));
    v = fmaxf(v, dpp_f32<0x4E>(v, v));
    v = fmaxf(v, dpp_f32<0x124>(v, v));
    v = fmaxf(v, dpp_f32<0x128>(v, v));
    v = fmaxf(v, dpp_f32<0x142, 0xA>(v, v));
    v = fmaxf(v, dpp_f32<0x143, 0xC>(v, v));
    return lane63(v);
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
    WS_MOE_TERMS = 34,  // router logits (large routers)
    WS_GEMM_PART = 35,  // split-K partial tiles of the small-M prefill GEMM
    WS_GEMM_ACC = 36,   // product before an accumulating add (paths without an in-place sum)
    WS_HEAD_CTL = 37,   // argmax key / counter block of a standalone lm-head + greedy call
    WS_TOPK = 38,       // top-K survivors of each 4096-logit chunk
    WS_PEN_HIST = 39,   // device copy of the penalty history
    WS_GEMM_W16 = 40,   // large-M prefill: the weights decoded to bf16 for the library GEMM
    WS_BLASLT = 41,     // hipBLASLt workspace
    WS_MAMBA_XN = 42,   // prefill: the RMS-normalised Mamba input where no GEMM prologue takes the norm
};
}  // namespace gh
