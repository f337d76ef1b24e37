// The persistent greedy decode loop: the model description it reads (filled
// by the caller-side model in granite.hip) and its launcher.
#pragma once
#include "gh_common.h"

namespace gh {

constexpr int PD_MAX_LAYERS = 16;

// The model's device pointers are global-memory pointers in device code, so the kernel's
// accesses compile to global_* instructions: generic (flat) ones also count against the LDS
// wait counter, and every LDS wait would then wait for all outstanding memory traffic.
#if defined(__HIP_DEVICE_COMPILE__)
#define PD_G __attribute__((address_space(1)))
#else
#define PD_G
#endif

// A host pointer to device memory as the model field type (a cast only in device compilation).
template <class T>
__host__ __device__ inline PD_G T* pd_g(T* p) {
    return (PD_G T*)p;
}

struct PdLayer {
    int type;  // 0 Mamba-2, 1 attention
    const PD_G float* attn_norm;
    const PD_G float* ffn_norm;
    // Mamba-2
    const PD_G uint8_t* in_proj;
    const PD_G float* conv_w;
    const PD_G float* conv_b;
    const PD_G float* dt_bias;
    const PD_G float* a_log;
    const PD_G float* Dp;
    const PD_G float* gnorm_w;
    const PD_G uint8_t* out_proj;
    PD_G float* conv_state;  // [conv_dim][ck-1]
    PD_G float* ssm_state;   // [H][P][N]
    // attention
    const PD_G uint8_t* wq;
    const PD_G uint8_t* wk;
    const PD_G uint8_t* wv;
    const PD_G uint8_t* wo;
    PD_G uint16_t* kc;  // [max_ctx][KV*hd] fp16
    PD_G uint16_t* vc;
    // MoE
    const PD_G float* router;
    const PD_G uint8_t* gate;
    const PD_G uint8_t* up;
    const PD_G uint8_t* down;
    const PD_G uint8_t* sh_gate;
    const PD_G uint8_t* sh_up;
    const PD_G uint8_t* sh_down;
};

// A tagged hand-over vector kept in PD_REP replicas `stride` words apart: a producer writes
// every replica, a consumer reads one (by its block index), so the blocks that all read a
// vector at once spread over PD_REP address ranges instead of one.
constexpr int PD_REP = 1;
struct PdBuf {
    PD_G uint64_t* p;
    int stride;  // words between replicas (even: replicas stay 16-byte aligned)
};

struct PdModel {
    int L, d, V, H, KV, hd, E, ne, K, SH, di, mh, mdh, mds, ck, kind, max_ctx;
    float eps, scale;
    const PD_G uint16_t* emb;       // [V][d] fp16 (tied lm head)
    const PD_G float* final_norm;
    // tagged hand-over buffers: 64-bit words (value bits | epoch << 32), zeroed before a launch
    PdBuf tx;     // residual stream [d]
    PdBuf tproj;  // Mamba in_proj output: z [di] | conv'd xBC [conv_dim] | raw dt [mh]
    PdBuf ty;     // Mamba scan output [di]
    PdBuf tq;     // attention q [H*hd]
    PdBuf tkv;    // the new token's k | v, fp16-rounded [2*KV*hd]
    PdBuf tpart;  // attention partials [H][splits][hd + 2]
    PdBuf tact;   // SwiGLU rows of every expert, then the shared expert [ne*E + SH]
    PdBuf troute; // selected experts (as float) [K] | their weights [K]
    size_t tag_words;  // total words of the tagged buffers (one allocation starting at tx)
    PD_G unsigned long long* keys;  // argmax key per step [max_ctx]
    PD_G int32_t* neg0;             // per step: logit 0 is -inf [max_ctx]
    PD_G uint32_t* done;            // lm-head jobs finished (all steps)
    PD_G int32_t* abort;            // set when a wait runs out: every block leaves
    PD_G int32_t* ctl;              // decode control block (granite.hip CTL_*)
    PD_G int32_t* gen_ids;
    PD_G float* logits;             // [V] of the last step
    PdLayer layers[PD_MAX_LAYERS];
};

constexpr int PD_MAX_SPLITS = 64;   // attention position splits (context <= 64 * PD_POS)
constexpr int PD_POS = 64;          // positions per attention job

// Whether the persistent loop supports this model (shapes, kinds); msg gets the reason.
bool pd_supported(const PdModel& m, int len0, int n_steps, const char** msg);
// Runs n_steps greedy decode steps in one cooperative launch. dev: the PdModel copy in
// device memory; the tagged buffers and counters must be zeroed before the call.
int pd_launch(const PdModel& host, const PdModel* dev, int len0, int step0, int n_steps);

}  // namespace gh
