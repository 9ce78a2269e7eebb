// model_kernels.h — argument blocks and launchers of k_model.hip.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "../../include/yuuka_hip.h"

namespace yk {

// Position source: a device int (graph replay / on-device advance) or the
// host value passed at submission.
struct ModelDyn {
    int32_t *pos_dev;
    int32_t pos;
};

struct AttnArgs {
    int kv_heads, heads, head_dim, kv_dim, rows, displacement, block_size, capacity;
    uint32_t fmt;  // 0 F32, 1 F16 KV rows
    int gated;     // 1: query rows hold [q | gate] per head (qwen35)
    float scale;
};

// Verify attention (k_attn.hip): one gated-attention layer's verify rows.
struct AttnVArgs {
    int kv_heads, heads, head_dim, kv_dim, rows, displacement, block_size, capacity;
    uint32_t fmt;  // 0 F32, 1 F16 KV rows
    int gated;     // 1: query rows hold [q | gate] per head (qwen35)
    int rope_dim;  // rotated dimensions per head (pairs i, i + rope_dim/2)
    float scale, eps;
    // requests of one launch (grid z): request j's rows start rq_rows rows
    // after request j-1's, its block table ceil(capacity / block_size)
    // entries after, its {token, position} pair two int32 after
    int nreq, rq_rows;
};

struct GdnArgs {
    int rows, groups, rank, state, conv_dim, inner, kernel;
    float eps, q_scale;
    int coef;  // 1: alpha / beta buffers hold the decay and sigmoid(beta)
    int nreq;  // requests in one launch (column-split kernels): states and rows request-major
};

// tokens null: every row embeds host_token.
hipError_t launch_embedding(const void *table, uint32_t dtype, uint64_t row_bytes, const int32_t *tokens, int vocab,
                            int cols, int rows, float *out, hipStream_t s, int host_token = 0);
hipError_t launch_rmsnorm_rows(const float *src, const float *w, float *dst, int cols, int rows, uint64_t src_stride,
                               uint64_t dst_stride, float eps, hipStream_t s);
// bg_reduce_kernel then rmsnorm_rows_kernel in one launch: out = sum of the
// split partials [splits][rows][cols] (split order) + res; dst = RMSNorm(out) * w.
// cols 1024, 2048 or 4096.
hipError_t launch_reduce_rmsnorm_rows(const float *part, uint64_t sstride, int splits, const float *res, float *out,
                                      const float *w, float *dst, int cols, int rows, uint64_t dst_stride, float eps,
                                      hipStream_t s);
hipError_t launch_rmsnorm_heads(const float *src, const float *w, float *dst, int size, int heads, int stride, int rows,
                                float eps, hipStream_t s);
hipError_t launch_rope(float *data, int heads, int stride, int rot_dim, int rows, uint64_t row_stride, double base,
                       const ModelDyn &dyn, int displacement, hipStream_t s);
hipError_t launch_kv_write(const float *k, const float *v, void *kpool, void *vpool, const int32_t *table, int kv_dim,
                           int rows, int block_size, uint32_t fmt, const ModelDyn &dyn, int displacement,
                           hipStream_t s);
uint64_t attention_scratch_bytes(const AttnArgs &a);
// max_pos_hint: largest row position the call can see (host-known), or -1.
int attn_verify_chunk(uint32_t fmt);
uint64_t attn_verify_scratch_bytes(const AttnVArgs &a);
uint32_t attn_verify_lds_bytes(const AttnVArgs &a);
// The MFMA verify-attention kernel applies (F16 pool, 256-dim heads, 64-dim
// rotation); it serves up to attn_verify_max_rows rows in one launch.
bool attn_verify_mfma(int fmt, int heads, int kv_heads, int head_dim, int rope_dim, int kv_dim);
int attn_verify_max_rows(const AttnVArgs &a);
hipError_t launch_rope_table(float2 *tab, int rows, int rot_dim, double base, const ModelDyn &dyn, int displacement,
                             hipStream_t s, int nreq = 1, int rq_rows = 0);
hipError_t launch_attn_verify(const float *q, const float *k, const float *v, void *kpool, void *vpool,
                              const int32_t *table, const float *q_norm, const float *k_norm, const float2 *rope,
                              float *out, const AttnVArgs &a, void *scratch, const ModelDyn &dyn, int max_pos_hint,
                              hipStream_t s);
uint32_t gdn_verify_lds_bytes(const GdnArgs &g);
hipError_t launch_gdn_verify(const float *conv_state, const float *state, const float *qkv, const float *z,
                             const float *alpha_raw, const float *beta_raw, const float *conv_w, const float *dt,
                             const float *a_log, const float *norm_w, float *out, float *conv_out, const GdnArgs &g,
                             hipStream_t s);
hipError_t launch_gdn_commit(float *conv_state, float *state, const float *qkv, const float *conv,
                             const float *alpha_raw, const float *beta_raw, const float *dt, const float *a_log,
                             const GdnArgs &g, const int32_t *accept_result, hipStream_t s);
uint32_t gdn_verify_cols_lds_bytes(const GdnArgs &g);
hipError_t launch_gdn_verify_cols(const float *conv_state, const float *state, const float *qkv,
                                  const float *alpha_raw, const float *beta_raw, const float *conv_w, const float *dt,
                                  const float *a_log, float *raw_out, float *conv_out, const GdnArgs &g,
                                  hipStream_t s);
// Per-layer buffers of a multi-layer GDN commit (one launch for a run of
// GDN_COMMIT ops that share shape and acceptance result).
struct GdnCommitLayer {
    float *conv_state, *state;
    const float *qkv, *conv, *alpha, *beta, *dt, *a_log;
};
constexpr int kGdnCommitMaxLayers = 48;
struct GdnCommitSet {
    GdnCommitLayer layer[kGdnCommitMaxLayers];
};
hipError_t launch_gdn_commit_cols_multi(const GdnCommitSet &set, int layers, const GdnArgs &g,
                                        const int32_t *accept_result, hipStream_t s);
hipError_t launch_gdn_commit_cols(float *conv_state, float *state, const float *qkv, const float *conv,
                                  const float *alpha_raw, const float *beta_raw, const float *dt, const float *a_log,
                                  const GdnArgs &g, const int32_t *accept_result, hipStream_t s);
hipError_t launch_attention(const float *q, const void *kpool, const void *vpool, const int32_t *table, float *out,
                            const AttnArgs &a, void *scratch, const ModelDyn &dyn, int max_pos_hint, hipStream_t s);
hipError_t launch_gdn_conv(const float *conv_state, const float *qkv, const float *w, float *out, const GdnArgs &g,
                           hipStream_t s);
// mode 0: verify (outputs, state untouched); mode 1: commit accepted rows.
hipError_t launch_gdn_scan(float *state, const float *conv, const float *alpha, const float *beta, const float *dt,
                           const float *a, float *out, const GdnArgs &g, int mode, const int32_t *accept_result,
                           hipStream_t s);
hipError_t launch_gdn_norm_gate(const float *raw, const float *z, const float *norm, float *out, const GdnArgs &g,
                                hipStream_t s);
hipError_t launch_gdn_conv_commit(float *conv_state, const float *qkv, const GdnArgs &g, const int32_t *accept_result,
                                  hipStream_t s);
// nreq requests: request j's position is dyn.pos_dev[2 j], its result
// accept_result[4 j .. 4 j + 3]; the step counter advances once.
hipError_t launch_advance(const ModelDyn &dyn, const int32_t *accept_result, int rows, uint64_t *step, int nreq,
                          hipStream_t s);

// Mixture of experts (k_moe.hip). Assignment layout of the reference's MoE
// plan ops: counts [E], assignment arrays [E][rows*used] in (row, slot) order.
struct MoeGemm {
    const float *x;           // activations [.][K]
    const void *w0, *w1;      // expert-stacked Q4_K matrices [E*N rows of K]; w1 optional
    uint64_t row_bytes;
    const int32_t *counts, *arows, *aslots;
    int rows, used, experts, K, N;
    int by_slot;              // activation row = row*used + slot (down), else row (gate/up)
    int swiglu;               // out0 = SiLU(W0 y) * (W1 y)
    float *out0, *out1;       // [rows*used][N]
    int packed = 0;           // w0 / w1 in launch_moe_pack_q4k's layout
    int shared = 0;           // expert `experts` is the shared expert: every row, output slot `used`
                              // (activation / output rows of used + 1 slots)
};
// Rewrites expert-stacked Q4_K matrices [rows][K] (rows % 16 == 0) into the
// grouped GEMM's packed layout (same byte count) in dst.
hipError_t launch_moe_pack_q4k(const void *src, void *dst, uint64_t rows, int K, hipStream_t s);
// Workspace of launch_moe_gemm: the quantized activation rows.
uint64_t moe_gemm_ws(int act_rows, int K);
hipError_t launch_moe_router(const float *y, int H, int rows, const float *w, int E, float *logits, const float *sv,
                             float *extra, hipStream_t s);
hipError_t launch_moe_route(const float *logits, int rows, int E, int used, int32_t *ids, float *weights,
                            int32_t *counts, int32_t *arows, int32_t *aslots, float *aweights, hipStream_t s);
hipError_t launch_moe_gemm(const MoeGemm &g, void *ws, hipStream_t s);
hipError_t launch_moe_combine(float *x, const float *eo, const float *w, int rows, int used, int H, const float *so,
                              const float *sg, hipStream_t s, bool shared_slot = false);

}  // namespace yk
