/*
 * qwen35_ref.h — CPU restatement of the reference qwen35 hybrid decoder
 * (model/qwen35 Go sources). TEST INFRASTRUCTURE ONLY: it is the logits oracle for
 * the device verify step and the timed CPU baseline of configs 2-5.
 *
 * The decoder runs one token at a time exactly as forwardOne
 * (model/qwen35/forward.go:116-155) does, re-reading every weight per token.
 */
#ifndef YUUKA_QWEN35_REF_H
#define YUUKA_QWEN35_REF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* model/qwen35/config.go:18-45 (the fields the decoder reads). */
typedef struct orc_q35_config {
    int32_t n_layers;
    int32_t hidden;
    int32_t ffn;
    int32_t heads;
    int32_t kv_heads;
    int32_t head_dim;
    int32_t rope_dim;
    int32_t vocab;
    int32_t conv_kernel;
    int32_t state_size;
    int32_t groups;
    int32_t rank;
    int32_t inner;
    int32_t full_interval;
    int32_t n_experts;     /* 0 for the dense model */
    int32_t n_experts_used;
    int32_t expert_ffn;
    int32_t shared_ffn;
    double rope_base;
    float eps;
    int32_t matmul_workers; /* <= 0: the reference GOMAXPROCS rule */
} orc_q35_config;

/* One packed matrix: data, rows (out features), cols (in features), dtype. */
typedef struct orc_q35_matrix {
    const uint8_t *data;
    int64_t rows;
    int64_t cols;
    uint32_t dtype;
    uint32_t pad;
} orc_q35_matrix;

/* model/qwen35/load.go:104-212 tensor set for one layer. */
typedef struct orc_q35_layer {
    const float *attn_norm;
    const float *post_norm;
    /* Gated DeltaNet (recurrent) layer */
    orc_q35_matrix qkv, gate, out, beta, alpha;
    const float *conv;     /* [conv_dim, kernel] */
    const float *dt;       /* [rank] */
    const float *a;        /* [rank] */
    const float *ssm_norm; /* [state_size] */
    /* Full attention layer */
    orc_q35_matrix q, k, v, o;
    const float *q_norm; /* [head_dim] */
    const float *k_norm; /* [head_dim] */
    /* Dense FFN */
    orc_q35_matrix ffn_gate, ffn_up, ffn_down;
    /* MoE FFN (qwen35moe) */
    orc_q35_matrix router;          /* [experts, hidden] */
    const float *shared_gate_vec;   /* [hidden] */
    orc_q35_matrix shared_gate, shared_up, shared_down;
    orc_q35_matrix gate_exps, up_exps, down_exps; /* rank-3, experts stacked by rows */
} orc_q35_layer;

typedef struct orc_q35_model {
    orc_q35_config cfg;
    orc_q35_matrix embedding; /* [vocab, hidden] */
    orc_q35_matrix output;    /* [vocab, hidden] */
    const float *output_norm;
    const orc_q35_layer *layers;
} orc_q35_model;

typedef struct orc_q35_pool orc_q35_pool;
typedef struct orc_q35_state orc_q35_state;

/* model/qwen35/kv_pool.go:33-63: blocks*block_size rows per full-attention
 * layer in format 0=F32, 1=F16, 2=Q8_0 (kv_format.go:15-28). */
orc_q35_pool *orc_q35_pool_new(const orc_q35_config *cfg, int32_t blocks, int32_t block_size,
                               int32_t format);
void orc_q35_pool_free(orc_q35_pool *pool);
/* Raw stored bytes of layer's K (which=0) or V (which=1) rows, or NULL. */
uint8_t *orc_q35_pool_data(orc_q35_pool *pool, int32_t layer, int32_t which, uint64_t *bytes);
int32_t orc_q35_pool_row_bytes(const orc_q35_pool *pool);

/* model/qwen35/state.go:104-169 NewPagedState: binds a block table (copied)
 * mapping ceil(capacity/block_size) logical blocks to pool blocks. */
orc_q35_state *orc_q35_state_new(const orc_q35_config *cfg, orc_q35_pool *pool,
                                 const int32_t *table, int32_t table_len, int32_t capacity);
void orc_q35_state_free(orc_q35_state *st);
/* state.go:174-189 (recurrent state cleared, pos 0; KV left as is). */
void orc_q35_state_reset(orc_q35_state *st);
int32_t orc_q35_state_pos(const orc_q35_state *st);
int orc_q35_state_set_pos(orc_q35_state *st, int32_t pos);
/* Pointers into one recurrent layer's conv state [(kernel-1)*conv_dim] and
 * matrix state [rank, state, state]; NULL for attention layers. */
float *orc_q35_state_conv(orc_q35_state *st, int32_t layer);
float *orc_q35_state_matrix(orc_q35_state *st, int32_t layer);
/* state.go:211-263 Snapshot / Restore. */
uint64_t orc_q35_snapshot_bytes(const orc_q35_state *st);
void orc_q35_snapshot(const orc_q35_state *st, uint8_t *out);
int orc_q35_restore(orc_q35_state *st, const uint8_t *data, uint64_t bytes);

/* forward.go:77-99 PrefillLogits when all_logits != 0 (logits is
 * [n, vocab]), otherwise forward.go:18-40 Forward (logits is [vocab] for the
 * last token). Returns 0 on success, negative on a range error. hidden_out,
 * when not NULL, receives the final normalized hidden rows [n, hidden]. */
int orc_q35_forward(const orc_q35_model *m, orc_q35_state *st, const int32_t *tokens, int32_t n,
                    int32_t all_logits, float *logits, float *hidden_out);

/* The residual stream after the last layer for each of n tokens, [n, hidden]
 * (forward.go:116-155 up to the output norm); no logits are computed. */
int orc_q35_forward_residual(const orc_q35_model *m, orc_q35_state *st, const int32_t *tokens,
                             int32_t n, float *residual_out);

/* Pieces exposed for kernel-level parity tests. */
void orc_rmsnorm(float *dst, const float *src, const float *weight, int32_t n, float eps);
void orc_rmsnorm_inplace(float *x, const float *weight, int32_t n, float eps);
void orc_l2norm_head(float *x, int32_t n, float eps, float extra);
void orc_rope(float *vec, int32_t heads, int32_t stride, int32_t head_dim, int32_t rot_dim,
              int32_t pos, double base);
float orc_sigmoid(float x);
float orc_silu(float x);
float orc_softplus(float x);
/* recurrent.go:56-105 gdnPerTokenScan over `rows` rows. */
void orc_gdn_scan(float *state, const float *conv, const float *alpha, const float *beta,
                  float *out, int32_t rows, int32_t groups, int32_t rank, int32_t state_size,
                  int32_t conv_dim);
/* recurrent.go:39-50 gdnNormGate. */
void orc_gdn_norm_gate(float *out, const float *z, const float *norm, int32_t rows, int32_t rank,
                       int32_t state_size, float eps);
/* forward.go:393-439 selectExperts. */
void orc_select_experts(const float *logits, int32_t n, int32_t k, int32_t *ids, float *weights);

#ifdef __cplusplus
}
#endif

#endif
