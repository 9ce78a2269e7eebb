/*
 * qwen35_ref.c — CPU restatement of model/qwen35 (forward.go, recurrent.go,
 * state.go, kv_pool.go, kv_format.go). TEST INFRASTRUCTURE ONLY.
 *
 * Arithmetic follows the Go expressions term by term: float32 values with
 * separately rounded multiply and add (-ffp-contract=off), float64 where the
 * Go code converts (norm sums, exp/log, RoPE angles).
 */
#include "qwen35_ref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "yuuka_oracle.h"

/* ---------------------------------------------------------------- helpers */

/* forward.go:460-470 */
void orc_rmsnorm(float *dst, const float *src, const float *weight, int32_t n, float eps) {
    double sum = 0.0;
    for (int32_t i = 0; i < n; i++) sum += (double)src[i] * (double)src[i];
    float mean = (float)(sum / (double)n);
    float scale = (float)(1.0 / sqrt((double)(mean + eps)));
    for (int32_t i = 0; i < n; i++) dst[i] = src[i] * scale * weight[i];
}

/* forward.go:472-482: x *= scale*weight (the product is formed first). */
void orc_rmsnorm_inplace(float *x, const float *weight, int32_t n, float eps) {
    double sum = 0.0;
    for (int32_t i = 0; i < n; i++) sum += (double)x[i] * (double)x[i];
    float mean = (float)(sum / (double)n);
    float scale = (float)(1.0 / sqrt((double)(mean + eps)));
    for (int32_t i = 0; i < n; i++) x[i] *= scale * weight[i];
}

/* forward.go:484-493 */
void orc_l2norm_head(float *x, int32_t n, float eps, float extra) {
    double sum = 0.0;
    for (int32_t i = 0; i < n; i++) sum += (double)x[i] * (double)x[i];
    float scale = (float)(1.0 / sqrt(sum + (double)eps)) * extra;
    for (int32_t i = 0; i < n; i++) x[i] *= scale;
}

/* forward.go:495-514 */
void orc_rope(float *vec, int32_t heads, int32_t stride, int32_t head_dim, int32_t rot_dim,
              int32_t pos, double base) {
    (void)head_dim;
    int32_t half = rot_dim / 2;
    for (int32_t i = 0; i < half; i++) {
        double theta = (double)pos * pow(base, -2.0 * (double)i / (double)rot_dim);
        float c = (float)cos(theta);
        float s = (float)sin(theta);
        for (int32_t h = 0; h < heads; h++) {
            int32_t off = h * stride + i;
            float x0 = vec[off];
            float x1 = vec[off + half];
            vec[off] = x0 * c - x1 * s;
            vec[off + half] = x0 * s + x1 * c;
        }
    }
}

/* forward.go:516-536 */
static void softmax_inplace(float *x, int32_t n) {
    if (n == 0) return;
    float mx = x[0];
    for (int32_t i = 1; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int32_t i = 0; i < n; i++) {
        float e = (float)exp((double)(x[i] - mx));
        x[i] = e;
        sum += e;
    }
    float inv = 1.0f / sum;
    for (int32_t i = 0; i < n; i++) x[i] *= inv;
}

/* forward.go:538-544 */
static float dotf(const float *a, const float *b, int32_t n) {
    float sum = 0.0f;
    for (int32_t i = 0; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* forward.go:552-565 */
float orc_sigmoid(float x) { return 1.0f / (1.0f + (float)exp((double)(-x))); }
float orc_silu(float x) { return x * orc_sigmoid(x); }
float orc_softplus(float x) {
    if (x > 20.0f) return x;
    return (float)log1p(exp((double)x));
}

static int matvec(const orc_q35_model *m, const orc_q35_matrix *w, float *dst, const float *x) {
    return orc_matmul(dst, x, 1, w->data, w->rows, w->cols, w->dtype, m->cfg.matmul_workers);
}

/* ------------------------------------------------------------------ KV pool */

struct orc_q35_pool {
    int32_t blocks, block_size, format, kv_dim, row_bytes, n_layers;
    uint8_t **k;
    uint8_t **v;
};

static int is_recurrent(const orc_q35_config *c, int32_t layer) {
    return (layer + 1) % c->full_interval != 0; /* config.go:280-282 */
}

static int32_t kv_row_bytes(int32_t format, int32_t kv_dim) { /* kv_format.go:75-91 */
    if (format == 0) return kv_dim * 4;
    if (format == 1) return kv_dim * 2;
    return (kv_dim + 31) / 32 * 34;
}

orc_q35_pool *orc_q35_pool_new(const orc_q35_config *cfg, int32_t blocks, int32_t block_size,
                               int32_t format) {
    if (blocks <= 0 || block_size <= 0 || format < 0 || format > 2) return NULL;
    orc_q35_pool *p = (orc_q35_pool *)calloc(1, sizeof(*p));
    p->blocks = blocks;
    p->block_size = block_size;
    p->format = format;
    p->kv_dim = cfg->kv_heads * cfg->head_dim;
    p->row_bytes = kv_row_bytes(format, p->kv_dim);
    p->n_layers = cfg->n_layers;
    p->k = (uint8_t **)calloc((size_t)cfg->n_layers, sizeof(uint8_t *));
    p->v = (uint8_t **)calloc((size_t)cfg->n_layers, sizeof(uint8_t *));
    size_t bytes = (size_t)blocks * (size_t)block_size * (size_t)p->row_bytes;
    for (int32_t i = 0; i < cfg->n_layers; i++) {
        if (is_recurrent(cfg, i)) continue;
        p->k[i] = (uint8_t *)calloc(bytes, 1);
        p->v[i] = (uint8_t *)calloc(bytes, 1);
    }
    return p;
}

void orc_q35_pool_free(orc_q35_pool *p) {
    if (!p) return;
    for (int32_t i = 0; i < p->n_layers; i++) {
        free(p->k[i]);
        free(p->v[i]);
    }
    free(p->k);
    free(p->v);
    free(p);
}

uint8_t *orc_q35_pool_data(orc_q35_pool *p, int32_t layer, int32_t which, uint64_t *bytes) {
    if (layer < 0 || layer >= p->n_layers) return NULL;
    if (bytes) *bytes = (uint64_t)p->blocks * (uint64_t)p->block_size * (uint64_t)p->row_bytes;
    return which == 0 ? p->k[layer] : p->v[layer];
}

int32_t orc_q35_pool_row_bytes(const orc_q35_pool *p) { return p->row_bytes; }

/* kv_format.go:93-137 EncodeRow */
static void encode_row(int32_t format, uint8_t *dst, const float *src, int32_t n) {
    if (format == 0) {
        memcpy(dst, src, (size_t)n * 4);
    } else if (format == 1) {
        for (int32_t i = 0; i < n; i++) {
            uint16_t h = orc_f32_to_f16(src[i]);
            dst[2 * i] = (uint8_t)h;
            dst[2 * i + 1] = (uint8_t)(h >> 8);
        }
    } else {
        for (int32_t blk = 0; blk < (n + 31) / 32; blk++) {
            int32_t start = blk * 32, end = start + 32 < n ? start + 32 : n;
            float max_abs = 0.0f;
            for (int32_t i = start; i < end; i++) {
                float a = (float)fabs((double)src[i]);
                if (a > max_abs) max_abs = a;
            }
            float scale = max_abs / 127.0f;
            uint8_t *o = dst + blk * 34;
            uint16_t hs = orc_f32_to_f16(scale);
            o[0] = (uint8_t)hs;
            o[1] = (uint8_t)(hs >> 8);
            for (int32_t i = 0; i < 32; i++) {
                int8_t q = 0;
                if (start + i < end && scale != 0.0f) q = (int8_t)round((double)(src[start + i] / scale));
                o[2 + i] = (uint8_t)q;
            }
        }
    }
}

/* kv_format.go:140-168 DecodeRow */
static void decode_row(int32_t format, float *dst, const uint8_t *src, int32_t n) {
    if (format == 0) {
        memcpy(dst, src, (size_t)n * 4);
    } else if (format == 1) {
        for (int32_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32((uint16_t)(src[2 * i] | (src[2 * i + 1] << 8)));
    } else {
        for (int32_t i = 0; i < n; i++) {
            const uint8_t *o = src + i / 32 * 34;
            float scale = orc_f16_to_f32((uint16_t)(o[0] | (o[1] << 8)));
            dst[i] = scale * (float)(int8_t)o[2 + i % 32];
        }
    }
}

/* -------------------------------------------------------------------- state */

struct orc_q35_state {
    orc_q35_config cfg;
    int32_t pos, capacity, conv_dim;
    int32_t *table;
    int32_t table_len;
    orc_q35_pool *pool;
    float **conv;
    float **mat;
    /* scratch (state.go:13-44) */
    float *x, *norm, *q, *k, *v, *attn, *tmp, *qkv, *z, *beta, *alpha, *cv, *gdn, *fg, *fu;
    float *scores, *sk, *d, *kvrow;
    float *router, *eg, *eu, *eo, *ew;
    int32_t *eid;
};

orc_q35_state *orc_q35_state_new(const orc_q35_config *cfg, orc_q35_pool *pool,
                                 const int32_t *table, int32_t table_len, int32_t capacity) {
    if (!cfg || !pool || !table || capacity <= 0) return NULL;
    if ((int64_t)table_len * pool->block_size < capacity) return NULL;
    orc_q35_state *s = (orc_q35_state *)calloc(1, sizeof(*s));
    s->cfg = *cfg;
    s->capacity = capacity;
    s->pool = pool;
    s->table = (int32_t *)malloc((size_t)table_len * sizeof(int32_t));
    memcpy(s->table, table, (size_t)table_len * sizeof(int32_t));
    s->table_len = table_len;
    s->conv_dim = 2 * cfg->groups * cfg->state_size + cfg->inner;
    s->conv = (float **)calloc((size_t)cfg->n_layers, sizeof(float *));
    s->mat = (float **)calloc((size_t)cfg->n_layers, sizeof(float *));
    for (int32_t i = 0; i < cfg->n_layers; i++) {
        if (!is_recurrent(cfg, i)) continue;
        s->conv[i] = (float *)calloc((size_t)(cfg->conv_kernel - 1) * (size_t)s->conv_dim, 4);
        s->mat[i] = (float *)calloc((size_t)cfg->rank * cfg->state_size * cfg->state_size, 4);
    }
    int32_t qdim = cfg->heads * cfg->head_dim * 2, kvdim = cfg->kv_heads * cfg->head_dim;
    int32_t odim = cfg->heads * cfg->head_dim;
    int32_t ffn = cfg->ffn > 0 ? cfg->ffn : 1;
    s->x = calloc((size_t)cfg->hidden, 4);
    s->norm = calloc((size_t)cfg->hidden, 4);
    s->q = calloc((size_t)qdim, 4);
    s->k = calloc((size_t)kvdim, 4);
    s->v = calloc((size_t)kvdim, 4);
    s->attn = calloc((size_t)odim, 4);
    s->tmp = calloc((size_t)cfg->hidden, 4);
    s->qkv = calloc((size_t)s->conv_dim, 4);
    s->z = calloc((size_t)cfg->inner, 4);
    s->beta = calloc((size_t)cfg->rank, 4);
    s->alpha = calloc((size_t)cfg->rank, 4);
    s->cv = calloc((size_t)s->conv_dim, 4);
    s->gdn = calloc((size_t)cfg->inner, 4);
    s->fg = calloc((size_t)ffn, 4);
    s->fu = calloc((size_t)ffn, 4);
    s->scores = calloc((size_t)capacity, 4);
    s->sk = calloc((size_t)cfg->state_size, 4);
    s->d = calloc((size_t)cfg->state_size, 4);
    s->kvrow = calloc((size_t)kvdim, 4);
    if (cfg->n_experts > 0) {
        int32_t width = cfg->expert_ffn > cfg->shared_ffn ? cfg->expert_ffn : cfg->shared_ffn;
        s->router = calloc((size_t)cfg->n_experts, 4);
        s->eg = calloc((size_t)width, 4);
        s->eu = calloc((size_t)width, 4);
        s->eo = calloc((size_t)cfg->hidden, 4);
        s->ew = calloc((size_t)cfg->n_experts_used, 4);
        s->eid = calloc((size_t)cfg->n_experts_used, 4);
    }
    return s;
}

void orc_q35_state_free(orc_q35_state *s) {
    if (!s) return;
    for (int32_t i = 0; i < s->cfg.n_layers; i++) {
        free(s->conv[i]);
        free(s->mat[i]);
    }
    free(s->conv); free(s->mat); free(s->table);
    free(s->x); free(s->norm); free(s->q); free(s->k); free(s->v); free(s->attn); free(s->tmp);
    free(s->qkv); free(s->z); free(s->beta); free(s->alpha); free(s->cv); free(s->gdn);
    free(s->fg); free(s->fu); free(s->scores); free(s->sk); free(s->d); free(s->kvrow);
    free(s->router); free(s->eg); free(s->eu); free(s->eo); free(s->ew); free(s->eid);
    free(s);
}

void orc_q35_state_reset(orc_q35_state *s) {
    s->pos = 0;
    int32_t cd = s->conv_dim;
    for (int32_t i = 0; i < s->cfg.n_layers; i++) {
        if (!s->conv[i]) continue;
        memset(s->conv[i], 0, (size_t)(s->cfg.conv_kernel - 1) * (size_t)cd * 4);
        memset(s->mat[i], 0, (size_t)s->cfg.rank * s->cfg.state_size * s->cfg.state_size * 4);
    }
}

int32_t orc_q35_state_pos(const orc_q35_state *s) { return s->pos; }

int orc_q35_state_set_pos(orc_q35_state *s, int32_t pos) { /* state.go:201-207 */
    if (pos < 0 || pos > s->capacity) return -1;
    s->pos = pos;
    return 0;
}

float *orc_q35_state_conv(orc_q35_state *s, int32_t layer) {
    return (layer >= 0 && layer < s->cfg.n_layers) ? s->conv[layer] : NULL;
}
float *orc_q35_state_matrix(orc_q35_state *s, int32_t layer) {
    return (layer >= 0 && layer < s->cfg.n_layers) ? s->mat[layer] : NULL;
}

static uint64_t layer_conv_elems(const orc_q35_state *s) {
    return (uint64_t)(s->cfg.conv_kernel - 1) * (uint64_t)s->conv_dim;
}
static uint64_t layer_mat_elems(const orc_q35_state *s) {
    return (uint64_t)s->cfg.rank * s->cfg.state_size * s->cfg.state_size;
}

uint64_t orc_q35_snapshot_bytes(const orc_q35_state *s) {
    uint64_t e = 0;
    for (int32_t i = 0; i < s->cfg.n_layers; i++)
        if (s->conv[i]) e += layer_conv_elems(s) + layer_mat_elems(s);
    return e * 4;
}

/* state.go:211-234: conv then matrix, per recurrent layer, little-endian f32. */
void orc_q35_snapshot(const orc_q35_state *s, uint8_t *out) {
    uint64_t off = 0;
    for (int32_t i = 0; i < s->cfg.n_layers; i++) {
        if (!s->conv[i]) continue;
        memcpy(out + off, s->conv[i], layer_conv_elems(s) * 4);
        off += layer_conv_elems(s) * 4;
        memcpy(out + off, s->mat[i], layer_mat_elems(s) * 4);
        off += layer_mat_elems(s) * 4;
    }
}

/* state.go:238-263 */
int orc_q35_restore(orc_q35_state *s, const uint8_t *data, uint64_t bytes) {
    if (bytes != orc_q35_snapshot_bytes(s)) return -1;
    uint64_t off = 0;
    for (int32_t i = 0; i < s->cfg.n_layers; i++) {
        if (!s->conv[i]) continue;
        memcpy(s->conv[i], data + off, layer_conv_elems(s) * 4);
        off += layer_conv_elems(s) * 4;
        memcpy(s->mat[i], data + off, layer_mat_elems(s) * 4);
        off += layer_mat_elems(s) * 4;
    }
    return 0;
}

/* kv_pool.go:119-129 rowOffset through memory/memory.go:254-266 Table.Map */
static int64_t row_offset(const orc_q35_state *s, int32_t pos) {
    int32_t bs = s->pool->block_size;
    int32_t idx = pos / bs;
    if (pos < 0 || idx >= s->table_len) return -1;
    int32_t block = s->table[idx];
    if (block < 0 || block >= s->pool->blocks) return -1;
    return ((int64_t)block * bs + pos % bs) * s->pool->row_bytes;
}

/* ------------------------------------------------------------------ layers */

/* recurrent.go:56-105 */
void orc_gdn_scan(float *state, const float *conv, const float *alpha, const float *beta,
                  float *out, int32_t rows, int32_t groups, int32_t rank, int32_t ss,
                  int32_t conv_dim) {
    int32_t key_dim = groups * ss;
    float *sk = (float *)malloc((size_t)ss * 4);
    float *d = (float *)malloc((size_t)ss * 4);
    for (int32_t r = 0; r < rows; r++) {
        const float *row = conv + (int64_t)r * conv_dim;
        for (int32_t h = 0; h < rank; h++) {
            int32_t kh = h % groups;
            const float *q = row + kh * ss;
            const float *k = row + key_dim + kh * ss;
            const float *v = row + 2 * key_dim + h * ss;
            float *mat = state + (int64_t)h * ss * ss;
            float decay = (float)exp((double)alpha[r * rank + h]);
            for (int64_t i = 0; i < (int64_t)ss * ss; i++) mat[i] *= decay;
            for (int32_t j = 0; j < ss; j++) sk[j] = 0.0f;
            for (int32_t i = 0; i < ss; i++) {
                float ki = k[i];
                const float *mrow = mat + (int64_t)i * ss;
                for (int32_t j = 0; j < ss; j++) sk[j] += mrow[j] * ki;
            }
            float b = beta[r * rank + h];
            for (int32_t j = 0; j < ss; j++) d[j] = (v[j] - sk[j]) * b;
            for (int32_t i = 0; i < ss; i++) {
                float ki = k[i];
                float *mrow = mat + (int64_t)i * ss;
                for (int32_t j = 0; j < ss; j++) mrow[j] += ki * d[j];
            }
            float *head = out + ((int64_t)r * rank + h) * ss;
            for (int32_t j = 0; j < ss; j++) head[j] = 0.0f;
            for (int32_t i = 0; i < ss; i++) {
                float qi = q[i];
                const float *mrow = mat + (int64_t)i * ss;
                for (int32_t j = 0; j < ss; j++) head[j] += mrow[j] * qi;
            }
        }
    }
    free(sk);
    free(d);
}

/* recurrent.go:39-50 */
void orc_gdn_norm_gate(float *out, const float *z, const float *norm, int32_t rows, int32_t rank,
                       int32_t ss, float eps) {
    for (int32_t r = 0; r < rows; r++) {
        for (int32_t h = 0; h < rank; h++) {
            float *row = out + ((int64_t)r * rank + h) * ss;
            orc_rmsnorm_inplace(row, norm, ss, eps);
            const float *gate = z + ((int64_t)r * rank + h) * ss;
            for (int32_t d = 0; d < ss; d++) row[d] *= orc_silu(gate[d]);
        }
    }
}

/* forward.go:393-439 */
void orc_select_experts(const float *logits, int32_t n, int32_t k, int32_t *ids, float *weights) {
    for (int32_t slot = 0; slot < k; slot++) {
        int32_t best = -1;
        for (int32_t e = 0; e < n; e++) {
            int used = 0;
            for (int32_t p = 0; p < slot; p++)
                if (ids[p] == e) { used = 1; break; }
            if (used) continue;
            if (best < 0 || logits[e] > logits[best]) best = e;
        }
        if (best < 0) {
            ids[slot] = 0;
            weights[slot] = 0.0f;
            continue;
        }
        ids[slot] = best;
    }
    if (k == 0) return;
    float mx = logits[ids[0]];
    for (int32_t s = 1; s < k; s++)
        if (logits[ids[s]] > mx) mx = logits[ids[s]];
    float total = 0.0f;
    for (int32_t s = 0; s < k; s++) {
        float w = (float)exp((double)(logits[ids[s]] - mx));
        weights[s] = w;
        total += w;
    }
    if (total > 0.0f)
        for (int32_t s = 0; s < k; s++) weights[s] /= total;
}

static orc_q35_matrix expert_slice(const orc_q35_matrix *m, int32_t expert, int64_t rows) {
    orc_q35_matrix e = *m;
    uint64_t rb = orc_row_bytes(m->dtype, (uint64_t)m->cols);
    e.data = m->data + (uint64_t)expert * (uint64_t)rows * rb;
    e.rows = rows;
    return e;
}

/* forward.go:295-315 and 320-389 */
static int forward_ffn(const orc_q35_model *m, const orc_q35_layer *L, orc_q35_state *s) {
    const orc_q35_config *c = &m->cfg;
    orc_rmsnorm(s->norm, s->x, L->post_norm, c->hidden, c->eps);
    if (c->n_experts <= 0) {
        if (matvec(m, &L->ffn_gate, s->fg, s->norm)) return -1;
        if (matvec(m, &L->ffn_up, s->fu, s->norm)) return -1;
        for (int32_t i = 0; i < c->ffn; i++) s->fg[i] = orc_silu(s->fg[i]) * s->fu[i];
        if (matvec(m, &L->ffn_down, s->tmp, s->fg)) return -1;
        for (int32_t i = 0; i < c->hidden; i++) s->x[i] += s->tmp[i];
        return 0;
    }
    if (matvec(m, &L->router, s->router, s->norm)) return -1;
    orc_select_experts(s->router, c->n_experts, c->n_experts_used, s->eid, s->ew);
    memset(s->tmp, 0, (size_t)c->hidden * 4);
    for (int32_t slot = 0; slot < c->n_experts_used; slot++) {
        int32_t id = s->eid[slot];
        if (id < 0 || id >= c->n_experts) return -2;
        orc_q35_matrix g = expert_slice(&L->gate_exps, id, c->expert_ffn);
        orc_q35_matrix u = expert_slice(&L->up_exps, id, c->expert_ffn);
        orc_q35_matrix dn = expert_slice(&L->down_exps, id, c->hidden);
        if (matvec(m, &g, s->eg, s->norm)) return -1;
        if (matvec(m, &u, s->eu, s->norm)) return -1;
        for (int32_t i = 0; i < c->expert_ffn; i++) s->eg[i] = orc_silu(s->eg[i]) * s->eu[i];
        if (matvec(m, &dn, s->eo, s->eg)) return -1;
        float w = s->ew[slot];
        for (int32_t i = 0; i < c->hidden; i++) s->tmp[i] += w * s->eo[i];
    }
    if (matvec(m, &L->shared_gate, s->eg, s->norm)) return -1;
    if (matvec(m, &L->shared_up, s->eu, s->norm)) return -1;
    for (int32_t i = 0; i < c->shared_ffn; i++) s->eg[i] = orc_silu(s->eg[i]) * s->eu[i];
    if (matvec(m, &L->shared_down, s->eo, s->eg)) return -1;
    float sg = orc_sigmoid(dotf(L->shared_gate_vec, s->norm, c->hidden));
    for (int32_t i = 0; i < c->hidden; i++) s->tmp[i] += sg * s->eo[i];
    for (int32_t i = 0; i < c->hidden; i++) s->x[i] += s->tmp[i];
    return 0;
}

/* forward.go:157-226 */
static int forward_full(const orc_q35_model *m, int32_t index, const orc_q35_layer *L,
                        orc_q35_state *s) {
    const orc_q35_config *c = &m->cfg;
    orc_rmsnorm(s->norm, s->x, L->attn_norm, c->hidden, c->eps);
    if (matvec(m, &L->q, s->q, s->norm)) return -1;
    if (matvec(m, &L->k, s->k, s->norm)) return -1;
    if (matvec(m, &L->v, s->v, s->norm)) return -1;
    int32_t hd = c->head_dim;
    for (int32_t h = 0; h < c->heads; h++) orc_rmsnorm_inplace(s->q + h * 2 * hd, L->q_norm, hd, c->eps);
    for (int32_t h = 0; h < c->kv_heads; h++) orc_rmsnorm_inplace(s->k + h * hd, L->k_norm, hd, c->eps);
    orc_rope(s->q, c->heads, 2 * hd, hd, c->rope_dim, s->pos, c->rope_base);
    orc_rope(s->k, c->kv_heads, hd, hd, c->rope_dim, s->pos, c->rope_base);

    int32_t kvdim = c->kv_heads * hd;
    int64_t off = row_offset(s, s->pos);
    if (off < 0) return -3;
    encode_row(s->pool->format, s->pool->k[index] + off, s->k, kvdim);
    encode_row(s->pool->format, s->pool->v[index] + off, s->v, kvdim);

    int32_t group = c->heads / c->kv_heads;
    float scale = (float)(1.0 / sqrt((double)hd));
    int32_t length = s->pos + 1;
    for (int32_t h = 0; h < c->heads; h++) {
        int32_t kvh = h / group;
        const float *q = s->q + h * 2 * hd;
        for (int32_t p = 0; p < length; p++) {
            int64_t o = row_offset(s, p);
            if (o < 0) return -3;
            decode_row(s->pool->format, s->kvrow, s->pool->k[index] + o, kvdim);
            s->scores[p] = dotf(q, s->kvrow + kvh * hd, hd) * scale;
        }
        softmax_inplace(s->scores, length);
        float *out = s->attn + h * hd;
        memset(out, 0, (size_t)hd * 4);
        for (int32_t p = 0; p < length; p++) {
            float wgt = s->scores[p];
            int64_t o = row_offset(s, p);
            decode_row(s->pool->format, s->kvrow, s->pool->v[index] + o, kvdim);
            const float *v = s->kvrow + kvh * hd;
            for (int32_t d = 0; d < hd; d++) out[d] += wgt * v[d];
        }
        const float *gate = s->q + h * 2 * hd + hd;
        for (int32_t d = 0; d < hd; d++) out[d] *= orc_sigmoid(gate[d]);
    }
    if (matvec(m, &L->o, s->tmp, s->attn)) return -1;
    for (int32_t i = 0; i < c->hidden; i++) s->x[i] += s->tmp[i];
    return forward_ffn(m, L, s);
}

/* forward.go:228-293 */
static int forward_recurrent(const orc_q35_model *m, int32_t index, const orc_q35_layer *L,
                             orc_q35_state *s) {
    const orc_q35_config *c = &m->cfg;
    orc_rmsnorm(s->norm, s->x, L->attn_norm, c->hidden, c->eps);
    if (matvec(m, &L->qkv, s->qkv, s->norm)) return -1;
    if (matvec(m, &L->gate, s->z, s->norm)) return -1;
    if (matvec(m, &L->beta, s->beta, s->norm)) return -1;
    if (matvec(m, &L->alpha, s->alpha, s->norm)) return -1;
    for (int32_t h = 0; h < c->rank; h++) {
        s->beta[h] = orc_sigmoid(s->beta[h]);
        s->alpha[h] = orc_softplus(s->alpha[h] + L->dt[h]) * L->a[h];
    }
    float *cst = s->conv[index];
    int32_t cd = s->conv_dim, K = c->conv_kernel;
    for (int32_t ch = 0; ch < cd; ch++) {
        float sum = 0.0f;
        int32_t base = ch * K, sb = ch * (K - 1);
        for (int32_t t = 0; t < K - 1; t++) sum += L->conv[base + t] * cst[sb + t];
        sum += L->conv[base + K - 1] * s->qkv[ch];
        s->cv[ch] = orc_silu(sum);
        for (int32_t t = 0; t < K - 2; t++) cst[sb + t] = cst[sb + t + 1];
        if (K > 1) cst[sb + K - 2] = s->qkv[ch];
    }
    int32_t ss = c->state_size, key_dim = c->groups * ss;
    float qscale = (float)(1.0 / sqrt((double)ss));
    for (int32_t h = 0; h < c->groups; h++) {
        orc_l2norm_head(s->cv + h * ss, ss, c->eps, qscale);
        orc_l2norm_head(s->cv + key_dim + h * ss, ss, c->eps, 1.0f);
    }
    orc_gdn_scan(s->mat[index], s->cv, s->alpha, s->beta, s->gdn, 1, c->groups, c->rank, ss, cd);
    orc_gdn_norm_gate(s->gdn, s->z, L->ssm_norm, 1, c->rank, ss, c->eps);
    if (matvec(m, &L->out, s->tmp, s->gdn)) return -1;
    for (int32_t i = 0; i < c->hidden; i++) s->x[i] += s->tmp[i];
    return forward_ffn(m, L, s);
}

/* forward.go:116-155 */
static int forward_one(const orc_q35_model *m, orc_q35_state *s, int32_t token, int want_logits,
                       float *logits, float *hidden_out, float *residual_out) {
    const orc_q35_config *c = &m->cfg;
    if (s->pos >= s->capacity) return -4;
    uint64_t rb = orc_row_bytes(m->embedding.dtype, (uint64_t)c->hidden);
    if (orc_dequantize_row(s->x, (uint64_t)c->hidden, m->embedding.dtype,
                           m->embedding.data + (uint64_t)token * rb, rb) != 0)
        return -5;
    for (int32_t i = 0; i < c->n_layers; i++) {
        int rc = is_recurrent(c, i) ? forward_recurrent(m, i, &m->layers[i], s)
                                    : forward_full(m, i, &m->layers[i], s);
        if (rc) return rc;
    }
    if (residual_out) memcpy(residual_out, s->x, (size_t)c->hidden * 4);
    orc_rmsnorm(s->norm, s->x, m->output_norm, c->hidden, c->eps);
    if (hidden_out) memcpy(hidden_out, s->norm, (size_t)c->hidden * 4);
    if (want_logits && matvec(m, &m->output, logits, s->norm)) return -1;
    s->pos++;
    return 0;
}

int orc_q35_forward(const orc_q35_model *m, orc_q35_state *s, const int32_t *tokens, int32_t n,
                    int32_t all_logits, float *logits, float *hidden_out) {
    if (n <= 0) return -6;
    if (s->pos + n > s->capacity) return -7;
    for (int32_t i = 0; i < n; i++) {
        if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab) return -8;
        int want = all_logits || i == n - 1;
        float *dst = all_logits ? logits + (int64_t)i * m->cfg.vocab : logits;
        float *hid = hidden_out ? hidden_out + (int64_t)(all_logits ? i : 0) * m->cfg.hidden : NULL;
        int rc = forward_one(m, s, tokens[i], want, dst, hid, NULL);
        if (rc) return rc;
    }
    return 0;
}

/* forward.go:116-155 without the output head: the residual stream after the
 * last layer, [n, hidden] (test hook for closed-form layer checks). */
int orc_q35_forward_residual(const orc_q35_model *m, orc_q35_state *s, const int32_t *tokens,
                             int32_t n, float *residual_out) {
    if (n <= 0) return -6;
    if (s->pos + n > s->capacity) return -7;
    for (int32_t i = 0; i < n; i++) {
        if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab) return -8;
        int rc = forward_one(m, s, tokens[i], 0, NULL, NULL,
                             residual_out + (int64_t)i * m->cfg.hidden);
        if (rc) return rc;
    }
    return 0;
}
