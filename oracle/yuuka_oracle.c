/*
 * yuuka_oracle.c — CPU restatement of the reference's quant, matmul and
 * speculative-accept code. TEST INFRASTRUCTURE ONLY: the parity checker and
 * the timed CPU baseline; never linked into the product library.
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off -fPIC -pthread).
 * Each function cites the reference file:line it restates.
 */
#include "yuuka_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline float bits_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* tensor/half.go:6-31 */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (uint32_t)(h >> 10) & 0x1fu;
    uint32_t mant = (uint32_t)h & 0x03ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            uint32_t e = 127 - 15 + 1;
            while ((mant & 0x0400u) == 0) {
                mant <<= 1;
                e--;
            }
            mant &= 0x03ffu;
            bits = sign | e << 23 | mant << 13;
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | mant << 13;
    } else {
        bits = sign | (exp + 112) << 23 | mant << 13;
    }
    return bits_f32(bits);
}

/* tensor/half.go:35-68: truncating-with-half-add rounding as the reference does. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t b = f32_bits(f);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    int32_t exp = (int32_t)((b >> 23) & 0xffu) - 127;
    uint32_t mant = b & 0x7fffffu;
    if (exp == 128) {
        return mant != 0 ? (uint16_t)(sign | 0x7e00u) : (uint16_t)(sign | 0x7c00u);
    }
    if (exp > 15) return (uint16_t)(sign | 0x7c00u);
    if (exp < -24) return sign;
    if (exp < -14) {
        uint32_t shift = (uint32_t)(-exp - 14);
        uint32_t full = mant | 0x800000u;
        uint32_t rounded = full + (1u << (shift + 12));
        return (uint16_t)(sign | (uint16_t)(rounded >> (shift + 13)));
    }
    uint32_t rounded = mant + 0x1000u;
    if (rounded & 0x800000u) {
        exp++;
        rounded = 0;
        if (exp > 15) return (uint16_t)(sign | 0x7c00u);
    }
    return (uint16_t)(sign | (uint16_t)((exp + 15) << 10) | (uint16_t)(rounded >> 13));
}

/* tensor/dtype.go:102-171 */
static int block_layout(uint32_t dtype, uint64_t *elems, uint64_t *bytes) {
    switch (dtype) {
    case ORC_F32: *elems = 1; *bytes = 4; return 0;
    case ORC_F16: *elems = 1; *bytes = 2; return 0;
    case ORC_Q8_0: *elems = 32; *bytes = 34; return 0;
    case ORC_Q4_K: *elems = 256; *bytes = 144; return 0;
    case ORC_Q5_K: *elems = 256; *bytes = 176; return 0;
    case ORC_Q6_K: *elems = 256; *bytes = 210; return 0;
    default: return -1;
    }
}

uint64_t orc_row_bytes(uint32_t dtype, uint64_t cols) {
    uint64_t e, b;
    if (block_layout(dtype, &e, &b) != 0 || cols == 0 || cols % e != 0) return 0;
    return cols / e * b;
}

/* tensor/quant.go:96-103 */
void orc_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
        return;
    }
    *d = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
}

/* tensor/quant.go:105-125 */
static void dequant_q4k(float *dst, const uint8_t *src, uint64_t bytes) {
    for (uint64_t off = 0, si = 0; si + 144 <= bytes; off += 256, si += 144) {
        float d = orc_f16_to_f32(rd16(src + si));
        float dm = orc_f16_to_f32(rd16(src + si + 2));
        const uint8_t *scales = src + si + 4;
        const uint8_t *qs = src + si + 16;
        int is = 0;
        for (int j = 0; j < 256; j += 64) {
            uint8_t s0, m0, s1, m1;
            orc_scale_min_k4(is, scales, &s0, &m0);
            orc_scale_min_k4(is + 1, scales, &s1, &m1);
            float d1 = d * (float)s0, min1 = dm * (float)m0;
            float d2 = d * (float)s1, min2 = dm * (float)m1;
            for (int l = 0; l < 32; l++) {
                dst[off + j + l] = d1 * (float)(qs[l] & 0x0f) - min1;
                dst[off + j + 32 + l] = d2 * (float)(qs[l] >> 4) - min2;
            }
            qs += 32;
            is += 2;
        }
    }
}

/* tensor/quant.go:127-158 (Q5_K, same scale packing plus a high bit plane) */
static void dequant_q5k(float *dst, const uint8_t *src, uint64_t bytes) {
    for (uint64_t off = 0, si = 0; si + 176 <= bytes; off += 256, si += 176) {
        float d = orc_f16_to_f32(rd16(src + si));
        float dm = orc_f16_to_f32(rd16(src + si + 2));
        const uint8_t *scales = src + si + 4;
        const uint8_t *qh = src + si + 16;
        const uint8_t *ql = src + si + 48;
        int is = 0;
        for (int j = 0; j < 256; j += 64) {
            uint8_t s0, m0, s1, m1;
            orc_scale_min_k4(is, scales, &s0, &m0);
            orc_scale_min_k4(is + 1, scales, &s1, &m1);
            float d1 = d * (float)s0, min1 = dm * (float)m0;
            float d2 = d * (float)s1, min2 = dm * (float)m1;
            uint8_t bit0 = (uint8_t)(1u << (2 * (j / 64)));
            uint8_t bit1 = (uint8_t)(bit0 << 1);
            for (int l = 0; l < 32; l++) {
                uint8_t h0 = (qh[l] & bit0) ? 16 : 0;
                uint8_t h1 = (qh[l] & bit1) ? 16 : 0;
                dst[off + j + l] = d1 * (float)((ql[l] & 0x0f) + h0) - min1;
                dst[off + j + 32 + l] = d2 * (float)((ql[l] >> 4) + h1) - min2;
            }
            ql += 32;
            is += 2;
        }
    }
}

/* tensor/quant.go:261-285; d*sc*q evaluates left to right: (d*sc)*q. */
static void dequant_q6k(float *dst, const uint8_t *src, uint64_t bytes) {
    for (uint64_t off = 0, si = 0; si + 210 <= bytes; off += 256, si += 210) {
        const uint8_t *ql = src + si;
        const uint8_t *qh = src + si + 128;
        const uint8_t *sc = src + si + 192;
        float d = orc_f16_to_f32(rd16(src + si + 208));
        for (int n = 0; n < 2; n++) {
            const uint8_t *qlN = ql + n * 64;
            const uint8_t *qhN = qh + n * 32;
            const uint8_t *scN = sc + n * 8;
            uint64_t base = off + (uint64_t)n * 128;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int8_t q1 = (int8_t)((qlN[l] & 0x0f) | (((qhN[l] >> 0) & 3) << 4)) - 32;
                int8_t q2 = (int8_t)((qlN[l + 32] & 0x0f) | (((qhN[l] >> 2) & 3) << 4)) - 32;
                int8_t q3 = (int8_t)((qlN[l] >> 4) | (((qhN[l] >> 4) & 3) << 4)) - 32;
                int8_t q4 = (int8_t)((qlN[l + 32] >> 4) | (((qhN[l] >> 6) & 3) << 4)) - 32;
                dst[base + l] = d * (float)(int8_t)scN[is + 0] * (float)q1;
                dst[base + l + 32] = d * (float)(int8_t)scN[is + 2] * (float)q2;
                dst[base + l + 64] = d * (float)(int8_t)scN[is + 4] * (float)q3;
                dst[base + l + 96] = d * (float)(int8_t)scN[is + 6] * (float)q4;
            }
        }
    }
}

/* tensor/quant.go:86-93 */
static void dequant_q8_0(float *dst, const uint8_t *src, uint64_t bytes) {
    for (uint64_t off = 0, si = 0; si + 34 <= bytes; off += 32, si += 34) {
        float d = orc_f16_to_f32(rd16(src + si));
        for (int i = 0; i < 32; i++) dst[off + i] = d * (float)(int8_t)src[si + 2 + i];
    }
}

/* tensor/quant.go:15-62 */
int orc_dequantize_row(float *dst, uint64_t n, uint32_t dtype, const uint8_t *src,
                       uint64_t src_bytes) {
    uint64_t e, b;
    if (block_layout(dtype, &e, &b) != 0 || src_bytes % b != 0) return -1;
    if (src_bytes / b * e != n) return -1;
    switch (dtype) {
    case ORC_F32:
        for (uint64_t i = 0; i < n; i++) dst[i] = bits_f32(rd32(src + i * 4));
        return 0;
    case ORC_F16:
        for (uint64_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32(rd16(src + i * 2));
        return 0;
    case ORC_Q8_0: dequant_q8_0(dst, src, src_bytes); return 0;
    case ORC_Q4_K: dequant_q4k(dst, src, src_bytes); return 0;
    case ORC_Q5_K: dequant_q5k(dst, src, src_bytes); return 0;
    case ORC_Q6_K: dequant_q6k(dst, src, src_bytes); return 0;
    default: return -1;
    }
}

/* tensor/quant.go:378-466 matmulRows (serial fp32 sum per output). */
static void matmul_rows(float *dst, const float *x, int batch, const uint8_t *w, int64_t rows,
                        int64_t cols, uint32_t dtype, int64_t r0, int64_t r1, uint64_t rb) {
    float values[256];
    for (int64_t row = r0; row < r1; row++) {
        const uint8_t *src = w + (uint64_t)row * rb;
        for (int b = 0; b < batch; b++) {
            const float *xb = x + (int64_t)b * cols;
            float sum = 0.0f;
            if (dtype == ORC_F32) {
                for (int64_t i = 0; i < cols; i++) sum += xb[i] * bits_f32(rd32(src + i * 4));
            } else if (dtype == ORC_F16) {
                for (int64_t i = 0; i < cols; i++) sum += xb[i] * orc_f16_to_f32(rd16(src + i * 2));
            } else if (dtype == ORC_Q8_0) {
                /* quant.go:409-417: xb*d*q evaluates (xb*d)*q */
                for (int64_t blk = 0, si = 0; blk < cols / 32; blk++, si += 34) {
                    float d = orc_f16_to_f32(rd16(src + si));
                    for (int i = 0; i < 32; i++)
                        sum += xb[blk * 32 + i] * d * (float)(int8_t)src[si + 2 + i];
                }
            } else {
                uint64_t bb = dtype == ORC_Q4_K ? 144 : dtype == ORC_Q5_K ? 176 : 210;
                for (int64_t off = 0, si = 0; off < cols; off += 256, si += (int64_t)bb) {
                    if (dtype == ORC_Q4_K) dequant_q4k(values, src + si, 144);
                    else if (dtype == ORC_Q5_K) dequant_q5k(values, src + si, 176);
                    else dequant_q6k(values, src + si, 210);
                    for (int i = 0; i < 256; i++) sum += xb[off + i] * values[i];
                }
            }
            dst[(int64_t)b * rows + row] = sum;
        }
    }
}

typedef struct {
    float *dst;
    const float *x;
    int batch;
    const uint8_t *w;
    int64_t rows, cols;
    uint32_t dtype;
    int64_t r0, r1;
    uint64_t rb;
} mm_task;

static void *mm_worker(void *arg) {
    mm_task *t = (mm_task *)arg;
    matmul_rows(t->dst, t->x, t->batch, t->w, t->rows, t->cols, t->dtype, t->r0, t->r1, t->rb);
    return NULL;
}

/* tensor/quant.go:341-376 matmul: contiguous row chunks, one per worker. */
int orc_matmul(float *dst, const float *x, int batch, const uint8_t *w, int64_t rows,
               int64_t cols, uint32_t dtype, int workers) {
    uint64_t rb = orc_row_bytes(dtype, (uint64_t)cols);
    if (rb == 0 || rows <= 0 || batch <= 0) return -1;
    if (workers <= 0) {
        workers = 1;
        if ((uint64_t)rows * rb >= 64 * 1024) workers = (int)sysconf(_SC_NPROCESSORS_ONLN);
    }
    if (workers > rows) workers = (int)rows;
    if (workers <= 1) {
        matmul_rows(dst, x, batch, w, rows, cols, dtype, 0, rows, rb);
        return 0;
    }
    int64_t chunk = (rows + workers - 1) / workers;
    pthread_t *th = (pthread_t *)calloc((size_t)workers, sizeof(pthread_t));
    mm_task *tasks = (mm_task *)calloc((size_t)workers, sizeof(mm_task));
    int started = 0;
    for (int wi = 0; wi < workers; wi++) {
        int64_t start = (int64_t)wi * chunk;
        if (start >= rows) break;
        int64_t end = start + chunk < rows ? start + chunk : rows;
        tasks[wi] = (mm_task){dst, x, batch, w, rows, cols, dtype, start, end, rb};
        if (pthread_create(&th[wi], NULL, mm_worker, &tasks[wi]) != 0) {
            mm_worker(&tasks[wi]);
            th[wi] = 0;
        }
        started = wi + 1;
    }
    for (int wi = 0; wi < started; wi++)
        if (th[wi]) pthread_join(th[wi], NULL);
    free(th);
    free(tasks);
    return 0;
}

/* engine/speculative.go:263-271 */
int32_t orc_argmax(const float *logits, int64_t n) {
    int64_t best = 0;
    for (int64_t i = 1; i < n; i++)
        if (logits[i] > logits[best]) best = i;
    return (int32_t)best;
}

/* engine/speculative.go:39-66 */
int orc_lookup_draft(const int32_t *history, int n_history, int max_draft, int min_match,
                     int32_t *out) {
    if (max_draft <= 0 || min_match <= 0 || n_history <= min_match) return 0;
    int max_n = n_history - 1 < 8 ? n_history - 1 : 8;
    for (int n = max_n; n >= min_match; n--) {
        const int32_t *suffix = history + n_history - n;
        for (int start = n_history - n - 1; start >= 0; start--) {
            int match = 1;
            for (int i = 0; i < n; i++) {
                if (history[start + i] != suffix[i]) {
                    match = 0;
                    break;
                }
            }
            if (!match) continue;
            int follow = start + n;
            int take = n_history - follow < max_draft ? n_history - follow : max_draft;
            if (take <= 0) continue;
            memcpy(out, history + follow, (size_t)take * sizeof(int32_t));
            return take;
        }
    }
    return 0;
}

/* Philox4x32-10, Salmon et al., SC'11: 10 rounds of two 32x32->64 multiplies
 * with the Weyl key schedule. */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
    const uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; r++) {
        uint64_t p0 = (uint64_t)M0 * c0;
        uint64_t p1 = (uint64_t)M1 * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        uint32_t n1 = (uint32_t)p1;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        uint32_t n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += W0;
        k1 += W1;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

double orc_u01(uint32_t hi, uint32_t lo) {
    uint64_t v = (((uint64_t)hi << 32) | lo) >> 11;
    return (double)v * (1.0 / 9007199254740992.0);
}

double orc_draw(uint64_t seed, uint64_t step, uint32_t row, uint32_t request, uint32_t purpose) {
    uint32_t ctr[4] = {(uint32_t)step, (uint32_t)(step >> 32), request, (row << 8) | (purpose & 0xffu)};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t o[4];
    orc_philox4x32_10(ctr, key, o);
    return orc_u01(o[0], o[1]);
}

/* Sorting key of engine/sampling.go:84-89: logit desc, id asc. */
typedef struct {
    float logit;
    int32_t id;
} cand;

static int cand_cmp(const void *a, const void *b) {
    const cand *x = (const cand *)a, *y = (const cand *)b;
    if (x->logit != y->logit) return x->logit > y->logit ? -1 : 1;
    return x->id < y->id ? -1 : (x->id > y->id);
}

/* engine/sampling.go:60-129 up to (not including) the draw. */
int64_t orc_target_weights(const float *logits, int64_t n, float temperature, int top_k,
                           float top_p, double *w, double *total, int32_t *best) {
    for (int64_t i = 0; i < n; i++) w[i] = 0.0;
    *total = 0.0;
    *best = orc_argmax(logits, n);
    if (temperature <= 0.0f || top_k == 1) {
        /* Greedy sampler (sampling.go:57,64-72): the target is one-hot. */
        w[*best] = 1.0;
        *total = 1.0;
        return 1;
    }
    if (top_p == 0.0f) top_p = 1.0f; /* NewSampler: 0 means off (sampling.go:46-48) */
    cand *c = (cand *)malloc((size_t)n * sizeof(cand));
    int64_t m = 0;
    for (int64_t i = 0; i < n; i++) {
        float l = logits[i];
        if (isinf(l) && l < 0) continue;
        if (isnan(l)) continue;
        c[m].logit = l;
        c[m].id = (int32_t)i;
        m++;
    }
    if (m == 0) {
        free(c);
        return 0;
    }
    qsort(c, (size_t)m, sizeof(cand), cand_cmp);
    *best = c[0].id;
    if (top_k > 0 && top_k < m) m = top_k;
    float maxl = c[0].logit;
    double *pr = (double *)malloc((size_t)m * sizeof(double));
    double tot = 0.0;
    for (int64_t i = 0; i < m; i++) {
        pr[i] = exp((double)(c[i].logit - maxl) / (double)temperature);
        tot += pr[i];
    }
    if (tot == 0.0 || isinf(tot)) {
        free(pr);
        free(c);
        return -1;
    }
    if (top_p < 1.0f) {
        double cum = 0.0;
        int64_t keep = 0;
        for (int64_t i = 0; i < m; i++) {
            cum += pr[i] / tot;
            keep = i + 1;
            if (cum >= (double)top_p) break;
        }
        m = keep;
    }
    /* Index-order total: the summation order is not semantic. */
    for (int64_t i = 0; i < m; i++) w[c[i].id] = pr[i];
    double t2 = 0.0;
    for (int64_t i = 0; i < n; i++) t2 += w[i];
    *total = t2;
    free(pr);
    free(c);
    return m;
}

void orc_accept_greedy(const float *logits, int64_t vocab, int k, const int32_t *drafts,
                       int *accepted, int32_t *next, int32_t *row_argmax) {
    int a = 0;
    int32_t nxt = -1;
    for (int i = 0; i <= k; i++) {
        int32_t want = orc_argmax(logits + (int64_t)i * vocab, vocab);
        if (row_argmax) row_argmax[i] = want;
    }
    for (int i = 0; i <= k; i++) {
        int32_t want = row_argmax ? row_argmax[i] : orc_argmax(logits + (int64_t)i * vocab, vocab);
        if (i < k && want == drafts[i]) {
            a++;
            continue;
        }
        nxt = want;
        break;
    }
    *accepted = a;
    *next = nxt;
}

/* Inverse CDF in index order over w with `removed` excluded. */
static int32_t sample_index(const double *w, int64_t n, int32_t removed, double total, double u) {
    double target = u * total;
    double cum = 0.0;
    int32_t last = -1;
    for (int64_t j = 0; j < n; j++) {
        if (j == removed || w[j] <= 0.0) continue;
        cum += w[j];
        last = (int32_t)j;
        if (target < cum) return (int32_t)j;
    }
    return last;
}

void orc_accept_stochastic(const float *logits, int64_t vocab, int k, const int32_t *drafts,
                           float temperature, int top_k, float top_p, uint64_t seed,
                           uint64_t step, uint32_t request, int *accepted, int32_t *next,
                           double *p_draft, double *u_accept) {
    double *w = (double *)malloc((size_t)vocab * sizeof(double));
    int a = 0;
    int32_t nxt = -1;
    for (int i = 0; i <= k; i++) {
        const float *row = logits + (int64_t)i * vocab;
        double total;
        int32_t best;
        int64_t kept = orc_target_weights(row, vocab, temperature, top_k, top_p, w, &total, &best);
        if (kept <= 0) {
            /* total 0/Inf or every logit invalid: the sampler returns its
             * first candidate, so the target is one-hot there. */
            for (int64_t j = 0; j < vocab; j++) w[j] = 0.0;
            w[best] = 1.0;
            total = 1.0;
        }
        if (i < k) {
            int32_t d = drafts[i];
            double pd = (d >= 0 && d < vocab) ? w[d] / total : 0.0;
            double u = orc_draw(seed, step, (uint32_t)i, request, 0);
            if (p_draft) p_draft[i] = pd;
            if (u_accept) u_accept[i] = u;
            if (u < pd) {
                a++;
                continue;
            }
            double rest = 0.0;
            for (int64_t j = 0; j < vocab; j++)
                if (j != d) rest += w[j];
            double u2 = orc_draw(seed, step, (uint32_t)i, request, 1);
            nxt = rest > 0.0 ? sample_index(w, vocab, d, rest, u2) : best;
            break;
        }
        double u2 = orc_draw(seed, step, (uint32_t)i, request, 1);
        nxt = sample_index(w, vocab, -1, total, u2);
    }
    *accepted = a;
    *next = nxt;
    free(w);
}
