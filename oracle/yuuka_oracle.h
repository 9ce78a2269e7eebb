/*
 * yuuka_oracle.h — CPU restatement of the reference speculative verify path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker and the timed
 * CPU baseline. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links it and has
 * no CPU fallback.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the RandomLemon/yuuka tree). Built with -O2 -ffp-contract=off so that every
 * a*b+c stays two rounded operations, as the Go amd64 compiler emits them at
 * the default GOAMD64=v1 level (no FMA instructions are generated there).
 *
 * Parity status per function is recorded in the header comment of each
 * function ("pinned by ..." or "parity unpinned").
 */
#ifndef YUUKA_ORACLE_H
#define YUUKA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes follow yuuka_dtype (backend/hip/bridge/yuuka_hip.h:198-207). */
enum {
    ORC_F32 = 0,
    ORC_F16 = 1,
    ORC_Q8_0 = 8,
    ORC_Q4_K = 12,
    ORC_Q5_K = 13,
    ORC_Q6_K = 14
};

/* tensor/half.go:6-31. Pinned by exhaustive comparison with the IEEE decode
 * (all 65536 inputs) and TestFloat16RoundTrip values. */
float orc_f16_to_f32(uint16_t h);
/* tensor/half.go:35-68. Pinned by TestFloat16RoundTrip (tensor/quant_test.go:14-35)
 * and by round-trip of every finite half. */
uint16_t orc_f32_to_f16(float f);

/* tensor/dtype.go:102-171: block elements/bytes; row bytes or 0 if invalid. */
uint64_t orc_row_bytes(uint32_t dtype, uint64_t cols);

/* tensor/quant.go:96-103 getScaleMinK4. */
void orc_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m);

/* tensor/quant.go:15-62 DequantizeRow for F32/F16/Q8_0/Q4_K/Q5_K/Q6_K.
 * Pinned by TestDequantizeQ4K/Q5K/Q6K KATs and a brute-force nibble sweep.
 * Returns 0 on success, -1 on a bad dtype or length. */
int orc_dequantize_row(float *dst, uint64_t n, uint32_t dtype, const uint8_t *src,
                       uint64_t src_bytes);

/* tensor/quant.go:341-466 matmul + matmulRows: dst[b, r] = sum_i x[b,i]*w[r,i]
 * with a serial fp32 sum per (row, b), dequantizing one 256-block at a time.
 * Rows are split into `workers` contiguous chunks (quant.go:346-375); workers
 * <= 0 uses the reference rule (GOMAXPROCS = all online cores when the matrix
 * is >= 64 KiB, else 1). Pinned by TestMatMulMatchesDequantizedDot
 * (tensor/quant_test.go:252-342). */
int orc_matmul(float *dst, const float *x, int batch, const uint8_t *w,
               int64_t rows, int64_t cols, uint32_t dtype, int workers);

/* engine/speculative.go:263-271 argmaxLogit: first strict maximum wins; a NaN
 * at index 0 stays selected. Pinned by brute force and the ordering rules. */
int32_t orc_argmax(const float *logits, int64_t n);

/* engine/speculative.go:39-66 lookupDraft. Pinned by TestLookupDraft vectors
 * (engine/speculative_test.go:139-151). Returns the draft length. */
int orc_lookup_draft(const int32_t *history, int n_history, int max_draft,
                     int min_match, int32_t *out);

/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11). Pinned against the
 * published known-answer vectors of the Random123 distribution and against
 * rocRAND's open-source rocrand_philox4x32_10.h. Not part of the reference. */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
/* 53-bit uniform in [0,1) from two 32-bit words (hi, lo). */
double orc_u01(uint32_t hi, uint32_t lo);

/* Target distribution of engine/sampling.go:60-129 (Sampler.Sample):
 * drop -Inf/NaN, order by (logit desc, id asc), keep top_k (>0), weights
 * exp(float64(logit-max)/T), top_p < 1 keeps the smallest sorted prefix whose
 * normalized cumulative mass reaches top_p, then renormalizes.
 * Writes the UNNORMALIZED weight of every vocab entry into w (0 for dropped
 * entries), returns the kept total through *total and the argmax through
 * *best. Returns the number of kept entries, 0 when every logit is invalid,
 * and -1 when total is 0 or Inf (the reference then returns candidates[0]).
 * Pinned by sampling_test.go:8-36 (greedy / top-k=1), V=1 (ExampleSampler),
 * and brute-force distribution checks. */
int64_t orc_target_weights(const float *logits, int64_t n, float temperature,
                           int top_k, float top_p, double *w, double *total,
                           int32_t *best);

/* Greedy verify-accept over M = k+1 rows of logits (row i holds the target
 * distribution for draft i, row k the bonus row). Restates the accept loop of
 * engine/speculative.go:191-208 with argmaxLogit per row. Outputs:
 *   *accepted in 0..k and *next = argmax(row accepted) (the correction when
 *   accepted < k, else the token the next step would emit).
 * row_argmax (optional, M entries) receives the per-row argmax. */
void orc_accept_greedy(const float *logits, int64_t vocab, int k, const int32_t *drafts,
                       int *accepted, int32_t *next, int32_t *row_argmax);

/* Stochastic verify-accept: speculative sampling (Leviathan et al. 2023,
 * Chen et al. 2023) with a one-hot draft distribution. Parity unpinned against
 * the reference (the reference has no stochastic speculative mode); defined in
 * this repository. For draft i: p = target(row i); u = philox(seed; step, i,
 * request, 0); accept iff u < p(d_i). First rejection at i: resample from p
 * with d_i removed (inverse CDF in index order, u2 = philox(seed; step, i,
 * request, 1)). All accepted: sample the bonus from row k the same way with
 * nothing removed. Per-row debug: p_draft[i], u[i] (optional). */
void orc_accept_stochastic(const float *logits, int64_t vocab, int k, const int32_t *drafts,
                           float temperature, int top_k, float top_p, uint64_t seed,
                           uint64_t step, uint32_t request, int *accepted, int32_t *next,
                           double *p_draft, double *u_accept);

/* Uniform draw for (seed; step, row, request, purpose). */
double orc_draw(uint64_t seed, uint64_t step, uint32_t row, uint32_t request, uint32_t purpose);

#ifdef __cplusplus
}
#endif

#endif
