/*
 * yuuka_hip.h — C ABI of the MI355X (gfx950) speculative-verify library.
 *
 * This is a drop-in replacement for the reference bridge header
 * backend/hip/bridge/yuuka_hip.h (ABI version 10). Every v10 type, enum value
 * and entry point keeps its exact name, signature and numeric value so the
 * unchanged Go binding (backend/hip/hip.go, RequiredABI = 10 at hip.go:49)
 * links and runs against libyuuka_hip.so. Citations name the reference
 * declaration each entry replaces (paths relative to the reference tree).
 *
 * Entry points outside the verify hot path (decode GEMVs, rocBLAS/WMMA
 * prefill GEMMs, MoE plan ops, ...) are exported and fail with
 * YUUKA_ERR_UNSUPPORTED and a message, which the Go side maps to
 * hip.ErrUnsupported (hip.go:26,348-363) and already falls back from.
 *
 * The extension block at the end (YUUKA_EXT_*) is additive: new symbols, new
 * op codes >= 64, and no change to any v10 layout.
 *
 * Conventions kept from the reference:
 *  - every call returns yuuka_status; the message of the last failure on the
 *    calling thread is yuuka_last_error() (reference :51-52);
 *  - no C++ exception crosses the ABI;
 *  - the caller owns every handle and frees it exactly once (reference :54-63);
 *  - a rejected plan op is not appended (reference :330-334).
 */
#ifndef YUUKA_HIP_H
#define YUUKA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference yuuka_hip.h:11 */
#define YUUKA_HIP_ABI_VERSION 10

#if defined(__GNUC__)
#define YUUKA_API __attribute__((visibility("default")))
#else
#define YUUKA_API
#endif

/* Opaque handles (reference :22-25). */
typedef struct yuuka_device yuuka_device;
typedef struct yuuka_buffer yuuka_buffer;
typedef struct yuuka_stream yuuka_stream;
typedef struct yuuka_event yuuka_event;

/* reference :27-34 */
typedef enum yuuka_status {
    YUUKA_OK = 0,
    YUUKA_ERR_INVALID_ARGUMENT = 1,
    YUUKA_ERR_UNSUPPORTED = 2,
    YUUKA_ERR_DEVICE = 3,
    YUUKA_ERR_ALLOCATION = 4,
    YUUKA_ERR_INTERNAL = 5
} yuuka_status;

/* reference :36-46 */
typedef struct yuuka_device_info {
    char name[256];
    char gcn_arch[64];
    char hip_version[64];
    uint64_t total_memory;
    uint32_t compute_units;
    uint32_t clock_mhz;
    int32_t pci_domain;
    int32_t pci_bus;
    int32_t pci_device;
} yuuka_device_info;

/* reference :48-49. Returns 10: the v10 contract is honoured in full. */
YUUKA_API uint32_t yuuka_abi_version(void);
/* reference :51-52. Thread-local; valid until the next failing call. */
YUUKA_API const char * yuuka_last_error(void);

/* reference :54-57 */
YUUKA_API yuuka_status yuuka_device_open(int32_t index, yuuka_device ** out);
YUUKA_API void yuuka_device_close(yuuka_device * dev);
YUUKA_API yuuka_status yuuka_device_info_get(const yuuka_device * dev, yuuka_device_info * info);

/* reference :59-63 */
YUUKA_API yuuka_status yuuka_buffer_alloc(yuuka_device * dev, uint64_t bytes, yuuka_buffer ** out);
YUUKA_API void yuuka_buffer_free(yuuka_buffer * buf);
YUUKA_API uint64_t yuuka_buffer_size(const yuuka_buffer * buf);
YUUKA_API void * yuuka_buffer_ptr(const yuuka_buffer * buf);

/* reference :65-71 */
YUUKA_API yuuka_status yuuka_stream_create(yuuka_device * dev, yuuka_stream ** out);
YUUKA_API void yuuka_stream_destroy(yuuka_stream * stream);
YUUKA_API yuuka_status yuuka_stream_synchronize(yuuka_stream * stream);
YUUKA_API yuuka_status yuuka_event_create(yuuka_device * dev, yuuka_event ** out);
YUUKA_API void yuuka_event_destroy(yuuka_event * event);
YUUKA_API yuuka_status yuuka_event_wait(yuuka_event * event);

/* reference :73-85 */
YUUKA_API yuuka_status yuuka_memcpy_h2d(yuuka_buffer * dst, const void * src, uint64_t bytes);
YUUKA_API yuuka_status yuuka_memcpy_d2h(void * dst, const yuuka_buffer * src, uint64_t bytes);
YUUKA_API yuuka_status yuuka_memcpy_d2h_at(void * dst, const yuuka_buffer * src,
                                           uint64_t offset, uint64_t bytes);
YUUKA_API yuuka_status yuuka_memset(yuuka_stream * stream, yuuka_buffer * dst, int value, uint64_t bytes);

/* reference :87-90 */
YUUKA_API yuuka_status yuuka_buffer_copy(yuuka_stream * stream,
                                yuuka_buffer * dst, uint64_t dst_offset,
                                const yuuka_buffer * src, uint64_t src_offset,
                                uint64_t bytes, yuuka_event * completion);

/* reference :92-95 */
YUUKA_API yuuka_status yuuka_dynamic_set(yuuka_stream * stream, yuuka_buffer * dynamic,
                                int32_t token, uint32_t position);

/* reference :97-100 */
YUUKA_API yuuka_status yuuka_add_f32(yuuka_stream * stream, yuuka_buffer * dst,
                           const yuuka_buffer * a, const yuuka_buffer * b,
                           uint64_t n, yuuka_event * completion);

/* Operation codes of the plan API (reference :104-149). */
typedef enum yuuka_op_code {
    YUUKA_OP_GEMV = 1,
    YUUKA_OP_RMSNORM = 2,
    YUUKA_OP_L2NORM = 3,
    YUUKA_OP_GATED_RMSNORM = 4,
    YUUKA_OP_ROPE = 5,
    YUUKA_OP_ATTENTION = 6,
    YUUKA_OP_CONV1D = 7,
    YUUKA_OP_GDN = 8,
    YUUKA_OP_SILU_MUL = 9,
    YUUKA_OP_ADD = 10,
    YUUKA_OP_COPY = 11,
    YUUKA_OP_SCALE = 12,
    YUUKA_OP_EMBEDDING = 13,
    YUUKA_OP_KV_WRITE = 14,
    YUUKA_OP_RMSNORM_HEADS = 15,
    YUUKA_OP_GEMM = 16,
    YUUKA_OP_GEMV_BATCH = 17,
    YUUKA_OP_RMSNORM_BATCH = 18,
    YUUKA_OP_RMSNORM_HEADS_BATCH = 19,
    YUUKA_OP_ROPE_BATCH = 20,
    YUUKA_OP_KV_WRITE_BATCH = 21,
    YUUKA_OP_ATTENTION_PREFILL = 22,
    YUUKA_OP_RECURRENT_CHUNK = 23,
    YUUKA_OP_EMBEDDING_BATCH = 24,
    YUUKA_OP_CAST_F16 = 25,
    YUUKA_OP_KV_WRITE_PAGED = 26,
    YUUKA_OP_ATTENTION_PAGED = 27,
    YUUKA_OP_KV_WRITE_BATCH_PAGED = 28,
    YUUKA_OP_ATTENTION_PREFILL_PAGED = 29,
    YUUKA_OP_MOE_ROUTE = 30,
    YUUKA_OP_MOE_GATE_UP = 31,
    YUUKA_OP_MOE_DOWN = 32,
    YUUKA_OP_MOE_REDUCE_ADD = 33,
    YUUKA_OP_GEMM_SWIGLU = 34,
    YUUKA_OP_DEQUANT_F16 = 35,
    YUUKA_OP_QUANT_Q8_1 = 36,
    YUUKA_OP_LM_HEAD = 37,
    YUUKA_OP_GEMV_Q8_1 = 38,
    YUUKA_OP_RECURRENT_TOKEN = 39,
    YUUKA_OP_CONV_L2NORM = 40,
    YUUKA_OP_GEMV_RESIDUAL = 41,
    YUUKA_OP_GEMV_PAIR = 42,
    YUUKA_OP_SILU_MUL_QUANT_Q8_1 = 43,
    YUUKA_OP_PREFILL_Q8_0_PAIR = 44
} yuuka_op_code;

/* reference :151-161 */
#define YUUKA_OP_FLAG_TAIL 0x1u
#define YUUKA_OP_FLAG_PREFILL_BLAS 0x2u
#define YUUKA_OP_FLAG_PREFILL_ATTENTION_TILED 0x4u
#define YUUKA_OP_FLAG_PREFILL_SPLIT_MASK 0x18u
#define YUUKA_OP_FLAG_PREFILL_SPLIT_1 0x08u
#define YUUKA_OP_FLAG_PREFILL_SPLIT_2 0x10u
#define YUUKA_OP_FLAG_PREFILL_SPLIT_4 0x18u

/* reference :171-174 */
#define YUUKA_GEMM_PATH_AUTO 0u
#define YUUKA_GEMM_PATH_BLAS 1u
#define YUUKA_GEMM_PATH_WMMA 2u
#define YUUKA_GEMM_PATH_MMQ 3u

/* Plan operation descriptor (reference :185-193). yuuka_plan_add copies it. */
typedef struct yuuka_op {
    uint32_t code;
    uint32_t flags;
    yuuka_buffer * buf[16];
    uint64_t off[16];
    uint64_t n[6];
    uint32_t u[4];
    float f[4];
} yuuka_op;

typedef struct yuuka_plan yuuka_plan;
typedef struct yuuka_graph yuuka_graph;

/* GGUF dtype codes (reference :198-207). */
typedef enum yuuka_dtype {
    YUUKA_DTYPE_F32 = 0,
    YUUKA_DTYPE_F16 = 1,
    YUUKA_DTYPE_Q4_0 = 2,
    YUUKA_DTYPE_Q5_0 = 6,
    YUUKA_DTYPE_Q8_0 = 8,
    YUUKA_DTYPE_Q4_K = 12,
    YUUKA_DTYPE_Q5_K = 13,
    YUUKA_DTYPE_Q6_K = 14
} yuuka_dtype;

/* reference :209-212. Single-row decode GEMV: served by the verify GEMM with
 * one row (Q4_K / Q6_K), else UNSUPPORTED. */
YUUKA_API yuuka_status yuuka_gemv(yuuka_stream * stream, yuuka_buffer * out,
                        const yuuka_buffer * x, const yuuka_buffer * w,
                        uint64_t n_in, uint64_t n_out, uint32_t dtype,
                        yuuka_event * completion);

/* reference :221-224, :235-238, :250-256, :266-270: prefill GEMM routes of
 * the reference (rocBLAS/rocWMMA/MMQ). Out of scope: UNSUPPORTED, except
 * yuuka_quantize_q8_1, the Q8_1 activation format the int8 decode matvec
 * (YUUKA_OP_GEMV_Q8_1) also reads. */
YUUKA_API yuuka_status yuuka_gemm(yuuka_stream * stream, yuuka_buffer * out,
                        const yuuka_buffer * x, const yuuka_buffer * w,
                        uint64_t n_in, uint64_t n_out, uint64_t batch,
                        uint32_t dtype, yuuka_event * completion);
YUUKA_API yuuka_status yuuka_gemm_wmma(yuuka_stream * stream, yuuka_buffer * out,
                        const yuuka_buffer * x, const yuuka_buffer * w,
                        uint64_t n_in, uint64_t n_out, uint64_t batch,
                        uint32_t dtype, yuuka_event * completion);
YUUKA_API yuuka_status yuuka_quantize_q8_1(yuuka_stream * stream, yuuka_buffer * qs,
                        yuuka_buffer * ds, const yuuka_buffer * x,
                        uint64_t n, uint64_t batch, yuuka_event * completion);
YUUKA_API yuuka_status yuuka_gemm_mmq(yuuka_stream * stream, yuuka_buffer * out,
                        const yuuka_buffer * qs, const yuuka_buffer * ds,
                        const yuuka_buffer * w, uint64_t n_in, uint64_t n_out,
                        uint64_t batch, uint32_t dtype, yuuka_event * completion);
YUUKA_API yuuka_status yuuka_gemm_blas(yuuka_stream * stream, yuuka_buffer * out,
                        yuuka_buffer * out16, const yuuka_buffer * x16,
                        const yuuka_buffer * w, uint64_t n_in, uint64_t n_out,
                        uint64_t batch, yuuka_event * completion);

/* The verify GEMM (reference :286-289, kernels/hip/gemm/lm_head.hip:61-173):
 *
 *   out[rows, n_out] = W[n_out, n_in] * x[rows, n_in]
 *
 * x and out are FP32 row-major; W is packed GGUF Q4_K or Q6_K (n_in a
 * multiple of 256). rows is 1..16 as in the reference. Submitted on stream,
 * completion recorded after the last kernel, no host synchronization.
 * Implementation: x is quantized to a 16-bit fixed-point split into two int8
 * planes, and the weights are decoded to int8 in registers and contracted on
 * the gfx950 int8 MFMA units with exact int32 sums per quant sub-block;
 * the K-quant scales are applied in FP32. */
YUUKA_API yuuka_status yuuka_lm_head(yuuka_stream * stream, yuuka_buffer * out,
                        const yuuka_buffer * x, const yuuka_buffer * w,
                        uint64_t n_in, uint64_t n_out, uint64_t rows,
                        uint32_t dtype, yuuka_event * completion);

/* reference :301-304, :308-309: FP16 staging helpers of the rocBLAS route.
 * yuuka_dequant_f16 is served for Q4_K/Q6_K (values rounded to FP16 from the
 * exact FP32 dequantization); the cast is served. */
YUUKA_API yuuka_status yuuka_dequant_f16(yuuka_stream * stream, yuuka_buffer * dst,
                        const yuuka_buffer * src, uint64_t n_in, uint64_t n_out,
                        uint32_t dtype, yuuka_event * completion);
YUUKA_API yuuka_status yuuka_cast_f32_to_f16(yuuka_stream * stream, yuuka_buffer * dst,
                        const yuuka_buffer * src, uint64_t n, yuuka_event * completion);

/* reference :318-321: batched GEMV (batch <= 16). Served by the verify GEMM
 * for Q4_K/Q6_K. */
YUUKA_API yuuka_status yuuka_gemv_batch(yuuka_stream * stream, yuuka_buffer * out,
                        const yuuka_buffer * x, const yuuka_buffer * w,
                        uint64_t n_in, uint64_t n_out, uint64_t batch,
                        uint32_t dtype, yuuka_event * completion);

/* Plan and graph API (reference :477-496). Supported op codes: LM_HEAD,
 * GEMV_BATCH (Q4_K/Q6_K), RMSNORM_BATCH, RMSNORM_HEADS_BATCH, ROPE_BATCH,
 * EMBEDDING_BATCH, KV_WRITE_BATCH_PAGED, ATTENTION_PREFILL_PAGED,
 * RECURRENT_CHUNK, ADD, SILU_MUL, COPY, MOE_ROUTE, MOE_GATE_UP, MOE_DOWN,
 * MOE_REDUCE_ADD (experts in Q4_K), plus the YUUKA_EXT_OP_* codes. The
 * v10 buffer layouts of the reference header (:336-476) are honoured.
 * Other codes are rejected with YUUKA_ERR_UNSUPPORTED and not appended. */
YUUKA_API yuuka_status yuuka_graph_create(yuuka_plan * plan, yuuka_stream * stream,
                                          yuuka_buffer * dynamic, int run_tail,
                                          yuuka_graph ** out);
YUUKA_API yuuka_status yuuka_graph_replay(yuuka_graph * graph, yuuka_stream * stream,
                                          yuuka_event * completion);
YUUKA_API void yuuka_graph_destroy(yuuka_graph * graph);
YUUKA_API yuuka_status yuuka_plan_create(yuuka_device * dev, yuuka_plan ** out);
YUUKA_API void yuuka_plan_destroy(yuuka_plan * plan);
YUUKA_API yuuka_status yuuka_plan_add(yuuka_plan * plan, const yuuka_op * op);
YUUKA_API yuuka_status yuuka_plan_execute(yuuka_plan * plan, yuuka_stream * stream,
                                          int32_t token, uint32_t position,
                                          int run_tail, yuuka_event * completion);
/* reference :493-496 */
YUUKA_API yuuka_status yuuka_plan_execute_profiled(
    yuuka_plan * plan, yuuka_stream * stream, int32_t token, uint32_t position,
    int run_tail, uint32_t * op_codes, uint64_t * op_times_ns,
    uint64_t capacity, uint64_t * op_count, yuuka_event * completion);

/* ======================================================================
 * Extension block. No counterpart in the reference v10 header unless a
 * citation says otherwise; additive only.
 * ====================================================================== */

#define YUUKA_EXT_VERSION 1

/* Version of the extension block compiled into the library. */
YUUKA_API uint32_t yuuka_ext_version(void);

/* Bit-exact FP32 dequantization of a packed matrix:
 *   dst[n_out, n_in] = dequant(W[n_out, n_in])
 * Same values as the reference CPU decoder tensor/quant.go:15-62
 * (DequantizeRow): every multiply and subtract separately rounded. Used to
 * prove the device decoder bit-exact. Q4_K, Q5_K, Q6_K, Q8_0, F16, F32. */
YUUKA_API yuuka_status yuuka_dequant_f32(yuuka_stream * stream, yuuka_buffer * dst,
                        const yuuka_buffer * src, uint64_t n_in, uint64_t n_out,
                        uint32_t dtype, yuuka_event * completion);

/* Acceptance modes of yuuka_verify_accept. */
#define YUUKA_ACCEPT_GREEDY 0u
#define YUUKA_ACCEPT_STOCHASTIC 1u

/* Parameters of one fused verify-accept call (host struct, copied). */
typedef struct yuuka_accept_params {
    uint32_t mode;        /* YUUKA_ACCEPT_* */
    uint32_t batch;       /* requests B >= 1 */
    uint32_t drafts;      /* k >= 0; every request holds k+1 logits rows */
    uint32_t vocab;       /* V */
    float temperature;    /* stochastic: T > 0; <= 0 means greedy target */
    uint32_t top_k;       /* 0 = off */
    float top_p;          /* >= 1 = off */
    uint32_t request_base;/* request index of batch entry 0 (Philox counter) */
    uint64_t seed;        /* Philox4x32-10 key */
    uint64_t step;        /* Philox counter word (verify step) */
    uint64_t row_stride;  /* floats between consecutive logits rows; 0 = V */
} yuuka_accept_params;

/* Fused verify-accept over the logits of one verify step (replaces the host
 * loop of engine/speculative.go:191-208 plus argmaxLogit :263-271; the
 * stochastic mode has no reference counterpart).
 *
 * logits: FP32 [B][k+1][V] (row stride params->row_stride), row i of request
 *         b is the target distribution for draft i, row k the bonus row.
 * drafts: int32 [B][k].
 * result: int32 [B][4] = {accepted in 0..k, next token, argmax of row 0,
 *         reserved}.
 * debug:  optional (may be NULL) FP64 [B][k+1][4] = {p(draft), u, row total,
 *         row max logit}.
 * Greedy: accept draft i iff argmax(row i) == draft i (lowest index among
 * equal maxima; a NaN at index 0 wins, later NaNs never do); next = argmax
 * of the first rejected row, or of row k when every draft is accepted.
 * Stochastic: the target p is the sampler's distribution
 * (engine/sampling.go:60-119): drop NaN and -Inf, order by (logit desc, id
 * asc), keep the first top_k (0 = all), weights exp(float64(logit-max)/T),
 * then keep the smallest prefix whose share reaches top_p (0 or >= 1 = all);
 * sums in float64. Draft i is accepted iff u_i < p(d_i) with
 * u_i = Philox(seed; step, i, request, 0); on the first rejection next is
 * drawn from p with d_i removed, and after full acceptance from row k, by
 * inverse CDF in index order with u = Philox(seed; step, i, request, 1). */
YUUKA_API yuuka_status yuuka_verify_accept(yuuka_stream * stream,
                        const yuuka_buffer * logits, uint64_t logits_offset,
                        const yuuka_buffer * drafts, uint64_t drafts_offset,
                        yuuka_buffer * result, uint64_t result_offset,
                        yuuka_buffer * debug, const yuuka_accept_params * params,
                        yuuka_event * completion);

/* yuuka_verify_accept without any allocation. No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments (no debug buffer) and results as yuuka_verify_accept; its
 * partial results live in one fixed device array per GPU of
 * YUUKA_NOALLOC_SCRATCH_BYTES, set up by yuuka_device_open. Calls whose
 * partials exceed it (yuuka_noalloc_accept_bytes) fail with
 * YUUKA_ERR_INVALID_ARGUMENT before anything is launched: at V = 151936 that
 * is above about 2048 rows (batch x (drafts + 1)). Every call on one GPU
 * shares the array: calls that overlap on one GPU (several streams) race;
 * calls on one stream are ordered. Nothing in the array needs clearing. */
#define YUUKA_NOALLOC_SCRATCH_BYTES (8u << 20)
YUUKA_API uint64_t yuuka_noalloc_accept_bytes(const yuuka_accept_params * params);
YUUKA_API yuuka_status yuuka_verify_accept_noalloc(yuuka_stream * stream,
                        const yuuka_buffer * logits, uint64_t logits_offset,
                        const yuuka_buffer * drafts, uint64_t drafts_offset,
                        yuuka_buffer * result, uint64_t result_offset,
                        const yuuka_accept_params * params, yuuka_event * completion);

/* Extension plan ops (codes >= 64; layouts below).
 *   QUANTIZE_X: buf0 FP32 x, buf1 quantized block (yuuka_quantized_bytes);
 *               n={n_in, rows}
 *   GEMM_Q:     buf0 packed W, buf1 quantized x, buf2 FP32 out, optional
 *               buf3 FP32 residual (out = W x + residual; may alias out);
 *               n={n_in, n_out, rows}; u0 = dtype (Q4_K / Q6_K)
 *   ACCEPT:     buf0 logits, buf1 int32 drafts, buf2 int32 result [batch][4],
 *               optional buf3 FP64 debug, optional buf4 uint64 step counter
 *               (else n[5] is the step); n={batch, drafts, vocab, row_stride,
 *               seed, step}; u0 mode, u1 top_k, u2 request_base, u3 drafts
 *               row stride in int32 (0 = drafts); f0 temperature, f1 top_p
 *               (yuuka_verify_accept semantics). Optional buf5 int32 [batch]
 *               forced acceptance lengths (benchmark configurations that
 *               prescribe the accept length): draft i of request b is
 *               accepted iff i < buf5[b], and next is the mode's token at
 *               the first rejected row (or row k).
 *   GDN_COMMIT: buf0 conv_state, buf1 matrix state, buf2 raw qkv rows,
 *               buf3 conv outputs (RECURRENT_CHUNK buf11), buf4 alpha,
 *               buf5 beta, buf6 dt, buf7 a, buf8 int32 acceptance result;
 *               n={rows, groups, heads, state, conv_dim, inner}; u0 kernel.
 *               Advances both states by result[0] + 1 rows (the accepted
 *               prefix of a RECURRENT_CHUNK run with YUUKA_EXT_FLAG_DEFER).
 *               u1 = requests (0 or 1: one): states, rows and the [u1][4]
 *               results request-major; the same u1 on RECURRENT_CHUNK
 *               (with DEFER and RAW_OUT) scans every request in one launch.
 *   ADVANCE:    buf0 dynamic buffer {token, position}, buf1 int32 result,
 *               optional buf2 uint64 step counter; n0 = rows, u0 = requests
 *               (0 means 1). Request j: position (buf0 + 8 j) += min(result
 *               (buf1 + 16 j)[0] + 1, rows); step += 1 once.
 *   GEMM_FUSED: buf0 FP32 x [rows][n_in], optional buf1 FP32 RMSNorm weight
 *               [n_in] (y = RMSNorm(x) * w, eps f0; else y = x); segments
 *               i = 0..3 (the leading non-null weights): buf2+i packed W_i
 *               (Q4_K or Q6_K, dtype in byte i of u0), buf6+i FP32 out_i
 *               [rows][N_i], buf10+i FP32 residual_i (epilogue 1, may alias
 *               out_i); n={n_in, rows, N_0, N_1, N_2, N_3}; u1 epilogue:
 *               0 out = y W^T, 1 out = y W^T + residual, 2 SwiGLU
 *               out_0 = SiLU(y W_0^T) * (y W_1^T) (two segments, same shape).
 *               rows <= 512: up to 8 rows one launch without workspace;
 *               more rows (batched requests) read each weight once per 64
 *               rows and use plan workspace for the quantized rows.
 *               Optional gated head norm of x (Gated DeltaNet output,
 *               recurrent.go:39-50): buf14 FP32 gate [rows][n_in] (SiLU
 *               already applied), buf15 FP32 head norm weight [128]; y =
 *               RMSNorm over each 128-element head * weight * gate (eps f0);
 *               excludes buf1. u2 bits 4i..4i+3: output map of segment i
 *               (epilogue 0 only): 0 none, 1 SiLU, 2 sigmoid, 3 Gated
 *               DeltaNet decay exp(softplus(v + dt[n]) * a[n]) with buf10+i
 *               holding {dt[N_i], a[N_i]} (recurrent.go:66-70).
 *   ROPE_TABLE: buf0 FP32 {cos, sin} [rows][rot_dim/2] of positions
 *               position + n2 + row; n={rows, rot_dim, displacement,
 *               requests (0: one), rows between requests (OWN_POS pairs)};
 *               f0 base (float64 angles as forward.go:495-514).
 *   ATTN_VERIFY: gated paged attention of the verify rows with the per-head
 *               q/k RMSNorm, RoPE and the KV write folded in: buf0 FP32 raw
 *               q rows [rows][heads][2*head_dim] (q | gate), buf1 raw k rows
 *               [rows][kv_dim], buf2 raw v rows, buf3 K pool, buf4 V pool,
 *               buf5 FP32 out [rows][heads][head_dim], buf6 int32 block
 *               table, buf7 q_norm [head_dim], buf8 k_norm [head_dim],
 *               buf9 ROPE_TABLE output; n={kv_heads, heads, head_dim, kv_dim,
 *               rows, displacement}; u={block_size, capacity, kv dtype (F32 or
 *               F16), rot_dim | requests << 8 | request_rows << 20};
 *               f={scale, eps}. Writes the rows' K/V to the pool at position
 *               + displacement + row. With requests > 1 (and OWN_POS) request
 *               j's rows start request_rows rows after request j-1's, its
 *               block table ceil(capacity / block_size) entries later and its
 *               {token, position} pair 8 bytes later (one launch).
 *   MOE_ROUTER: FP32 router of the MoE FFN (ffn_gate_inp, forward.go:328):
 *               buf0 FP32 y [rows][hidden], buf1 FP32 router weight
 *               [experts][hidden], buf2 FP32 logits [rows][experts];
 *               optional buf3 FP32 shared-expert gate vector [hidden]
 *               (ffn_gate_inp_shexp) with buf4 FP32 [rows] receiving its
 *               dot product (before the sigmoid); n={hidden, experts, rows}.
 *   MOE_COMBINE: MOE_REDUCE_ADD plus the shared expert (forward.go:336-388):
 *               buf0 x [rows][hidden] += sum_slot w * expert_out +
 *               sigmoid(buf4[row]) * buf3[row]; buf1 expert_out
 *               [rows*used][hidden], buf2 weights [rows][used], optional
 *               buf3 shared expert output [rows][hidden] and buf4 its gate
 *               logit [rows]; n={hidden, rows, used}.
 * The v10 MoE ops (MOE_ROUTE, MOE_GATE_UP, MOE_DOWN, MOE_REDUCE_ADD) keep
 * the layouts above; experts are served in Q4_K. The route op fills the
 * assignment bins in (row, slot) order and writes every count, so it needs
 * no memset and is deterministic.
 * YUUKA_EXT_FLAG_DEFER on RECURRENT_CHUNK: compute the outputs of every row
 * but leave both states untouched (verify mode; see GDN_COMMIT). */
#define YUUKA_EXT_OP_QUANTIZE_X 64u
#define YUUKA_EXT_OP_GEMM_Q 65u
#define YUUKA_EXT_OP_ACCEPT 66u
#define YUUKA_EXT_OP_GDN_COMMIT 67u
#define YUUKA_EXT_OP_ADVANCE 68u
#define YUUKA_EXT_OP_GEMM_FUSED 69u
#define YUUKA_EXT_OP_ROPE_TABLE 70u
#define YUUKA_EXT_OP_ATTN_VERIFY 71u
#define YUUKA_EXT_OP_MOE_ROUTER 72u
#define YUUKA_EXT_OP_MOE_COMBINE 73u
/*   ROUTER_NORMAL: synthetic router logits (BASELINE configs[4] states
 *               "router logits N(0,1)"; no counterpart in the reference):
 *               buf0 FP32 logits [rows][experts] are overwritten with i.i.d.
 *               standard normal draws (Box-Muller over Philox4x32-10 keyed by
 *               n2 = seed, counter {step, layer n3, row, pair}); optional buf1
 *               uint64 step counter (0 when null); n={rows, experts, seed,
 *               layer}. */
#define YUUKA_EXT_OP_ROUTER_NORMAL 74u
#define YUUKA_EXT_FLAG_DEFER 0x100u
/* With YUUKA_EXT_FLAG_DEFER: buf10 receives the raw per-head scan outputs;
 * the gated RMSNorm is left to the consumer (GEMM_FUSED gated head norm). */
#define YUUKA_EXT_FLAG_RAW_OUT 0x200u
/* On RECURRENT_CHUNK and GDN_COMMIT: the alpha buffer holds the decay
 * exp(softplus(alpha + dt) * a) and the beta buffer sigmoid(beta) (the
 * GEMM_FUSED output maps 3 and 2 produce them). */
#define YUUKA_EXT_FLAG_GDN_COEF 0x400u
/* On ROPE_TABLE and ATTN_VERIFY: buf15 holds the op's own {token,
 * position} int32 pair (a request of a batched plan) instead of the plan's
 * dynamic buffer. */
#define YUUKA_EXT_FLAG_OWN_POS 0x1000u
/* On MOE_GATE_UP: buf6 receives SiLU(gate) * up (forward.go:348-351) and
 * buf7 is not written (may be null). */
#define YUUKA_EXT_FLAG_MOE_SWIGLU 0x800u
/* On MOE_GATE_UP and MOE_DOWN: the expert matrices are in the packed layout
 * that yuuka_moe_pack_q4k writes (same byte count as the v10 layout). */
#define YUUKA_EXT_FLAG_MOE_PACKED 0x2000u
/* On MOE_GATE_UP and MOE_DOWN: expert index `experts` (the weights hold
 * experts + 1 matrices) is the shared expert, applied to every row as slot
 * `used`: the activation rows of MOE_DOWN and the output rows of both have
 * used + 1 slots. On MOE_COMBINE: the shared expert's output is slot `used`
 * of buf1 (rows of used + 1 slots; buf3 null, buf4 its gate logit). */
#define YUUKA_EXT_FLAG_MOE_SHARED 0x4000u

/* Rewrites expert-stacked Q4_K matrices (the v10 MoE layout, rows of n_in
 * columns, rows % 16 == 0, n_in % 256 == 0) into the packed layout of
 * YUUKA_EXT_FLAG_MOE_PACKED: per 16-row tile and 256-column super-block,
 * 2304 contiguous bytes holding the grouped GEMM's per-lane 16-byte quant
 * pieces and the 16 rows' block headers, so that its weight loads are
 * contiguous. dst and src hold rows * n_in / 256 * 144 bytes each and must
 * not overlap. No counterpart in the reference (its MoE kernels read the
 * GGUF rows directly). */
YUUKA_API yuuka_status yuuka_moe_pack_q4k(yuuka_stream * stream, yuuka_buffer * dst, const yuuka_buffer * src,
                        uint64_t rows, uint64_t n_in, yuuka_event * completion);

/* Timing events (extension): an event created with timing enabled, recorded
 * on a stream, and the elapsed milliseconds between two recorded events. */
YUUKA_API yuuka_status yuuka_event_create_timed(yuuka_device * dev, yuuka_event ** out);
YUUKA_API yuuka_status yuuka_event_record(yuuka_event * event, yuuka_stream * stream);
YUUKA_API yuuka_status yuuka_event_elapsed_ms(yuuka_event * start, yuuka_event * end, float * ms);

/* Split form of the verify GEMM. yuuka_quantize_activations writes the int8
 * planes of x[rows, n_in] (rows <= 16) into xq, which must hold
 * yuuka_quantized_bytes(n_in, rows) bytes; yuuka_gemm_quantized then computes
 * out[rows, n_out] = W * x from them. One quantization can feed every GEMM
 * that reads the same activation (q/k/v, gate/up). Workspace for split-K
 * partial sums comes from the stream. */
YUUKA_API uint64_t yuuka_quantized_bytes(uint64_t n_in, uint64_t rows);
YUUKA_API yuuka_status yuuka_quantize_activations(yuuka_stream * stream, yuuka_buffer * xq,
                        const yuuka_buffer * x, uint64_t n_in, uint64_t rows,
                        yuuka_event * completion);
YUUKA_API yuuka_status yuuka_gemm_quantized(yuuka_stream * stream, yuuka_buffer * out,
                        const yuuka_buffer * xq, const yuuka_buffer * w, uint64_t n_in,
                        uint64_t n_out, uint64_t rows, uint32_t dtype,
                        yuuka_event * completion);

/* ----------------------------------------------------------------------
 * qwen35 verify engine (extension). Host side of the speculative verify
 * path in C++ over the plan API above: the counterpart of the reference's
 * engine/gpu (runtime.go, session.go, plan.go) and engine/speculative.go.
 * Every step is one captured HIP graph: embedding, 32 layers, LM head,
 * fused acceptance, on-device GDN commit of the accepted prefix and
 * position advance; the host only uploads k+1 token ids and reads 16 bytes.
 * ---------------------------------------------------------------------- */
typedef struct yuuka_q35 yuuka_q35;

/* model/qwen35/config.go:18-45 plus session geometry. */
typedef struct yuuka_q35_config {
    int32_t n_layers, hidden, ffn, heads, kv_heads, head_dim, rope_dim, vocab;
    int32_t conv_kernel, state_size, groups, rank, inner, full_interval;
    double rope_base;
    float eps;
    int32_t capacity;    /* tokens of context per request */
    int32_t block_size;  /* paged KV block (16) */
    uint32_t kv_dtype;   /* YUUKA_DTYPE_F16 (reference default) or F32 */
    int32_t max_rows;    /* largest row block of one request in one step (<= 32) */
    int32_t batch;       /* concurrent requests (0 means 1) */
    int32_t kv_blocks;   /* blocks of the KV pool the requests share (0: every
                            request can hold its whole capacity) */
    /* qwen35moe FFN (config.go MoE fields; n_experts 0 = dense FFN) */
    int32_t n_experts, n_experts_used, expert_ffn, shared_ffn;
    /* nonzero: the router logits of every MoE layer are replaced, after the
     * router, by i.i.d. N(0,1) draws seeded with this value and the step
     * counter (ROUTER_NORMAL; the routing of BASELINE configs[4]) */
    uint32_t router_normal_seed;
} yuuka_q35_config;

typedef struct yuuka_q35_tensor {
    const void * data;   /* host bytes in GGUF packing */
    uint64_t rows, cols;
    uint32_t dtype;
    uint32_t pad;
} yuuka_q35_tensor;

/* model/qwen35/load.go:104-212 tensor set of one layer (host pointers). */
typedef struct yuuka_q35_layer_weights {
    const float * attn_norm;
    const float * post_norm;
    yuuka_q35_tensor qkv, gate, out, beta, alpha;
    const float * conv;      /* [conv_dim, kernel] */
    const float * dt;
    const float * a;
    const float * ssm_norm;  /* [state_size] */
    yuuka_q35_tensor q, k, v, o;
    const float * q_norm;
    const float * k_norm;
    yuuka_q35_tensor ffn_gate, ffn_up, ffn_down;
    /* MoE FFN (load.go ffn_gate_inp, ffn_gate_inp_shexp, *_shexp, *_exps):
     * router [experts][hidden] FP32, shared-expert gate vector [hidden],
     * shared expert SwiGLU, experts stacked by rows ([experts*ffn][hidden]
     * for gate/up, [experts*hidden][ffn] for down), Q4_K. */
    yuuka_q35_tensor router;
    const float * shared_gate_vec;
    yuuka_q35_tensor shared_gate, shared_up, shared_down, gate_exps, up_exps, down_exps;
} yuuka_q35_layer_weights;

typedef struct yuuka_q35_weights {
    yuuka_q35_tensor embedding, output;
    const float * output_norm;
    const yuuka_q35_layer_weights * layers;
} yuuka_q35_weights;

/* Acceptance settings of one engine (yuuka_accept_params semantics). */
typedef struct yuuka_q35_accept {
    uint32_t mode;
    float temperature;
    uint32_t top_k;
    float top_p;
    uint64_t seed;
} yuuka_q35_accept;

YUUKA_API yuuka_status yuuka_q35_create(yuuka_device * dev, const yuuka_q35_config * cfg,
                                        const yuuka_q35_weights * weights, yuuka_q35 ** out);
YUUKA_API void yuuka_q35_destroy(yuuka_q35 * q);
/* state.go:174-189: recurrent state cleared, position 0, step counter 0. */
YUUKA_API yuuka_status yuuka_q35_reset(yuuka_q35 * q);
YUUKA_API int32_t yuuka_q35_position(const yuuka_q35 * q);
/* GPU time of the last step's graph (HIP events on the engine stream). */
YUUKA_API float yuuka_q35_last_step_ms(const yuuka_q35 * q);
/* Processes n tokens (session.go:195-242 Prefill); *last_logits (may be
 * NULL) receives the logits of the final token [vocab]. */
YUUKA_API yuuka_status yuuka_q35_prefill(yuuka_q35 * q, const int32_t * tokens, int32_t n,
                                         float * last_logits);
/* One verify step over rows = k+1 tokens {pending, d1..dk}: logits of every
 * row, acceptance on device, commit of the accepted prefix. result[4] =
 * {accepted, next token, argmax row 0, 0}. Graph-captured per row count. */
YUUKA_API yuuka_status yuuka_q35_verify(yuuka_q35 * q, const int32_t * tokens, int32_t rows,
                                        const yuuka_q35_accept * accept, int32_t * result);
/* Copies the logits rows of the last verify or prefill step [rows][vocab]. */
YUUKA_API yuuka_status yuuka_q35_logits(yuuka_q35 * q, float * out, int32_t rows);
/* Per expert of MoE layer `layer`: how many rows of the last step selected
 * it (of the last block of 512 rows when the step had more); counts holds
 * n >= n_experts entries. Every layer's routing is kept, so a caller can
 * tell which expert matrices a step streamed (benchmark accounting; no
 * counterpart in the reference). */
YUUKA_API yuuka_status yuuka_q35_moe_counts(yuuka_q35 * q, int32_t layer, int32_t * counts, int32_t n);
/* state.go:211-263 Snapshot/Restore: all recurrent state (conv then matrix,
 * per recurrent layer, little-endian FP32) and the position. */
YUUKA_API uint64_t yuuka_q35_snapshot_bytes(const yuuka_q35 * q);
YUUKA_API yuuka_status yuuka_q35_snapshot(yuuka_q35 * q, void * out, int32_t * position);
YUUKA_API yuuka_status yuuka_q35_restore(yuuka_q35 * q, const void * data, uint64_t bytes, int32_t position);

/* Batched engine (cfg.batch requests). Each request has its own position,
 * recurrent state and KV block table over a shared pool with reference
 * counts (memory/memory.go Table, memory/prefix.go sharing). The functions
 * above act on request 0. */
YUUKA_API int32_t yuuka_q35_request_position(const yuuka_q35 * q, int32_t request);
/* Clears one request's recurrent state and position and returns its KV
 * blocks to the pool (a block is reused once no table references it). */
YUUKA_API yuuka_status yuuka_q35_reset_request(yuuka_q35 * q, int32_t request);
/* Prefill of one request (yuuka_q35_prefill semantics). */
YUUKA_API yuuka_status yuuka_q35_prefill_request(yuuka_q35 * q, int32_t request, const int32_t * tokens,
                                                 int32_t n, float * last_logits);
/* Prefix sharing: request dst takes request src's prefix (its position,
 * recurrent state and the KV blocks of its full blocks, shared by
 * reference; a partial last block is copied). dst is reset first. */
YUUKA_API yuuka_status yuuka_q35_fork(yuuka_q35 * q, int32_t src, int32_t dst);
/* One step over requests 0..n_req-1 with `rows` tokens each (tokens
 * [n_req][rows]). mode 0: verify (k = rows-1 drafts per request, fused
 * acceptance per request with Philox request index = request, commit of
 * each request's accepted prefix); forced (may be NULL) gives per-request
 * acceptance lengths that replace the accept test (benchmark settings).
 * mode 1: prefill (every row committed). result [n_req][4] as
 * yuuka_q35_verify (mode 1: {rows-1, -1, argmax of the last row... } is
 * not defined; pass NULL). */
YUUKA_API yuuka_status yuuka_q35_step_batch(yuuka_q35 * q, int32_t n_req, const int32_t * tokens, int32_t rows,
                                            int32_t mode, const yuuka_q35_accept * accept,
                                            const int32_t * forced, int32_t * result);

/* engine/speculative.go:13-34 options and :48-49 counters. */
typedef struct yuuka_q35_generate_opts {
    int32_t max_tokens;
    int32_t max_draft;   /* k: drafts verified per step (<= max_rows - 1) */
    int32_t min_match;   /* prompt-lookup suffix length (lookupDraft) */
    int32_t stop_token;  /* < 0: none */
    yuuka_q35_accept accept;
} yuuka_q35_generate_opts;

typedef struct yuuka_q35_generate_stats {
    int32_t output_tokens;
    int32_t steps;
    int32_t draft_tokens;
    int32_t accepted_draft;
    double prefill_ms;
    double decode_ms;
} yuuka_q35_generate_stats;

/* engine/speculative.go:68-261 generateSpeculative over this engine: prompt
 * prefill, then per step prompt-lookup drafts (lookupDraft, padded to k with
 * the pending token so every step verifies k+1 rows), one yuuka_q35_verify,
 * emit accepted drafts and the correction/bonus token. out_tokens holds at
 * least max_tokens entries. */
YUUKA_API yuuka_status yuuka_q35_generate(yuuka_q35 * q, const int32_t * prompt, int32_t n_prompt,
                                          const yuuka_q35_generate_opts * opts, int32_t * out_tokens,
                                          yuuka_q35_generate_stats * stats);

#ifdef __cplusplus
}
#endif

#endif
