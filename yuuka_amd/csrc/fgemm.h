// fgemm.h — fused verify GEMM (k_fgemm.hip): argument block and launcher.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/yuuka_hip.h"

namespace yk {

constexpr int kFusedMaxSeg = 4;
constexpr int kFusedWaves = 8;                   // waves per workgroup (they split K)
constexpr uint32_t kFusedLds = 160 * 1024;       // LDS per workgroup on gfx950

enum FusedEpilogue : int {
    kEpiStore = 0,     // out = y W^T
    kEpiResidual = 1,  // out = y W^T + res (res may alias out)
    kEpiSwiglu = 2,    // seg0.out = SiLU(y W0^T) * (y W1^T); segments 0, 1 same shape
};

struct FusedSeg {
    const void *w;       // packed rows (Q4_K or Q6_K)
    uint32_t w_bytes;    // bytes of the packed matrix (loads past it read 0)
    uint32_t row_bytes;  // bytes of one packed row
    int n;               // output rows
    int dtype;
    float *out;          // [rows][n]
    const float *res;    // [rows][n] (kEpiResidual)
    int wg_begin;        // first workgroup (set by the launcher)
    int act;             // kEpiStore output map: 0 none, 1 SiLU, 2 sigmoid, 3 Gated DeltaNet decay
                         // exp(softplus(v + p0[n]) * p1[n]) (recurrent.go:66-70)
    const float *p0, *p1;  // per-row parameters of act 3 (dt, a)
};

struct FusedGemmArgs {
    const float *x;     // [rows][K] activations
    const float *norm;  // optional RMSNorm weight [K]
    // Optional gated head norm (Gated DeltaNet output, recurrent.go:39-50):
    // y = RMSNorm_head(x) * head_norm * gate over heads of 128 elements, with
    // gate = SiLU(z) already applied by its producer. Excludes `norm`.
    const float *gate;       // [rows][K]
    const float *head_norm;  // [128]
    float eps;
    int K, rows;
    int chunk_sb;       // super-blocks of K quantized into LDS at a time
    int epilogue;       // FusedEpilogue
    int nseg;
    int groups;         // row tiles (16*tt rows) over all segments (set by the launcher)
    int wk;             // streaming path: waves splitting K (1, 2, 4 or 8), 0 = items dealt to waves one by one (set by the launcher)
    FusedSeg seg[kFusedMaxSeg];
};

// Largest K chunk (in 256-element super-blocks) whose activations fit LDS
// next to the partial-sum area of a tt-tile launch (0 if none fits).
int fused_gemm_chunk_sb(int rows, int K, int tt, bool norm, bool gated = false);
uint32_t fused_gemm_lds_bytes(int rows, int K, int chunk_sb, int tt, bool norm, bool gated = false);
// Largest row count the streaming kernel (one launch per layer projection
// at verify shapes) serves for this K; larger row counts take the chunked
// kernel. 0 when K has no super-block.
int fused_gemm_stream_rows(int K, bool norm, bool gated);
// Verify GEMM over many rows (k_bgemm.hip): same arguments and results for
// rows 9..512 (K <= 16384), reading every weight once per block of 48 or 80
// rows; `ws` holds fused_gemm_rows_ws(rows, K, total output channels) bytes
// (the quantized activations and split-K partial sums).
uint64_t fused_gemm_rows_ws(int rows, int K, const int *n, int nseg, bool swiglu);
hipError_t launch_fused_gemm_rows(const FusedGemmArgs &a, void *ws, hipStream_t s);
// A run of many-row GEMMs (rows > 8) launched in turn. Where g[i] splits K
// and g[i + 1] normalises g[i]'s residual output, or reads g[i]'s SwiGLU
// output as it is, g[i]'s split reduction runs inside g[i + 1]'s prologue
// (bit-identical to the separate reduce). Every member's quantized rows sit
// at the start of ws and its partial sums at part_off (at least the largest
// member's quantized rows). defer_last: when the last member is a split
// residual GEMM its reduction is left to the caller (*last).
struct BgDeferred {
    bool on;
    const float *part;  // [splits][rows][n]
    uint64_t sstride;
    int splits;
};
hipError_t launch_fused_gemm_rows_chain(const FusedGemmArgs *g, int n, void *ws, uint64_t part_off, bool defer_last,
                                        hipStream_t s, BgDeferred *last);
// Workspace of launch_fused_gemm_rows in two parts: quantized rows, partial sums.
void fused_gemm_rows_ws_parts(int rows, int K, const int *n, int nseg, bool swiglu, uint64_t *quant, uint64_t *part);
// tt: 16-row tiles per workgroup (1, 2 or 4; even for kEpiSwiglu).
hipError_t launch_fused_gemm(const FusedGemmArgs &a, int tt, hipStream_t s);

}  // namespace yk
