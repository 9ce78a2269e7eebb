// k_fgemm.hip — fused verify GEMM kernels and launchers (device code in
// fgemm_dev.h).
#include "fgemm_dev.h"

namespace yk {
namespace {

// Streaming kernel: a separate instantiation per (dtype, tiles, activation
// units per wave, prologue mode) so that it carries none of the chunked
// path's registers or scratch.
template <int DT, int TT, int KU, int MODE, bool BAL>
__global__ __launch_bounds__(kThreads) void fgemm_stream_kernel(const FusedGemmArgs A) {
    extern __shared__ __align__(16) uint8_t lds[];
    const bool swiglu = A.epilogue == kEpiSwiglu;
    const int rows_out = swiglu ? 8 * TT : 16 * TT;
    const int nsb = A.K / 256;
    const ActLayout L0(A.rows, 1, nsb, nsb, MODE == 1, -1, MODE == 2, false);
    float *inv_w = reinterpret_cast<float *>(lds + L0.total);
    float *red = reinterpret_cast<float *>(lds + L0.total + kInvBytes);
    stream_groups<DT, TT, KU, MODE, BAL>(A, lds, inv_w, red, rows_out, swiglu);
}

template <int DTM, int TT, int NA>
__global__ __launch_bounds__(kThreads) void fgemm_kernel(const FusedGemmArgs A) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const bool swiglu = A.epilogue == kEpiSwiglu;
    const int rows_out = swiglu ? 8 * TT : 16 * TT;  // output rows of one group
    const int nsb = A.K / 256;
    const int M = A.rows;
    const ActLayout L0(M, NA, min(A.chunk_sb, nsb), nsb, A.norm != nullptr, -1, A.gate != nullptr);
    const bool one_chunk = A.chunk_sb >= nsb;  // activations stay in LDS across groups
    float *inv_rms = reinterpret_cast<float *>(lds + L0.total);
    float *red = reinterpret_cast<float *>(lds + L0.total + kInvBytes);
    for (int grp = blockIdx.x; grp < A.groups; grp += gridDim.x) {
        const GroupRows<TT> G(A, grp, rows_out, swiglu, r);
        float acc[TT][NA][4];
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int a = 0; a < NA; a++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[t][a][i] = 0.0f;
        const bool first = grp == (int)blockIdx.x;
        for (int c0 = 0; c0 < nsb; c0 += A.chunk_sb) {
            const ActLayout L(M, NA, min(A.chunk_sb, nsb), nsb, A.norm != nullptr, min(A.chunk_sb, nsb - c0),
                              A.gate != nullptr);
            const bool pro = first || !one_chunk;
            if (c0 && pro) lds_barrier();  // previous chunk's LDS reads are done
            if constexpr (DTM != 0) chunk_pass<DTM, TT, NA>(A, L, lds, c0, nsb, G.rs, G.row_off, acc, pro);
            else if (G.dt == kQ4K) chunk_pass<kQ4K, TT, NA>(A, L, lds, c0, nsb, G.rs, G.row_off, acc, pro);
            else chunk_pass<kQ6K, TT, NA>(A, L, lds, c0, nsb, G.rs, G.row_off, acc, pro);
        }
        if (first) {
            lds_barrier();
            compute_inv_rms(A, L0, lds, inv_rms, nsb);
        }
        group_epilogue<TT, NA>(A, red, inv_rms, acc, G.n0, G.N, G.s, rows_out, swiglu);
    }
}

}  // namespace

uint32_t fused_gemm_lds_bytes(int rows, int K, int chunk_sb, int tt, bool norm, bool gated) {
    const int na = rows <= 8 ? 1 : 2;
    const int nsb = K / 256;
    const ActLayout L(rows, na, std::min(chunk_sb, nsb), nsb, norm, -1, gated);
    return L.total + kInvBytes + (uint32_t)kWaves * tt * na * 4 * 64 * 4;
}

int fused_gemm_chunk_sb(int rows, int K, int tt, bool norm, bool gated) {
    const int nsb = K / 256;
    for (int c = nsb; c >= 1; c--)
        if (fused_gemm_lds_bytes(rows, K, c, tt, norm, gated) <= kFusedLds) return c;
    return 0;
}


// Streaming launch: every resident workgroup gets floor or ceil of G / R row
// tiles. Ring mode: the waves split into the row-group x K-group shape that
// minimizes the largest per-wave item count (ties: more row groups), among
// the shapes whose per-tile partials fit LDS (one slot per wave and tile of
// its row group).
template <int DT, int TT, int KU, int MODE, bool BAL>
static hipError_t launch_stream1(const FusedGemmArgs &a, uint32_t lds, hipStream_t s) {
    auto k = fgemm_stream_kernel<DT, TT, KU, MODE, BAL>;
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr = true;
    }
    FusedGemmArgs b = a;
    // one workgroup per CU: a second one would quantize the same activations
    // again on the same CU
    const unsigned res = std::min(resident_wgs(reinterpret_cast<const void *>(k), lds), (unsigned)device_cus());
    const int nsb = b.K / 256;
    const unsigned R = std::min((unsigned)b.groups, res);
    const int per_wg = (int)((b.groups + R - 1) / R);
    b.wk = 0;
    if (!BAL) {
        const uint32_t slot = (uint32_t)kWaves * TT * 4 * 64 * 4;  // one partial per wave
        const uint32_t base = lds - slot;
        int best = 1 << 30;
        uint32_t best_lds = 0;
        for (int wr = 1; wr <= kWaves; wr *= 2) {
            const int wk = kWaves / wr;
            const int niter = (per_wg + wr - 1) / wr;
            const uint32_t need = base + slot * (uint32_t)niter;
            const int items = niter * ((nsb + wk - 1) / wk);
            if (need <= kFusedLds && items <= best) {
                best = items;
                b.wk = wk;
                best_lds = need;
            }
        }
        if (!b.wk) return hipErrorInvalidValue;  // no shape fits LDS
        lds = best_lds;
    }
    k<<<R, kThreads, lds, s>>>(b);
    return hipGetLastError();
}

template <int DT, int TT, int KU, int MODE>
static hipError_t launch_stream(const FusedGemmArgs &a, uint32_t lds, bool balanced, hipStream_t s) {
    return balanced ? launch_stream1<DT, TT, KU, MODE, true>(a, lds, s) : launch_stream1<DT, TT, KU, MODE, false>(a, lds, s);
}

template <int DT, int TT>
static hipError_t launch_stream_ku(const FusedGemmArgs &a, int ku, int mode, uint32_t lds, bool bal, hipStream_t s) {
    if (mode == 2) return launch_stream<DT, TT, 8, 2>(a, lds, bal, s);
    if (mode == 1) return ku <= 8 ? launch_stream<DT, TT, 8, 1>(a, lds, bal, s) : launch_stream<DT, TT, 16, 1>(a, lds, bal, s);
    if (ku <= 8) return launch_stream<DT, TT, 8, 0>(a, lds, bal, s);
    if (ku <= 16) return launch_stream<DT, TT, 16, 0>(a, lds, bal, s);
    return launch_stream<DT, TT, 24, 0>(a, lds, bal, s);
}

// Largest row count the streaming kernel serves for this K and prologue
// (its activation units per wave stay within the register budget).
int fused_gemm_stream_rows(int K, bool norm, bool gated) {
    const int nsb = K / 256;
    if (nsb < 1) return 0;
    const int cap = gated ? 8 : (norm ? 16 : 24);
    return std::min(8, cap * kWaves / nsb);
}


template <int DTM, int TT, int NA>
static hipError_t launch_tt(const FusedGemmArgs &a, unsigned grid, uint32_t lds, hipStream_t s) {
    FusedGemmArgs b = a;
    b.wk = kWaves;
    auto k = fgemm_kernel<DTM, TT, NA>;
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr = true;
    }
    const unsigned res = resident_wgs(reinterpret_cast<const void *>(k), lds);
    grid = std::min(grid, res);
    k<<<grid, kThreads, lds, s>>>(b);
    return hipGetLastError();
}

template <int DTM>
static hipError_t launch_dt(const FusedGemmArgs &a, int tt, unsigned grid, uint32_t lds, hipStream_t s) {
    const bool na1 = a.rows <= 8;
    switch (tt) {
    case 1: return na1 ? launch_tt<DTM, 1, 1>(a, grid, lds, s) : launch_tt<DTM, 1, 2>(a, grid, lds, s);
    case 2: return na1 ? launch_tt<DTM, 2, 1>(a, grid, lds, s) : launch_tt<DTM, 2, 2>(a, grid, lds, s);
    case 4:
        if constexpr (DTM == kQ4K) return na1 ? launch_tt<DTM, 4, 1>(a, grid, lds, s) : launch_tt<DTM, 4, 2>(a, grid, lds, s);
        return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}



hipError_t launch_fused_gemm(const FusedGemmArgs &a, int tt, hipStream_t s) {
    unsigned grid = 0;
    const FusedGemmArgs b = with_groups(a, tt, &grid);
    // Launches run persistent group loops over at most the resident
    // workgroups; each workgroup quantizes the activations once.
    bool mixed = false;
    for (int i = 1; i < b.nseg; i++) mixed |= b.seg[i].dtype != b.seg[0].dtype;
    int ku = 0, mode = 0;
    uint32_t slds = 0;
    bool bal = false;
    if (stream_shape(b, tt, mixed, &ku, &mode, &slds, &bal)) {
        if (mixed) return launch_stream_ku<0, 1>(b, ku, mode, slds, bal, s);
        if (b.seg[0].dtype == kQ4K)
            return tt == 1 ? launch_stream_ku<kQ4K, 1>(b, ku, mode, slds, bal, s)
                           : launch_stream_ku<kQ4K, 2>(b, ku, mode, slds, bal, s);
        return launch_stream_ku<kQ6K, 1>(b, ku, mode, slds, bal, s);
    }
    const uint32_t lds = fused_gemm_lds_bytes(b.rows, b.K, b.chunk_sb, tt, b.norm != nullptr, b.gate != nullptr);
    if (mixed) return launch_dt<0>(b, tt, grid, lds, s);
    if (b.seg[0].dtype == kQ4K) return launch_dt<kQ4K>(b, tt, grid, lds, s);
    return launch_dt<kQ6K>(b, tt, grid, lds, s);
}

}  // namespace yk
