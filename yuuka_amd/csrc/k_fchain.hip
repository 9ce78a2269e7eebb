// k_fchain.hip — chained streaming verify GEMMs: a run of dependent
// projections of one layer (out-projection, FFN gate/up, FFN down, next
// in-projection or the LM head) as one persistent launch instead of one
// launch per projection.
//
// Every stage is the streaming GEMM of fgemm_dev.h (the same arithmetic as
// the plain launch, so the results are bit-identical). One workgroup per CU;
// stage s + 1 requests its first weight items, then waits until every
// workgroup has counted stage s as stored, then loads its activations. So a
// stage's HBM latency and wave start overlap the previous stage's tail
// instead of following a kernel boundary. Activations, residuals and outputs
// of a chain stage are accessed at device scope (sc1), so the XCDs' L2
// caches need no write-back or invalidation between stages.
//
// Replaces, for the verify step, the per-projection launches of the
// reference plan (engine/gpu/plan.go:569-682 via bridge.cpp:3453-3870).
#include "fgemm_dev.h"

namespace yk {
namespace {

// Streaming shapes a chained launch serves: (dtype, tiles, activation units
// per wave, prologue mode, balanced). A GEMM of another shape is launched on
// its own.
struct ChainVariant {
    int dt, tt, ku, mode;
    bool bal;
};
constexpr ChainVariant kChainVariants[] = {
    {kQ4K, 1, 8, 1, true},    // 0: Gated DeltaNet in-projection (RMSNorm)
    {kQ4K, 1, 8, 2, true},    // 1: Gated DeltaNet out-projection (gated head norm)
    {kQ4K, 2, 8, 1, true},    // 2: FFN gate/up (SwiGLU)
    {kQ4K, 1, 24, 0, true},   // 3: FFN down
    {kQ4K, 1, 16, 0, true},   // 4: attention out-projection
    {0, 1, 8, 1, true},       // 5: attention in-projection (Q4_K q, k + Q6_K v)
    {kQ6K, 1, 8, 1, false},   // 6: LM head (ring mode)
};
constexpr int kNumChainVariants = (int)(sizeof(kChainVariants) / sizeof(kChainVariants[0]));

struct ChainArgs {
    FusedGemmArgs a[kFusedChainMax];
    uint32_t *sync;
};

template <int I>
__device__ __forceinline__ void chain_stage(const FusedGemmArgs &A, uint8_t *lds, const ChainCtl &ctl) {
    constexpr ChainVariant V = kChainVariants[I];
    const bool swiglu = A.epilogue == kEpiSwiglu;
    const int rows_out = swiglu ? 8 * V.tt : 16 * V.tt;
    const int nsb = A.K / 256;
    const ActLayout L0(A.rows, 1, nsb, nsb, V.mode == 1, -1, V.mode == 2, false);
    float *inv_w = reinterpret_cast<float *>(lds + L0.total);
    float *red = reinterpret_cast<float *>(lds + L0.total + kInvBytes);
    stream_groups<V.dt, V.tt, V.ku, V.mode, V.bal, 1>(A, lds, inv_w, red, rows_out, swiglu, ctl);
}

// Counts this workgroup's stage s as stored: every wave's device-scope
// stores are complete before the count.
__device__ __forceinline__ void chain_signal(uint32_t *ctr) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (threadIdx.x == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// sync[s] counts stage s; sync[kFusedChainMax] counts finished workgroups
// (the last one resets every counter for the next launch, when every
// workgroup is past every wait); sync[kFusedChainMax + 1] is the error word
// of a wait that gave up.
template <int N, int V0, int V1, int V2, int V3>
__global__ __launch_bounds__(kThreads) void fgemm_chain_kernel(const ChainArgs C) {
    extern __shared__ __align__(16) uint8_t lds[];
    uint32_t *sync = C.sync;
    uint32_t *err = sync + kFusedChainMax + 1;
    chain_stage<V0>(C.a[0], lds, ChainCtl{nullptr, gridDim.x, err});
    if constexpr (N > 1) {
        chain_signal(sync + 0);
        chain_stage<V1>(C.a[1], lds, ChainCtl{sync + 0, gridDim.x, err});
    }
    if constexpr (N > 2) {
        chain_signal(sync + 1);
        chain_stage<V2>(C.a[2], lds, ChainCtl{sync + 1, gridDim.x, err});
    }
    if constexpr (N > 3) {
        chain_signal(sync + 2);
        chain_stage<V3>(C.a[3], lds, ChainCtl{sync + 2, gridDim.x, err});
    }
    if (threadIdx.x == 0) {
        const uint32_t done = __hip_atomic_fetch_add(sync + kFusedChainMax, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done + 1 == gridDim.x) {
            for (int s = 0; s + 1 < N; s++) __hip_atomic_store(sync + s, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(sync + kFusedChainMax, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

using ChainLaunch = hipError_t (*)(const ChainArgs &, uint32_t, hipStream_t);

template <int N, int V0, int V1, int V2, int V3>
hipError_t chain_launch(const ChainArgs &C, uint32_t lds, hipStream_t s) {
    auto k = fgemm_chain_kernel<N, V0, V1, V2, V3>;
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr = true;
    }
    // every workgroup must be resident at once (the stages wait on each other)
    const unsigned cus = (unsigned)device_cus();
    if (resident_wgs(reinterpret_cast<const void *>(k), lds) < cus) return hipErrorInvalidConfiguration;
    k<<<cus, kThreads, lds, s>>>(C);
    return hipGetLastError();
}

// The compositions of the hybrid decoder's verify step: the out-projection
// of a Gated DeltaNet (1) or attention (4) layer, FFN gate/up (2) and down
// (3), then the next layer's in-projection (0 or 5) or the LM head (6).
struct ChainEntry {
    int n, v[kFusedChainMax];
    ChainLaunch fn;
};
const ChainEntry kChains[] = {
    {4, {1, 2, 3, 0}, chain_launch<4, 1, 2, 3, 0>}, {4, {1, 2, 3, 5}, chain_launch<4, 1, 2, 3, 5>},
    {4, {4, 2, 3, 0}, chain_launch<4, 4, 2, 3, 0>}, {4, {4, 2, 3, 5}, chain_launch<4, 4, 2, 3, 5>},
    {4, {1, 2, 3, 6}, chain_launch<4, 1, 2, 3, 6>}, {4, {4, 2, 3, 6}, chain_launch<4, 4, 2, 3, 6>},
};

const ChainEntry *find_chain(const FusedChainStage *st, int n) {
    for (const ChainEntry &e : kChains) {
        if (e.n != n) continue;
        bool ok = true;
        for (int i = 0; i < n; i++) ok &= e.v[i] == st[i].variant;
        if (ok) return &e;
    }
    return nullptr;
}

}  // namespace

bool fused_gemm_chain_stage(const FusedGemmArgs &a, int tt, FusedChainStage *out) {
    unsigned grid = 0;
    FusedGemmArgs b = with_groups(a, tt, &grid);
    bool mixed = false;
    for (int i = 1; i < b.nseg; i++) mixed |= b.seg[i].dtype != b.seg[0].dtype;
    int ku = 0, mode = 0;
    uint32_t slds = 0;
    bool bal = false;
    if (!stream_shape(b, tt, mixed, &ku, &mode, &slds, &bal)) return false;
    const int dt = mixed ? 0 : b.seg[0].dtype;
    // the activation bucket the plain launch instantiates (launch_stream_ku)
    const int kub = mode == 2 ? 8 : (mode == 1 ? (ku <= 8 ? 8 : 16) : (ku <= 8 ? 8 : (ku <= 16 ? 16 : 24)));
    int v = -1;
    for (int i = 0; i < kNumChainVariants; i++) {
        const ChainVariant &c = kChainVariants[i];
        if (c.dt == dt && c.tt == tt && c.ku == kub && c.mode == mode && c.bal == bal) v = i;
    }
    if (v < 0) return false;
    b.wk = 0;
    if (!bal) {  // ring mode: the row-group x K-group shape of the plain launch
        const unsigned R = (unsigned)device_cus();
        const int nsb = b.K / 256;
        const int per_wg = (int)((b.groups + R - 1) / R);
        int best = 1 << 30;
        b.wk = kWaves;
        for (int wr = 1; wr <= kWaves; wr *= 2) {
            const int wk = kWaves / wr;
            const int items = ((per_wg + wr - 1) / wr) * ((nsb + wk - 1) / wk);
            if (items <= best) {
                best = items;
                b.wk = wk;
            }
        }
    }
    out->a = b;
    out->variant = v;
    out->lds = slds;
    return true;
}

bool fused_gemm_chain_supported(const FusedChainStage *st, int n) {
    return n >= 2 && n <= kFusedChainMax && find_chain(st, n) != nullptr;
}

hipError_t launch_fused_gemm_chain(const FusedChainStage *st, int n, uint32_t *sync, hipStream_t s) {
    const ChainEntry *e = n >= 2 && n <= kFusedChainMax && sync ? find_chain(st, n) : nullptr;
    if (!e) return hipErrorInvalidValue;
    ChainArgs C{};
    uint32_t lds = 0;
    for (int i = 0; i < n; i++) {
        C.a[i] = st[i].a;
        lds = std::max(lds, st[i].lds);
    }
    C.sync = sync;
    return e->fn(C, lds, s);
}

}  // namespace yk
