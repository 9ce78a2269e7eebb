// k_accept.hip — fused verify-accept over the k+1 logits rows of one verify
// step, batched over requests.
//
// Greedy mode restates the accept loop of engine/speculative.go:191-208 with
// argmaxLogit (:263-271): draft i is accepted iff the first maximum of row i
// equals it. Stochastic mode is speculative sampling with a one-hot draft
// (no reference counterpart): accept iff u < p(d), else resample from p with
// d removed; the target p follows engine/sampling.go:60-119 (drop NaN/-Inf,
// top-k in (logit desc, id asc) order, weights exp(float64(logit - max) / T),
// top-p smallest prefix).
//
// Kernels (the passes over a row are separate launches so that the exact row
// maximum is known before any exponential is taken):
//   1. stats:    per (request, row, chunk): maximum and its first index.
//   2. select:   (top-k / top-p only) one workgroup per row finds the row's
//                cut by radix selection over the order key of the logits.
//   3. weights:  (stochastic) per chunk: float64 sum of the kept weights with
//                the draft removed, and the draft's own weight.
//   4. finalize: one workgroup per request walks the rows in order, decides,
//                and for a rejection or the bonus row draws by inverse CDF
//                in index order (chunk prefix, then a scan inside the chunk).
#include <hip/hip_runtime.h>

#include <climits>

#include "internal.h"

namespace yk {
namespace {

struct Stat {
    float v;
    int i;
};

// a beats b: larger value, or equal value and lower index. NaN never wins.
__device__ __forceinline__ bool beats(float av, int ai, float bv, int bi) {
    return av > bv || (av == bv && ai < bi);
}

struct Geo {
    int B, R, k, V, C, L;
    uint64_t stride;
    int ds;  // int32 elements between consecutive requests' drafts
};

__device__ __forceinline__ const float *row_ptr(const float *logits, const Geo &g, int b, int row) {
    return logits + ((uint64_t)b * g.R + row) * g.stride;
}

// Per (request, row, chunk) maximum. A chunk of L (a multiple of 4) logits
// is read by `wpc` waves (1: four chunks per workgroup, for short chunks;
// 4: one chunk per workgroup), with 16-byte loads when the rows are 16-byte
// aligned. The maximum under `beats` does not depend on the order in which
// elements are visited, so the split does not change the result.
__global__ __launch_bounds__(256) void accept_stats_kernel(const float *__restrict__ logits, Geo g,
                                                           Stat *__restrict__ stats, int vec, int wpc) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = blockIdx.x * (4 / wpc) + wave / wpc, row = blockIdx.y, b = blockIdx.z;
    const int t = (wave % wpc) * 64 + lane, nt = wpc * 64;
    const bool live = c < g.C;
    float bv = -INFINITY;
    int bi = INT_MAX;
    if (live) {
        const float *p = row_ptr(logits, g, b, row);
        const int begin = c * g.L;
        const int end = min(begin + g.L, g.V);
        if (vec) {
            const int end4 = begin + ((end - begin) & ~3);
            auto take4 = [&](const float4 v, int j) {
                if (beats(v.x, j, bv, bi)) { bv = v.x; bi = j; }
                if (beats(v.y, j + 1, bv, bi)) { bv = v.y; bi = j + 1; }
                if (beats(v.z, j + 2, bv, bi)) { bv = v.z; bi = j + 2; }
                if (beats(v.w, j + 3, bv, bi)) { bv = v.w; bi = j + 3; }
            };
            int j = begin + t * 4;
            // four 16-byte loads in flight per thread
            for (; j + 3 * nt * 4 < end4; j += 4 * nt * 4) {
                float4 v[4];
#pragma unroll
                for (int u = 0; u < 4; u++) v[u] = *reinterpret_cast<const float4 *>(p + j + u * nt * 4);
#pragma unroll
                for (int u = 0; u < 4; u++) take4(v[u], j + u * nt * 4);
            }
            for (; j < end4; j += nt * 4) take4(*reinterpret_cast<const float4 *>(p + j), j);
            const int jt = end4 + t;
            if (jt < end && beats(p[jt], jt, bv, bi)) {
                bv = p[jt];
                bi = jt;
            }
        } else {
            for (int j = begin + t; j < end; j += nt) {
                const float v = p[j];
                if (beats(v, j, bv, bi)) {
                    bv = v;
                    bi = j;
                }
            }
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (beats(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (wpc == 1) {
        if (live && lane == 0) stats[((uint64_t)b * g.R + row) * g.C + c] = Stat{bv, bi};
        return;
    }
    __shared__ Stat ws[4];
    if (lane == 0) ws[wave] = Stat{bv, bi};
    __syncthreads();
    if (threadIdx.x == 0 && live) {
        Stat s = ws[0];
        for (int w = 1; w < 4; w++)
            if (beats(ws[w].v, ws[w].i, s.v, s.i)) s = ws[w];
        stats[((uint64_t)b * g.R + row) * g.C + c] = s;
    }
}

// Truncation cut of one row (top-k / top-p): an element is kept iff its
// order key is above `key`, or equal to it with an id of at most `id`. The
// default {0, INT_MAX} keeps every valid logit.
struct Cut {
    uint32_t key;
    int32_t id;
};

// Monotone map of a float onto uint32 (larger logit, larger key). -0 maps
// with +0, since the sampler's sort compares values (sampling.go:84-89).
__device__ __forceinline__ uint32_t order_key(float l) {
    uint32_t u = __float_as_uint(l);
    if ((u << 1) == 0u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t key) {
    return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// NaN and -Inf are dropped (sampling.go:75-80).
__device__ __forceinline__ bool valid_logit(float l) { return l == l && l != -INFINITY; }

__device__ __forceinline__ bool in_cut(uint32_t key, int j, const Cut &c) {
    return key > c.key || (key == c.key && j <= c.id);
}

// exp(float64(logit - max) / T) (sampling.go:97), zero outside the cut.
__device__ __forceinline__ double weight_of(float l, int j, float mx, double t, const Cut &c) {
    if (!valid_logit(l) || !in_cut(order_key(l), j, c)) return 0.0;
    return exp((double)(l - mx) / t);
}

__device__ __forceinline__ Cut row_cut(const Cut *cuts, const Geo &g, int b, int row) {
    return cuts ? cuts[(uint64_t)b * g.R + row] : Cut{0u, INT_MAX};
}

__global__ __launch_bounds__(256) void accept_weights_kernel(const float *__restrict__ logits, Geo g,
                                                             const int32_t *__restrict__ drafts,
                                                             const Stat *__restrict__ stats,
                                                             const Cut *__restrict__ cuts, double t,
                                                             double *__restrict__ sums,
                                                             double *__restrict__ wdraft) {
    const int c = blockIdx.x, row = blockIdx.y, b = blockIdx.z;
    const float *p = row_ptr(logits, g, b, row);
    __shared__ float mx_s;
    if (threadIdx.x < 64) {  // wave 0 reduces the row's chunk maxima
        const Stat *st = stats + ((uint64_t)b * g.R + row) * g.C;
        float bv = -INFINITY;
        int bi = INT_MAX;
        for (int cc = threadIdx.x; cc < g.C; cc += 64)
            if (beats(st[cc].v, st[cc].i, bv, bi)) { bv = st[cc].v; bi = st[cc].i; }
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        if (threadIdx.x == 0) mx_s = bv;
    }
    __syncthreads();
    const float mx = mx_s;
    const Cut cut = row_cut(cuts, g, b, row);
    const int d = row < g.k ? drafts[(uint64_t)b * g.ds + row] : -1;
    const int begin = c * g.L;
    const int end = min(begin + g.L, g.V);
    double acc = 0.0;
    // eight logit loads in flight per thread; the sum keeps index order
    constexpr int kU = 8;
    int j = begin + threadIdx.x;
    for (; j + (kU - 1) * 256 < end; j += kU * 256) {
        float l[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) l[u] = p[j + u * 256];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const double w = weight_of(l[u], j + u * 256, mx, t, cut);
            if (j + u * 256 == d)
                wdraft[(uint64_t)b * g.R + row] = w;
            else
                acc += w;
        }
    }
    for (; j < end; j += 256) {
        const double w = weight_of(p[j], j, mx, t, cut);
        if (j == d)
            wdraft[(uint64_t)b * g.R + row] = w;
        else
            acc += w;
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    __shared__ double ws[4];
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) sums[((uint64_t)b * g.R + row) * g.C + c] = ws[0] + ws[1] + ws[2] + ws[3];
}

// ---------------------------------------------------------------- truncation
// Per-row cut for top-k / top-p (sampling.go:84-113) without sorting: radix
// selection over the 32-bit order key, one workgroup per row, histograms in
// LDS. Each wave fills its own histogram and the waves are combined in wave
// order, so weight sums do not depend on wave scheduling.
constexpr int kSelWaves = 16;

struct SelShared {
    uint32_t cnt[kSelWaves][256];
    double wsum[kSelWaves][256];
    uint32_t tc[256];
    double tw[256];
    uint32_t prefix;    // digits chosen so far
    int bucket;         // bucket chosen by the last scan (-1: none)
    uint32_t before_c;  // count of the buckets ahead of it in scan order
    double before_w;    // their weight
    double total_w;     // all weight of the first pass
    uint32_t total_c;
    int id;             // result of an id selection
    float mx;
};

// Top-p candidates held in LDS (dynamic shared memory of the select kernel):
// the ids of the first digit's boundary bucket, collected by the second pass
// when they fit, so that the third and fourth digits read those logits
// (from L2: the second pass has just read the row) instead of the row. Each
// wave fills its own segment in a fixed order, so the later passes add the
// same values in the same order on every run.
constexpr int kCandCap = 24576;
constexpr int kCandWave = kCandCap / kSelWaves;  // per-wave segment
struct Cands {
    int *j;       // [wave][kCandWave]
    uint32_t *n;  // [wave] candidates found (more than kCandWave: not all stored)
};

// Histogram of the next digit over the row's elements that `sel` admits;
// with C, the admitted elements are also appended to the candidate list.
template <bool W, bool C = false, class Sel, class Dig>
__device__ __forceinline__ void hist_pass(const float *__restrict__ p, int V, float mx, double t, SelShared &s,
                                          Sel sel, Dig dig, Cands cand = Cands{nullptr, nullptr}) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int b = lane; b < 256; b += 64) {
        s.cnt[wave][b] = 0u;
        if (W) s.wsum[wave][b] = 0.0;
    }
    __syncthreads();
    constexpr int kStride = kSelWaves * 64;
    // eight loads in flight per thread (the row is read from L2 / the
    // Infinity Cache once per pass: latency, not bandwidth, bounds the pass)
    constexpr int kU = 8;
    uint32_t wn = 0u;  // candidates of this wave so far
    for (int j0 = threadIdx.x; j0 < V; j0 += kU * kStride) {
        float l[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) l[u] = j0 + u * kStride < V ? p[j0 + u * kStride] : NAN;
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const int j = j0 + u * kStride;
            const bool take = valid_logit(l[u]) && sel(l[u], j);
            if (C) {
                // this wave's segment, in (iteration, lane) order: the list is
                // the same on every run, whatever the waves' timing
                const uint64_t m = __ballot(take);
                const uint32_t at = wn + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
                if (take && at < (uint32_t)kCandWave) cand.j[wave * kCandWave + at] = j;
                wn += (uint32_t)__popcll(m);
            }
            if (!take) continue;
            const int b = dig(l[u], j);
            atomicAdd(&s.cnt[wave][b], 1u);
            if (W) unsafeAtomicAdd(&s.wsum[wave][b], exp((double)(l[u] - mx) / t));
        }
    }
    if (C && lane == 0) cand.n[wave] = wn;
    __syncthreads();
    if (threadIdx.x < 256) {
        uint32_t c = 0u;
        double w = 0.0;
        for (int q = 0; q < kSelWaves; q++) {
            c += s.cnt[q][threadIdx.x];
            if (W) w += s.wsum[q][threadIdx.x];
        }
        s.tc[threadIdx.x] = c;
        s.tw[threadIdx.x] = w;
    }
    __syncthreads();
}

// hist_pass over the candidate list instead of the row.
template <bool W, class Sel, class Dig>
__device__ __forceinline__ void hist_cands(const float *__restrict__ p, const Cands cand, float mx, double t,
                                           SelShared &s, Sel sel, Dig dig) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int b = lane; b < 256; b += 64) {
        s.cnt[wave][b] = 0u;
        if (W) s.wsum[wave][b] = 0.0;
    }
    __syncthreads();
    const uint32_t n = min(cand.n[wave], (uint32_t)kCandWave);  // (the caller checked every segment fits)
    for (uint32_t i = lane; i < n; i += 64) {  // wave w walks segment w
        const int j = cand.j[wave * kCandWave + i];
        const float l = p[j];
        if (!sel(l, j)) continue;
        const int b = dig(l, j);
        atomicAdd(&s.cnt[wave][b], 1u);
        if (W) unsafeAtomicAdd(&s.wsum[wave][b], exp((double)(l - mx) / t));
    }
    __syncthreads();
    if (threadIdx.x < 256) {
        uint32_t c = 0u;
        double w = 0.0;
        for (int q = 0; q < kSelWaves; q++) {
            c += s.cnt[q][threadIdx.x];
            if (W) w += s.wsum[q][threadIdx.x];
        }
        s.tc[threadIdx.x] = c;
        s.tw[threadIdx.x] = w;
    }
    __syncthreads();
}

// Wave 0: walk the buckets in scan order (descending keys, or ascending for
// ids) to the first non-empty one where the running count reaches need_c (or
// the running weight reaches need_w); append its digit to the prefix. Lane l
// takes scan positions [4 l, 4 l + 4): its running start is the
// lanes-before-it prefix (a fixed shuffle tree, so the sums are the same on
// every run), then its own buckets in order; the first lane that reaches
// the need picks. (One thread walking 256 LDS entries took ~16 us a pass.)
__device__ __forceinline__ void scan_buckets(SelShared &s, bool descending, bool by_weight, uint32_t need_c,
                                             double need_w, int shift) {
    const int lane = threadIdx.x & 63;
    uint32_t bc[4], lc = 0u;
    double bw[4], lw = 0.0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = 4 * lane + i, b = descending ? 255 - q : q;
        bc[i] = s.tc[b];
        bw[i] = s.tw[b];
        lc += bc[i];
        lw += bw[i];
    }
    uint32_t ic = lc;  // inclusive prefix over lanes
    double iw = lw;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t tc = __shfl_up(ic, off);
        const double tw = __shfl_up(iw, off);
        if (lane >= off) {
            ic += tc;
            iw += tw;
        }
    }
    const uint32_t ec = __shfl_up(ic, 1);
    const double ew = __shfl_up(iw, 1);
    uint32_t c = s.before_c + (lane ? ec : 0u);
    double w = s.before_w + (lane ? ew : 0.0);
    int pick = -1;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (pick >= 0 || !bc[i]) continue;
        if (by_weight ? (w + bw[i] >= need_w) : (c + bc[i] >= need_c)) {
            pick = 4 * lane + i;
            continue;
        }
        c += bc[i];
        w += bw[i];
    }
    const uint64_t hit = __ballot(pick >= 0);
    const int first = hit ? __ffsll((unsigned long long)hit) - 1 : -1;
    if (first < 0) {
        if (lane == 0) s.bucket = -1;
        return;
    }
    if (lane == first) {
        const int b = descending ? 255 - pick : pick;
        s.bucket = b;
        s.before_c = c;
        s.before_w = w;
        s.prefix |= (uint32_t)b << shift;
    }
}

// Wave 0: the sums of the 256 bucket counts and weights (fixed tree order).
__device__ __forceinline__ void bucket_totals(const SelShared &s, uint32_t *c_out, double *w_out) {
    const int lane = threadIdx.x & 63;
    uint32_t c = 0u;
    double w = 0.0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        c += s.tc[4 * lane + i];
        w += s.tw[4 * lane + i];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        c += __shfl_xor(c, off);
        w += __shfl_xor(w, off);
    }
    *c_out = c;
    *w_out = w;
}

// The need-th smallest id (1-based) among the elements with order key `key`
// that lie inside `cut`.
__device__ int select_id(const float *p, int V, SelShared &s, uint32_t key, Cut cut, uint32_t need) {
    // One ordered sweep: 8 slices of kSelWaves * 64 consecutive ids per
    // step, the matches of each wave counted by ballot, and the step where
    // the running count reaches `need` resolved by rank.
    constexpr int kT = kSelWaves * 64, kU = 8;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (threadIdx.x == 0) s.id = INT_MAX;
    uint32_t before = 0u;
    for (int base = 0; base < V; base += kU * kT) {
        float l[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const int j = base + u * kT + threadIdx.x;
            l[u] = p[min(j, V - 1)];
        }
        bool m[kU];
        uint64_t bal[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const int j = base + u * kT + threadIdx.x;
            m[u] = j < V && valid_logit(l[u]) && order_key(l[u]) == key && in_cut(key, j, cut);
            bal[u] = __ballot(m[u]);
            if (lane == 0) s.cnt[u][wave] = (uint32_t)__popcll(bal[u]);
        }
        __syncthreads();
        uint32_t tot = 0u;
        for (int q = 0; q < kU * kSelWaves; q++) tot += s.cnt[q / kSelWaves][q % kSelWaves];
        if (before + tot >= need) {
            uint32_t r = before;
#pragma unroll
            for (int u = 0; u < kU; u++) {
                uint32_t pw = 0u;
                for (int q = 0; q < kSelWaves; q++) pw += q < wave ? s.cnt[u][q] : 0u;
                const uint32_t rank = r + pw + (uint32_t)__popcll(bal[u] & ((1ull << lane) - 1ull)) + 1u;
                if (m[u] && rank == need) s.id = base + u * kT + threadIdx.x;
                for (int q = 0; q < kSelWaves; q++) r += s.cnt[u][q];
            }
            break;
        }
        before += tot;
        __syncthreads();  // the counts are read before the next step overwrites them
    }
    __syncthreads();
    const int id = s.id;
    __syncthreads();  // every thread has read the result before the state is reused
    return id;
}

// First top-p digit of one chunk of a row: counts and weights of the
// elements inside the top-k cut by the top byte of their order key. One
// workgroup per (chunk, row, request), so the float64 exponentials of the
// whole vocabulary spread over the GPU; the select kernel adds the chunks in
// chunk order (deterministic).
struct Hist0 {
    uint32_t c[256];
    double w[256];
};

__global__ __launch_bounds__(256) void accept_hist_kernel(const float *__restrict__ logits, Geo g,
                                                          const Stat *__restrict__ stats,
                                                          const Cut *__restrict__ cuts, double t,
                                                          Hist0 *__restrict__ out) {
    const int c = blockIdx.x, row = blockIdx.y, b = blockIdx.z;
    const int wave = threadIdx.x >> 6;
    const float *p = row_ptr(logits, g, b, row);
    __shared__ float mx_s;
    __shared__ uint32_t cnt[4][256];
    __shared__ double ws[4][256];
    for (int i = threadIdx.x; i < 4 * 256; i += 256) {
        (&cnt[0][0])[i] = 0u;
        (&ws[0][0])[i] = 0.0;
    }
    if (threadIdx.x < 64) {  // wave 0 reduces the row's chunk maxima
        const Stat *st = stats + ((uint64_t)b * g.R + row) * g.C;
        float bv = -INFINITY;
        int bi = INT_MAX;
        for (int cc = threadIdx.x; cc < g.C; cc += 64)
            if (beats(st[cc].v, st[cc].i, bv, bi)) { bv = st[cc].v; bi = st[cc].i; }
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        if (threadIdx.x == 0) mx_s = bv;
    }
    __syncthreads();
    const float mx = mx_s;
    const Cut cut = row_cut(cuts, g, b, row);
    const int begin = c * g.L, end = min(begin + g.L, g.V);
    constexpr int kU = 8;  // loads in flight per thread
    for (int j0 = begin + threadIdx.x; j0 < end; j0 += kU * 256) {
        float lv[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) lv[u] = j0 + 256 * u < end ? p[j0 + 256 * u] : NAN;
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const int j = j0 + 256 * u;
            const float l = lv[u];
            if (!valid_logit(l)) continue;
            const uint32_t k = order_key(l);
            if (!in_cut(k, j, cut)) continue;
            atomicAdd(&cnt[wave][k >> 24], 1u);
            unsafeAtomicAdd(&ws[wave][k >> 24], exp((double)(l - mx) / t));
        }
    }
    __syncthreads();
    Hist0 &o = out[((uint64_t)b * g.R + row) * g.C + c];
    const int q = threadIdx.x;
    o.c[q] = cnt[0][q] + cnt[1][q] + cnt[2][q] + cnt[3][q];
    o.w[q] = ((ws[0][q] + ws[1][q]) + ws[2][q]) + ws[3][q];
}

// mode 0: top-k then top-p in one launch; 1: top-k only; 2: top-p only, the
// top-k cut (top_k > 0) read from `cuts` and the first digit's histogram
// summed from accept_hist_kernel's chunks.
__global__ __launch_bounds__(1024) void accept_select_kernel(const float *__restrict__ logits, Geo g,
                                                             const Stat *__restrict__ stats, int top_k,
                                                             float top_p, double t, Cut *__restrict__ cuts,
                                                             int mode, const Hist0 *__restrict__ h0) {
    const int row = blockIdx.x, b = blockIdx.y;
    const float *p = row_ptr(logits, g, b, row);
    __shared__ SelShared s;
    if (threadIdx.x < 64) {  // the row maximum from the per-chunk statistics
        const Stat *st = stats + ((uint64_t)b * g.R + row) * g.C;
        float bv = -INFINITY;
        int bi = INT_MAX;
        for (int cc = threadIdx.x; cc < g.C; cc += 64)
            if (beats(st[cc].v, st[cc].i, bv, bi)) { bv = st[cc].v; bi = st[cc].i; }
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        if (threadIdx.x == 0) s.mx = bv;
    }
    __syncthreads();
    const float mx = s.mx;
    Cut cut{0u, INT_MAX};
    if (mode == 2 && top_k > 0) cut = cuts[(uint64_t)b * g.R + row];

    // top-k: the top_k-th element in (logit desc, id asc) order (sampling.go:90-92).
    if (top_k > 0 && mode != 2) {
        if (threadIdx.x == 0) {
            s.prefix = 0u;
            s.before_c = 0u;
            s.before_w = 0.0;
        }
        __syncthreads();
        bool all = false;
        for (int pass = 0; pass < 4; pass++) {
            const int shift = 24 - 8 * pass;
            const uint32_t mask = pass ? ~0u << (shift + 8) : 0u;
            const uint32_t pre = s.prefix;
            hist_pass<false>(
                p, g.V, mx, t, s, [=](float l, int) { return (order_key(l) & mask) == pre; },
                [=](float l, int) { return (order_key(l) >> shift) & 255u; });
            if (threadIdx.x < 64) {
                uint32_t tot_c = s.total_c;
                if (pass == 0) {
                    double unused;
                    bucket_totals(s, &tot_c, &unused);
                    if (threadIdx.x == 0) s.total_c = tot_c;
                }
                if (tot_c > (uint32_t)top_k) scan_buckets(s, true, false, (uint32_t)top_k, 0.0, shift);
            }
            __syncthreads();
            if (s.total_c <= (uint32_t)top_k) {
                all = true;
                break;
            }
        }
        if (!all) {
            const uint32_t key = s.prefix;
            const uint32_t need = (uint32_t)top_k - s.before_c;
            const uint32_t ties = s.tc[s.bucket];
            __syncthreads();
            cut.key = key;
            cut.id = need < ties ? select_id(p, g.V, s, key, Cut{0u, INT_MAX}, need) : INT_MAX;
        }
    }

    // top-p: the smallest prefix whose cumulative share reaches top_p
    // (sampling.go:104-113), within the top-k set.
    if (top_p > 0.0f && top_p < 1.0f && mode != 1) {
        __syncthreads();
        if (threadIdx.x == 0) {
            s.prefix = 0u;
            s.before_c = 0u;
            s.before_w = 0.0;
        }
        __syncthreads();
        bool found = true;
        // mode 2: the second pass keeps the first digit's bucket in LDS when
        // it fits; the later passes then scan only those elements
        extern __shared__ uint8_t sel_dyn[];
        const Cands cand{reinterpret_cast<int *>(sel_dyn), reinterpret_cast<uint32_t *>(sel_dyn + kCandCap * 4)};
        bool compact = false;
        for (int pass = 0; pass < 4 && found; pass++) {
            const int shift = 24 - 8 * pass;
            const uint32_t mask = pass ? ~0u << (shift + 8) : 0u;
            const uint32_t pre = s.prefix;
            const Cut ck = cut;
            const auto sel_fn = [=](float l, int j) {
                const uint32_t k = order_key(l);
                return in_cut(k, j, ck) && (k & mask) == pre;
            };
            const auto dig_fn = [=](float l, int) { return (order_key(l) >> shift) & 255u; };
            const bool collect = mode == 2 && pass == 1 && s.tc[s.bucket] <= (uint32_t)kCandCap;
            if (pass == 0 && h0) {  // chunk histograms, added in chunk order
                if (threadIdx.x < 256) {
                    const Hist0 *hr = h0 + ((uint64_t)b * g.R + row) * g.C;
                    uint32_t cc = 0u;
                    double w = 0.0;
                    for (int ch = 0; ch < g.C; ch++) {
                        cc += hr[ch].c[threadIdx.x];
                        w += hr[ch].w[threadIdx.x];
                    }
                    s.tc[threadIdx.x] = cc;
                    s.tw[threadIdx.x] = w;
                }
                __syncthreads();
            } else if (compact) {
                hist_cands<true>(p, cand, mx, t, s, sel_fn, dig_fn);
            } else if (collect) {
                hist_pass<true, true>(p, g.V, mx, t, s, sel_fn, dig_fn, cand);
                bool fits = true;
                for (int w = 0; w < kSelWaves; w++) fits = fits && cand.n[w] <= (uint32_t)kCandWave;
                compact = fits;  // else the later digits read the row
            } else {
                hist_pass<true>(p, g.V, mx, t, s, sel_fn, dig_fn);
            }
            if (threadIdx.x < 64) {
                double tot = s.total_w;
                if (pass == 0) {
                    uint32_t unused;
                    bucket_totals(s, &unused, &tot);
                    if (threadIdx.x == 0) s.total_w = tot;
                }
                if (tot > 0.0 && !isinf(tot))
                    scan_buckets(s, true, true, 0u, (double)top_p * tot, shift);
                else if (threadIdx.x == 0)
                    s.bucket = -1;
            }
            __syncthreads();
            found = s.bucket >= 0;
        }
        if (found) {
            // The tie group at the boundary: add its members one by one as the
            // sampler's running sum does.
            if (threadIdx.x == 0) {
                const uint32_t key = s.prefix;
                const uint32_t ties = s.tc[s.bucket];
                const double tot = s.total_w;
                const double wt = exp((double)(key_value(key) - mx) / t);
                double cum = s.before_w / tot;
                uint32_t m = ties;
                for (uint32_t i = 1; i <= ties; i++) {
                    cum += wt / tot;
                    if (cum >= (double)top_p) {
                        m = i;
                        break;
                    }
                }
                s.before_c = m;  // kept members of the tie group
                s.total_c = ties;
            }
            __syncthreads();
            const uint32_t key = s.prefix, m = s.before_c, ties = s.total_c;
            __syncthreads();
            Cut nc{key, key == cut.key ? cut.id : INT_MAX};
            if (m < ties) nc.id = select_id(p, g.V, s, key, cut, m);
            cut = nc;
        }
    }
    if (threadIdx.x == 0) cuts[(uint64_t)b * g.R + row] = cut;
}

// Philox4x32-10 (Salmon et al., SC'11).
__device__ __forceinline__ void philox(uint32_t c[4], uint32_t k0, uint32_t k1) {
    for (int r = 0; r < 10; r++) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
        const uint32_t n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
        const uint32_t n3 = (uint32_t)p0;
        c[0] = n0; c[1] = n1; c[2] = n2; c[3] = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

__device__ __forceinline__ double draw(uint64_t seed, uint64_t step, uint32_t row, uint32_t request,
                                       uint32_t purpose) {
    uint32_t c[4] = {(uint32_t)step, (uint32_t)(step >> 32), request, (row << 8) | (purpose & 0xffu)};
    philox(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    const uint64_t v = ((((uint64_t)c[0]) << 32) | c[1]) >> 11;
    return (double)v * (1.0 / 9007199254740992.0);
}

// Router logits replaced by i.i.d. N(0,1) draws: thread per (row, expert
// pair), one Philox block per pair, Box-Muller on two 53-bit uniforms (u1 in
// (0, 1]).
__global__ __launch_bounds__(256) void router_normal_kernel(float *__restrict__ logits, int rows, int E,
                                                            uint64_t seed, uint32_t layer,
                                                            const uint64_t *__restrict__ step_ptr) {
    const int pairs = (E + 1) / 2;
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= rows * pairs) return;
    const int r = idx / pairs, p = idx - r * pairs;
    const uint64_t step = step_ptr ? *step_ptr : 0;
    uint32_t c[4] = {(uint32_t)step, (uint32_t)(step >> 32), layer, ((uint32_t)r << 16) | (uint32_t)p};
    philox(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    const double u1 = (double)(((((uint64_t)c[0]) << 32 | c[1]) >> 11) + 1) * (1.0 / 9007199254740992.0);
    const double u2 = (double)((((uint64_t)c[2]) << 32 | c[3]) >> 11) * (1.0 / 9007199254740992.0);
    const double rad = sqrt(-2.0 * log(u1)), ang = 6.283185307179586 * u2;
    float *row = logits + (uint64_t)r * E;
    row[2 * p] = (float)(rad * cos(ang));
    if (2 * p + 1 < E) row[2 * p + 1] = (float)(rad * sin(ang));
}

// Block-wide inverse CDF inside chunk `c` of a row: the first index j (j != d,
// weight > 0) whose running weight sum exceeds `target`. Returns -1 when the
// target lies beyond the chunk's own sum (rounding), with *last the last
// positive-weight index of the chunk.
__device__ int scan_chunk(const float *p, const Geo &g, int c, int d, float mx, double t, const Cut &cut,
                          double target, double *shared_prefix, int *shared_pick) {
    const int begin = c * g.L;
    const int end = min(begin + g.L, g.V);
    const int len = end - begin;
    const int per = (len + 255) / 256;
    const int lo = begin + threadIdx.x * per;
    const int hi = min(lo + per, end);
    double local = 0.0;
    int j = lo;
    for (; j + 7 < hi; j += 8) {  // eight loads in flight, summed in index order
        float l[8];
#pragma unroll
        for (int u = 0; u < 8; u++) l[u] = p[j + u];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (j + u != d) local += weight_of(l[u], j + u, mx, t, cut);
    }
    for (; j < hi; j++)
        if (j != d) local += weight_of(p[j], j, mx, t, cut);
    shared_prefix[threadIdx.x] = local;
    if (threadIdx.x == 0) *shared_pick = -1;
    __syncthreads();
    if (threadIdx.x == 0) {  // exclusive prefix in thread order, 16 reads in flight at a time
        double run = 0.0;
        for (int t0 = 0; t0 < 256; t0 += 16) {
            double v[16];
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = shared_prefix[t0 + i];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                shared_prefix[t0 + i] = run;
                run += v[i];
            }
        }
    }
    __syncthreads();
    double run = shared_prefix[threadIdx.x];
    if (run <= target && target < run + local) {
        for (int j = lo; j < hi; j++) {
            if (j == d) continue;
            const double w = weight_of(p[j], j, mx, t, cut);
            if (w <= 0.0) continue;
            run += w;
            if (target < run) {
                *shared_pick = j;
                break;
            }
        }
        if (*shared_pick < 0) {  // rounding at the boundary: last positive weight
            for (int j = hi - 1; j >= lo; j--)
                if (j != d && weight_of(p[j], j, mx, t, cut) > 0.0) {
                    *shared_pick = j;
                    break;
                }
        }
    }
    __syncthreads();
    return *shared_pick;
}

__global__ __launch_bounds__(256) void accept_finalize_kernel(
    const float *__restrict__ logits, Geo g, const int32_t *__restrict__ drafts,
    const Stat *__restrict__ stats, const double *__restrict__ sums,
    const double *__restrict__ wdraft, const Cut *__restrict__ cuts, int stochastic, double t, uint64_t seed,
    uint64_t step,
    uint32_t request_base, int32_t *__restrict__ result, double *__restrict__ debug,
    const uint64_t *__restrict__ step_dev, const int32_t *__restrict__ forced) {
    const int b = blockIdx.x;
    if (step_dev) step = *step_dev;
    const uint32_t request = request_base + (uint32_t)b;
    __shared__ double prefix[256];
    __shared__ int pick;
    __shared__ int decided_next;
    __shared__ int accepted_s;
    __shared__ int argmax0;
    __shared__ Stat row_best_s[256];
    __shared__ double row_rest_s[256];
    __shared__ float row_p0_s[256];  // logit 0 of each row
    __shared__ int row_d_s[256];     // each row's draft (-1 on the bonus row)
    if (threadIdx.x == 0) {
        decided_next = -1;
        accepted_s = 0;
    }
    // Per-row maxima and weight sums: one wave per row, lanes over chunks.
    {
        const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
        for (int row = wave; row <= g.k; row += 4) {
            const Stat *st = stats + ((uint64_t)b * g.R + row) * g.C;
            Stat best{-INFINITY, INT_MAX};
            double rest = 0.0;
            for (int c = lane; c < g.C; c += 64) {
                if (beats(st[c].v, st[c].i, best.v, best.i)) best = st[c];
                if (stochastic) rest += sums[((uint64_t)b * g.R + row) * g.C + c];
            }
            for (int off = 32; off > 0; off >>= 1) {
                const float ov = __shfl_xor(best.v, off);
                const int oi = __shfl_xor(best.i, off);
                if (beats(ov, oi, best.v, best.i)) best = Stat{ov, oi};
                rest += __shfl_xor(rest, off);
            }
            if (lane == 0) {
                row_best_s[row] = best;
                row_rest_s[row] = rest;
                row_p0_s[row] = row_ptr(logits, g, b, row)[0];
                row_d_s[row] = row < g.k ? drafts[(uint64_t)b * g.ds + row] : -1;
            }
        }
    }
    __syncthreads();
    for (int row = 0; row <= g.k; row++) {
        const float *p = row_ptr(logits, g, b, row);
        __shared__ Stat best_s;
        __shared__ int action;  // 0 accept, 1 done (next decided), 2 resample
        __shared__ double target_s;
        __shared__ int cstar;
        __shared__ float mx_s;
        __shared__ double cs_s[256];  // the row's chunk weight sums, for thread 0's walk below
        if (stochastic)
            for (int c = threadIdx.x; c < g.C && c < 256; c += 256) cs_s[c] = sums[((uint64_t)b * g.R + row) * g.C + c];
        __syncthreads();
        if (threadIdx.x == 0) {
            Stat best = row_best_s[row];
            const float p0 = row_p0_s[row];
            if (p0 != p0) best = Stat{p0, 0};  // argmaxLogit keeps a NaN at index 0
            best_s = best;
            if (row == 0) argmax0 = best.i;
            const int d = row_d_s[row];
            double dbg[4] = {0.0, 0.0, 0.0, (double)best.v};
            action = 1;
            // forced: a prescribed acceptance length replaces the accept test;
            // the token at the first rejected row is still the mode's choice
            const int flen = forced ? forced[b] : -1;
            if (!stochastic) {
                if (row < g.k && (forced ? row < flen : best.i == d)) {
                    action = 0;
                } else {
                    decided_next = best.i;
                }
            } else {
                // The sampler's first candidate: the maximum over valid logits;
                // with none valid, argmaxLogit's answer (sampling.go:83-89).
                Stat sb = row_best_s[row];
                if (sb.v == -INFINITY) sb = best;
                best_s = sb;
                const double *cs = g.C <= 256 ? cs_s : sums + ((uint64_t)b * g.R + row) * g.C;
                const double rest = row_rest_s[row];
                const double wd = (row < g.k && d >= 0 && d < g.V) ? wdraft[(uint64_t)b * g.R + row] : 0.0;
                double total = rest + wd;
                const bool onehot = !(total > 0.0) || isinf(total);
                dbg[2] = total;
                if (row < g.k) {
                    const double pd = onehot ? (d == sb.i ? 1.0 : 0.0) : wd / total;
                    const double u = draw(seed, step, (uint32_t)row, request, 0);
                    dbg[0] = pd;
                    dbg[1] = u;
                    if (forced ? row < flen : u < pd) {
                        action = 0;
                    } else if (onehot || !(rest > 0.0)) {
                        decided_next = sb.i;
                    } else {
                        const double u2 = draw(seed, step, (uint32_t)row, request, 1);
                        const double target = u2 * rest;
                        double run = 0.0;
                        int c = 0;
                        for (; c < g.C - 1; c++) {
                            if (target < run + cs[c]) break;
                            run += cs[c];
                        }
                        target_s = target - run;
                        cstar = c;
                        mx_s = sb.v;
                        action = 2;
                    }
                } else {
                    if (onehot) {
                        decided_next = sb.i;
                    } else {
                        const double u2 = draw(seed, step, (uint32_t)row, request, 1);
                        const double target = u2 * total;
                        double run = 0.0;
                        int c = 0;
                        for (; c < g.C - 1; c++) {
                            if (target < run + cs[c]) break;
                            run += cs[c];
                        }
                        target_s = target - run;
                        cstar = c;
                        mx_s = sb.v;
                        action = 2;
                    }
                }
            }
            if (debug) {
                double *o = debug + (((uint64_t)b * g.R) + row) * 4;
                for (int i = 0; i < 4; i++) o[i] = dbg[i];
            }
        }
        __syncthreads();
        if (action == 0) {
            if (threadIdx.x == 0) accepted_s++;
            __syncthreads();
            continue;
        }
        if (action == 2) {
            const int d = row < g.k ? drafts[(uint64_t)b * g.ds + row] : -1;
            const int j = scan_chunk(p, g, cstar, d, mx_s, t, row_cut(cuts, g, b, row), target_s, prefix, &pick);
            if (threadIdx.x == 0) decided_next = j >= 0 ? j : best_s.i;
        }
        break;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int32_t *o = result + (uint64_t)b * 4;
        o[0] = accepted_s;
        o[1] = decided_next;
        o[2] = argmax0;
        o[3] = 0;
    }
}

Geo make_geo(const yuuka_accept_params &p) {
    Geo g;
    g.B = (int)p.batch;
    g.k = (int)p.drafts;
    g.R = g.k + 1;
    g.V = (int)p.vocab;
    g.stride = p.row_stride ? p.row_stride : p.vocab;
    g.ds = g.k;
    int c = (2048 + g.B * g.R - 1) / (g.B * g.R);
    c = c < 1 ? 1 : (c > 256 ? 256 : c);
    int L = (g.V + c - 1) / c;
    L = (L + 3) & ~3;
    g.L = L;
    g.C = (g.V + L - 1) / L;
    return g;
}

}  // namespace

uint64_t accept_scratch_bytes(const yuuka_accept_params &p) {
    const Geo g = make_geo(p);
    const uint64_t n = (uint64_t)g.B * g.R * g.C;
    return ((n * sizeof(Stat) + 255) & ~255ull) + n * sizeof(double) +
           (uint64_t)g.B * g.R * (sizeof(double) + sizeof(Cut)) + 256 + n * sizeof(Hist0);
}

hipError_t launch_router_normal(float *logits, int rows, int E, uint64_t seed, uint32_t layer, const uint64_t *step,
                                hipStream_t s) {
    const int n = rows * ((E + 1) / 2);
    if (n > 0) router_normal_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(logits, rows, E, seed, layer, step);
    return hipGetLastError();
}

hipError_t launch_verify_accept(const float *logits, const int32_t *drafts, int32_t *result,
                                double *debug, const yuuka_accept_params &p, void *scratch,
                                hipStream_t stream, const uint64_t *step_dev, uint32_t draft_stride,
                                const int32_t *forced) {
    Geo g = make_geo(p);
    if (draft_stride) g.ds = (int)draft_stride;
    const uint64_t n = (uint64_t)g.B * g.R * g.C;
    auto *base = static_cast<uint8_t *>(scratch);
    Stat *stats = reinterpret_cast<Stat *>(base);
    double *sums = reinterpret_cast<double *>(base + ((n * sizeof(Stat) + 255) & ~255ull));
    double *wdraft = sums + n;
    Cut *cuts = reinterpret_cast<Cut *>(wdraft + (uint64_t)g.B * g.R);
    Hist0 *h0 = reinterpret_cast<Hist0 *>(
        (reinterpret_cast<uintptr_t>(cuts + (uint64_t)g.B * g.R) + 255) & ~(uintptr_t)255);
    const bool stochastic = p.mode == YUUKA_ACCEPT_STOCHASTIC && p.temperature > 0.0f && p.top_k != 1;
    const double t = stochastic ? (double)p.temperature : 1.0;
    // top_p 0 means off (sampling.go:46-48); top_k at or above the vocabulary keeps everything.
    const bool top_k_on = p.top_k > 1 && p.top_k < p.vocab;
    const bool top_p_on = p.top_p > 0.0f && p.top_p < 1.0f;
    const bool truncate = stochastic && (top_k_on || top_p_on);
    const dim3 grid((unsigned)g.C, (unsigned)g.R, (unsigned)g.B);
    // 16-byte loads need every row start 16-byte aligned
    const int vec = (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && (g.stride & 3) == 0;
    // one wave per chunk up to 8 logits per lane, else a workgroup per chunk
    const int wpc = g.L <= 512 * 4 ? 1 : 4;
    const dim3 sgrid((unsigned)((g.C + 4 / wpc - 1) / (4 / wpc)), (unsigned)g.R, (unsigned)g.B);
    accept_stats_kernel<<<sgrid, 256, 0, stream>>>(logits, g, stats, vec, wpc);
    const dim3 sel((unsigned)g.R, (unsigned)g.B);
    const int tk = top_k_on ? (int)p.top_k : 0;
    if (truncate && !top_p_on) {
        accept_select_kernel<<<sel, kSelWaves * 64, 0, stream>>>(logits, g, stats, tk, 1.0f, t, cuts, 0, nullptr);
    } else if (truncate) {
        // top-k cut, then the first top-p digit over all chunks in parallel,
        // then the remaining top-p digits per row
        if (top_k_on)
            accept_select_kernel<<<sel, kSelWaves * 64, 0, stream>>>(logits, g, stats, tk, 1.0f, t, cuts, 1, nullptr);
        accept_hist_kernel<<<grid, 256, 0, stream>>>(logits, g, stats, top_k_on ? cuts : nullptr, t, h0);
        static bool attr = false;
        constexpr uint32_t cand_lds = kCandCap * 4 + kSelWaves * 4;
        if (!attr) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(accept_select_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)cand_lds);
            attr = true;
        }
        accept_select_kernel<<<sel, kSelWaves * 64, cand_lds, stream>>>(logits, g, stats, tk, p.top_p, t, cuts, 2, h0);
    }
    const Cut *cut_arg = truncate ? cuts : nullptr;
    if (stochastic)
        accept_weights_kernel<<<grid, 256, 0, stream>>>(logits, g, drafts, stats, cut_arg, t, sums, wdraft);
    accept_finalize_kernel<<<(unsigned)g.B, 256, 0, stream>>>(logits, g, drafts, stats, sums, wdraft, cut_arg,
                                                             stochastic ? 1 : 0, t, p.seed, p.step,
                                                             p.request_base, result, debug, step_dev, forced);
    return hipGetLastError();
}

}  // namespace yk
