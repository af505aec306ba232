// Directed Hausdorff distance between point clouds, as a fused streaming max-min that never
// forms the p1 x p2 distance matrix.
//
// Semantics (reference CPU loop, csrc/ops/cpu/hausdorff_kernel.cpp:25-51): for every cloud
// pair, value = sqrt(max_m min_n d(m, n)) with d summed over k in order in fp32 without
// contraction; x1 index = the last m (iteration order) whose min equals the max; x2 index =
// the first n reaching that m's min.  The reference breaks out of the n loop as soon as
// d < (max so far); any m it skips that way has min < final max, so the result is the same
// for any schedule that prunes an m only when it has seen a d below a value that some other
// m's exact min reaches.  That is what the kernels here do:
//
//   1. relayout: each cloud to SoA [d][p] in iteration order (the shuffle permutation, when
//      given, is applied here, so every later scan is contiguous);
//   2. seed: per cloud pair, the 8 points of x1 farthest from x2's bounding box get an exact
//      full scan; their largest min is a first threshold T (a lower bound of the answer);
//   3. scan (d <= 3): x2 clouds are counting-sorted by grid cell once; every lane takes one m
//      and checks the 64 sorted x2 points at m's cell, stopping at the first d < T; the m left
//      are scanned by the whole wave (64 n per step, dropping m at the first d < T).  When the
//      flags fit (pairs x p1 bits <= 32 MiB), x1 is sorted by cell too, in a frame shared
//      with x2, so that neighbouring lanes check overlapping windows, and the m left are
//      flagged and scanned in iteration order by a second kernel.
//      (d > 3: every wave takes one m at a time over x2 in iteration order, the first points
//      from LDS.)  An m scanned to the end has its exact min; it is folded into the pair's key
//      (float bits of min << 32 | m position) with a 64-bit atomicMax, which also raises T for
//      everyone.  Equal mins resolve to the larger m position = the last m.
//   4. finalize: one wave per pair rescans the winning m for the first n position reaching
//      its min, and writes sqrt, and the (permuted) indices.
//
// Non-negative fp32 bit patterns order like the values, so the packed key orders by
// (value, m position) exactly.  That argument needs finite coordinates: with a NaN or an
// infinity the loop's updates depend on the order of the NaN sums (a row whose last sum is NaN
// is never folded, and the candidate indices then carry over from earlier rows).  Each batch is
// therefore checked for values that are not finite while its points are first read, and the
// pairs of a batch that holds one take the reference's loop in its own order instead
// (hdx::exact_pair), written over whatever the pruned kernels left.
#include <algorithm>
#include <mutex>

#include "common.hpp"
#include "hausdorff_exact.hpp"

#pragma clang fp contract(off)

namespace tpw {
namespace {

constexpr int kThreads = 256;
constexpr int kSeeds = 8;
constexpr int kLdsFloats = 8192;  // 32 KiB of x2 points per block

__device__ __forceinline__ float sqdist(const float *a, const float *xs, int64_t stride,
                                        int64_t n, int d) {
    float s = 0.0f;
    for (int k = 0; k < d; ++k) {
        const float diff = a[k] - xs[k * stride + n];
        s = s + diff * diff;
    }
    return s;
}

template <int D>
__device__ __forceinline__ float sqdist_fixed(const float (&a)[D], const float *xs, int64_t stride,
                                              int64_t n) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < D; ++k) {
        const float diff = a[k] - xs[k * stride + n];
        s = s + diff * diff;
    }
    return s;
}

__device__ __forceinline__ int64_t cdiv_dev(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Work unit of a 1-D grid's block: blocks go round-robin over the 8 XCDs (blockIdx.x % 8 picks
// the XCD), so when total % 8 == 0 each XCD is given a contiguous range of units.  Kernels order
// their units by the cloud they read most, so that an XCD works through a few clouds at a time
// and keeps them in its own L2.
__device__ __forceinline__ int64_t xcd_unit(int64_t total) {
    const int64_t L = blockIdx.x;
    return (total & 7) == 0 ? (L & 7) * (total >> 3) + (L >> 3) : L;
}

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float threshold_of(const unsigned long long *key) {
    unsigned long long k = __hip_atomic_load(key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __uint_as_float((uint32_t)(k >> 32));
}

__device__ __forceinline__ void fold_key(unsigned long long *key, float mn, int64_t m) {
    const unsigned long long k = ((unsigned long long)__float_as_uint(mn) << 32) | (uint64_t)m;
    atomicMax(key, k);
}

// Measurement counters of the cell-grid path (d <= 3), armed by tpw_hausdorff_counters: [0]
// point pairs whose squared distance a kernel evaluated, [1] cell-box tests of the cell scan.
// Kernels take the array's device address, or null when counting is off; each wave adds its
// own totals once, at its end.
__device__ unsigned long long g_hd_counts[2];

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += (uint32_t)__shfl_xor((int)v, off, 64);
    return v;
}
__device__ __forceinline__ void add_counts(unsigned long long *counts, uint32_t evals, uint32_t tests) {
    if (!counts) return;  // the same in every lane
    evals = wave_sum_u32(evals);
    tests = wave_sum_u32(tests);
    if ((threadIdx.x & 63) == 0) {
        if (evals) atomicAdd(&counts[0], (unsigned long long)evals);
        if (tests) atomicAdd(&counts[1], (unsigned long long)tests);
    }
}

// Point at iteration position `pos` of cloud c of an input [clouds][p][D] as given (the
// shuffle permutation perm[batch][p], batch = c / cpb, maps positions to rows when given).
template <int D>
__device__ __forceinline__ void point_at(const float *x, const int64_t *perm, int64_t c, int64_t cpb, int64_t p,
                                         int64_t pos, float (&a)[D]) {
    const int64_t src = perm ? perm[(c / cpb) * p + pos] : pos;
    const float *s = x + (c * p + src) * D;
#pragma unroll
    for (int k = 0; k < D; ++k) a[k] = s[k];
}

// A cell-sorted point is one 16-byte record: its D <= 3 coordinates, then (dword 3) its
// iteration position, so that one vector load brings the whole point and a sorted point still
// names its place in the reference's loop order.
__device__ __forceinline__ float rec_coord(const float4 &v, int k) { return k == 0 ? v.x : k == 1 ? v.y : v.z; }
__device__ __forceinline__ uint32_t rec_pos(const float4 &v) { return __float_as_uint(v.w); }
template <int D>
__device__ __forceinline__ float4 make_rec(const float (&a)[D], uint32_t pos) {
    return make_float4(a[0], D > 1 ? a[D > 1 ? 1 : 0] : 0.0f, D > 2 ? a[D > 2 ? 2 : 0] : 0.0f, __uint_as_float(pos));
}
// d(a, record) summed over k in order, as sqdist_fixed
template <int D>
__device__ __forceinline__ float rec_dist(const float (&a)[D], const float4 &v) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < D; ++k) {
        const float diff = a[k] - rec_coord(v, k);
        s = s + diff * diff;
    }
    return s;
}

// Whether x1 position m is one of the pair's seeds (whose exact mins are in the key already).
__device__ __forceinline__ bool is_seed(const uint32_t *seedm, int64_t pair, int64_t m) {
    bool r = false;
#pragma unroll
    for (int s = 0; s < kSeeds; ++s) r = r | (seedm[pair * kSeeds + s] == (uint32_t)m);
    return r;
}

// xs[c][k][pos] = x[c][perm ? perm[batch_of(c)][pos] : pos][k]; a point with a coordinate that
// is not finite (v - v != 0: NaN or an infinity) sets its batch's word of nonfin (preset to 0).
__global__ void soa_kernel(const float *__restrict__ x, const int64_t *__restrict__ perm,
                           int64_t clouds, int64_t clouds_per_batch, int64_t p, int d,
                           float *__restrict__ xs, uint32_t *__restrict__ nonfin) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= clouds * p) return;
    const int64_t c = t / p, pos = t - c * p;
    const int64_t src = perm ? perm[(c / clouds_per_batch) * p + pos] : pos;
    const float *s = x + (c * p + src) * d;
    float *o = xs + c * d * p + pos;
    bool bad = false;
    for (int k = 0; k < d; ++k) {
        const float v = s[k];
        bad = bad || !(v - v == 0.0f);
        o[(int64_t)k * p] = v;
    }
    if (bad) atomicOr(&nonfin[c / clouds_per_batch], 1u);
}

// A signed int that orders like the float (NaN excluded): the bit pattern, with the magnitude
// bits flipped for negative values.  The map is its own inverse.
__device__ __forceinline__ int ordered_int(float f) {
    const int i = __float_as_int(f);
    return i < 0 ? i ^ 0x7fffffff : i;
}
__device__ __forceinline__ float ordered_float(int i) { return __int_as_float(i < 0 ? i ^ 0x7fffffff : i); }
constexpr uint32_t kOrderedPosInf = 0x7f800000u, kOrderedNegInf = 0x807fffffu;

// Up to 8 ranges of 32-bit words to set; word i of a range gets v[i & 1].
struct Fill {
    uint32_t *p;
    int64_t n;
    uint32_t v[2];
};
struct Fills {
    Fill f[8];
    int count;
};

__global__ void fill_kernel(Fills fs) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    // constant indices only (a dynamically indexed copy of the argument would live in LDS)
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        if (r >= fs.count) break;
        uint32_t *p = fs.f[r].p;
        const int64_t n = fs.f[r].n;
        const uint32_t v0 = fs.f[r].v[0], v1 = fs.f[r].v[1];
        for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < n; t += stride)
            p[t] = (t & 1) ? v1 : v0;
    }
}

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int mask) {
    const uint32_t lo = __shfl_xor((uint32_t)v, mask, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), mask, 64);
    return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = shfl_xor_u64(v, off);
        v = o > v ? o : v;
    }
    return v;
}
__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = shfl_xor_u64(v, off);
        v = o < v ? o : v;
    }
    return v;
}

// Bounding boxes: row r (one coordinate of one cloud, SoA) is rows [0, rowsA) of xsA (length
// pA) then rows of xsB (length pB); block (r, y) reduces points [y chunk, (y + 1) chunk) of
// the row and folds its min / max into keys[r][0..1] (ordered ints, preset to +inf / -inf)
// with atomics.  NaN is ignored, as fminf / fmaxf ignore it.
__global__ __launch_bounds__(kThreads) void bbox_rows_kernel(const float *__restrict__ xsA, int64_t rowsA,
                                                             int64_t pA, const float *__restrict__ xsB,
                                                             int64_t pB, int64_t chunk, int *__restrict__ keys) {
    __shared__ float red[2][kThreads / 64];
    const int64_t r = blockIdx.x;
    const bool inA = r < rowsA;
    const int64_t p = inA ? pA : pB;
    const float *row = inA ? xsA + r * pA : xsB + (r - rowsA) * pB;
    const int64_t beg = (int64_t)blockIdx.y * chunk;
    if (beg >= p) return;
    const int64_t end = beg + chunk < p ? beg + chunk : p;
    float lo[4] = {INFINITY, INFINITY, INFINITY, INFINITY}, hi[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    int64_t n = beg + threadIdx.x;
    for (; n + 3 * kThreads < end; n += 4 * kThreads) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float v = row[n + u * kThreads];
            lo[u] = fminf(lo[u], v);
            hi[u] = fmaxf(hi[u], v);
        }
    }
    for (; n < end; n += kThreads) {
        const float v = row[n];
        lo[0] = fminf(lo[0], v);
        hi[0] = fmaxf(hi[0], v);
    }
    float l = fminf(fminf(lo[0], lo[1]), fminf(lo[2], lo[3]));
    float h = fmaxf(fmaxf(hi[0], hi[1]), fmaxf(hi[2], hi[3]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        l = fminf(l, __shfl_xor(l, off, 64));
        h = fmaxf(h, __shfl_xor(h, off, 64));
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        red[0][wave] = l;
        red[1][wave] = h;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kThreads / 64; ++w) {
            l = fminf(l, red[0][w]);
            h = fmaxf(h, red[1][w]);
        }
        atomicMin(&keys[r * 2], ordered_int(l));
        atomicMax(&keys[r * 2 + 1], ordered_int(h));
    }
}

// Boxes as floats ([cloud][k][0..1]) from the keys of bbox_rows_kernel: x1 clouds (rows1 rows,
// when bbox1 is given) and x2 clouds (rows2 rows); then, when boxb is given, each batch's box
// over both sides' clouds (the frame the sorted mode shares between x1 and x2).
__global__ void box_finish_kernel(const int *__restrict__ keys, int64_t rows1, int64_t rows2,
                                  float *__restrict__ bbox1, float *__restrict__ bbox2, int64_t batch,
                                  int64_t b1, int64_t b2, int d, float *__restrict__ boxb) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < rows1) {
        bbox1[t * 2] = ordered_float(keys[t * 2]);
        bbox1[t * 2 + 1] = ordered_float(keys[t * 2 + 1]);
    } else if (t < rows1 + rows2) {
        const int64_t r = t - rows1;
        bbox2[r * 2] = ordered_float(keys[t * 2]);
        bbox2[r * 2 + 1] = ordered_float(keys[t * 2 + 1]);
    } else if (boxb && t < rows1 + rows2 + batch * d) {
        const int64_t q = t - rows1 - rows2;
        const int64_t bb = q / d, k = q - bb * d;
        int lo = (int)kOrderedPosInf, hi = (int)kOrderedNegInf;
        for (int64_t c = 0; c < b1; ++c) {
            lo = min(lo, keys[((bb * b1 + c) * d + k) * 2]);
            hi = max(hi, keys[((bb * b1 + c) * d + k) * 2 + 1]);
        }
        for (int64_t c = 0; c < b2; ++c) {
            lo = min(lo, keys[(rows1 + (bb * b2 + c) * d + k) * 2]);
            hi = max(hi, keys[(rows1 + (bb * b2 + c) * d + k) * 2 + 1]);
        }
        boxb[q * 2] = ordered_float(lo);
        boxb[q * 2 + 1] = ordered_float(hi);
    }
}

struct PairPtrs {
    const float *x1;
    const float *x2;
};

__device__ __forceinline__ PairPtrs pair_ptrs(const float *xs1, const float *xs2, int64_t pair,
                                              int64_t b1, int64_t b2, int64_t p1, int64_t p2,
                                              int d) {
    const int64_t per_batch = b1 * b2;
    const int64_t bb = pair / per_batch;
    const int64_t rem = pair - bb * per_batch;
    const int64_t i = rem / b2, j = rem - i * b2;
    PairPtrs r;
    r.x1 = xs1 + (bb * b1 + i) * d * p1;
    r.x2 = xs2 + (bb * b2 + j) * d * p2;
    return r;
}

// Exact min over all n of d(m, n), computed by one wave (all lanes return it), for a fixed
// feature count D: the point's coordinates stay in registers and each lane keeps four points
// in flight (the min is order-independent, so the result is that of one pass).
template <int D>
__device__ float full_scan_min_fixed(const float (&a)[D], const float *X2, int64_t p2) {
    const int lane = threadIdx.x & 63;
    float best[4] = {INFINITY, INFINITY, INFINITY, INFINITY};
    int64_t n0 = 0;
    for (; n0 + 256 <= p2; n0 += 256) {
#pragma unroll
        for (int u = 0; u < 4; ++u) best[u] = fminf(best[u], sqdist_fixed<D>(a, X2, p2, n0 + 64 * u + lane));
    }
    for (int64_t n = n0 + lane; n < p2; n += 64) best[0] = fminf(best[0], sqdist_fixed<D>(a, X2, p2, n));
    return wave_min(fminf(fminf(best[0], best[1]), fminf(best[2], best[3])));
}

// Exact min over all n of d(m, n), computed by one wave (all lanes return it).
__device__ float full_scan_min(const float *a, const float *X2, int64_t p2, int d) {
    const int lane = threadIdx.x & 63;
    float best = INFINITY;
    for (int64_t n0 = 0; n0 < p2; n0 += 64) {
        const int64_t n = n0 + lane;
        if (n < p2) best = fminf(best, sqdist(a, X2, p2, n, d));
    }
    return wave_min(best);
}

// D > 0: a fixed feature count (coordinates in registers); D == 0: any d <= 64.
template <int D>
__global__ __launch_bounds__(kThreads) void seed_kernel(const float *__restrict__ xs1,
                                                        const float *__restrict__ xs2,
                                                        const float *__restrict__ bbox,
                                                        int64_t b1, int64_t b2, int64_t p1,
                                                        int64_t p2, int d,
                                                        unsigned long long *__restrict__ keys) {
    __shared__ float candL[kThreads];
    __shared__ int64_t candM[kThreads];
    __shared__ int64_t seeds[kSeeds];
    const int64_t pair = blockIdx.x;
    const PairPtrs P = pair_ptrs(xs1, xs2, pair, b1, b2, p1, p2, d);
    const int64_t bb = pair / (b1 * b2);
    const int64_t j = pair % b2;
    const float *box = bbox + (bb * b2 + j) * d * 2;

    float bestL = -1.0f;
    int64_t bestM = 0;
    for (int64_t m = threadIdx.x; m < p1; m += kThreads) {
        float L = 0.0f;
        for (int k = 0; k < d; ++k) {
            const float v = P.x1[k * p1 + m];
            const float e = fmaxf(fmaxf(box[2 * k] - v, v - box[2 * k + 1]), 0.0f);
            L = L + e * e;
        }
        if (L > bestL) {
            bestL = L;
            bestM = m;
        }
    }
    candL[threadIdx.x] = bestL;
    candM[threadIdx.x] = bestM;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int s = 0; s < kSeeds; ++s) {
            int arg = 0;
            for (int t = 1; t < kThreads; ++t)
                if (candL[t] > candL[arg]) arg = t;
            seeds[s] = candM[arg];
            candL[arg] = -2.0f;
        }
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int s = wave; s < kSeeds; s += kThreads / 64) {
        const int64_t m = seeds[s];
        if (m >= p1) continue;
        float mn;
        if constexpr (D > 0) {
            float a[D];
#pragma unroll
            for (int k = 0; k < D; ++k) a[k] = P.x1[k * p1 + m];
            mn = full_scan_min_fixed<D>(a, P.x2, p2);
        } else {
            float a[64];
            const int dd = d < 64 ? d : 64;
            for (int k = 0; k < dd; ++k) a[k] = P.x1[k * p1 + m];
            mn = d <= 64 ? full_scan_min(a, P.x2, p2, d) : 0.0f;
        }
        if (lane == 0 && d <= 64) fold_key(&keys[pair], mn, m);
    }
}

template <int D>
__global__ __launch_bounds__(kThreads) void scan_kernel(const float *__restrict__ xs1,
                                                        const float *__restrict__ xs2,
                                                        int64_t b1, int64_t b2, int64_t p1,
                                                        int64_t p2, int64_t m_per_block,
                                                        int64_t lds_points,
                                                        const uint32_t *__restrict__ seedm,
                                                        unsigned long long *__restrict__ keys) {
    __shared__ float lds[kLdsFloats];
    const int64_t pair = blockIdx.y;
    const PairPtrs P = pair_ptrs(xs1, xs2, pair, b1, b2, p1, p2, D);
    const int64_t chunk = p2 < lds_points ? p2 : lds_points;
    for (int64_t t = threadIdx.x; t < chunk * D; t += kThreads) {
        const int64_t k = t / chunk, n = t - k * chunk;
        lds[t] = P.x2[k * p2 + n];
    }
    __syncthreads();

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t mbeg = (int64_t)blockIdx.x * m_per_block;
    const int64_t mend = mbeg + m_per_block < p1 ? mbeg + m_per_block : p1;
    unsigned long long *key = &keys[pair];
    for (int64_t m = mbeg + wave; m < mend; m += kThreads / 64) {
        if (is_seed(seedm, pair, m)) continue;  // the same in every lane
        float a[D];
#pragma unroll
        for (int k = 0; k < D; ++k) a[k] = P.x1[k * p1 + m];
        float T = threshold_of(key);
        float best = INFINITY;
        bool pruned = false;
        int64_t n0 = 0;
        for (; n0 < chunk; n0 += 64) {
            const int64_t n = n0 + lane;
            const float dd = n < chunk ? sqdist_fixed<D>(a, lds, chunk, n) : INFINITY;
            if (__any(dd < T)) {
                pruned = true;
                break;
            }
            best = fminf(best, dd);
        }
        if (!pruned) {
            for (; n0 < p2; n0 += 64) {
                const int64_t n = n0 + lane;
                const float dd = n < p2 ? sqdist_fixed<D>(a, P.x2, p2, n) : INFINITY;
                if (__any(dd < T)) {
                    pruned = true;
                    break;
                }
                best = fminf(best, dd);
                if ((n0 & 4095) == 4032) T = threshold_of(key);
            }
        }
        if (!pruned) {
            const float mn = wave_min(best);
            if (lane == 0) fold_key(key, mn, m);
        }
    }
}

// Generic-d variant (features in registers up to 64, x2 read from global memory).
__global__ __launch_bounds__(kThreads) void scan_kernel_any(const float *__restrict__ xs1,
                                                            const float *__restrict__ xs2,
                                                            int64_t b1, int64_t b2, int64_t p1,
                                                            int64_t p2, int d,
                                                            int64_t m_per_block,
                                                            unsigned long long *__restrict__ keys) {
    const int64_t pair = blockIdx.y;
    const PairPtrs P = pair_ptrs(xs1, xs2, pair, b1, b2, p1, p2, d);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t mbeg = (int64_t)blockIdx.x * m_per_block;
    const int64_t mend = mbeg + m_per_block < p1 ? mbeg + m_per_block : p1;
    unsigned long long *key = &keys[pair];
    for (int64_t m = mbeg + wave; m < mend; m += kThreads / 64) {
        float a[64];
        for (int k = 0; k < d; ++k) a[k] = P.x1[k * p1 + m];
        float T = threshold_of(key);
        float best = INFINITY;
        bool pruned = false;
        for (int64_t n0 = 0; n0 < p2; n0 += 64) {
            const int64_t n = n0 + lane;
            const float dd = n < p2 ? sqdist(a, P.x2, p2, n, d) : INFINITY;
            if (__any(dd < T)) {
                pruned = true;
                break;
            }
            best = fminf(best, dd);
            if ((n0 & 4095) == 4032) T = threshold_of(key);
        }
        if (!pruned) {
            const float mn = wave_min(best);
            if (lane == 0) fold_key(key, mn, m);
        }
    }
}

// One wave per pair: first n position reaching the winning m's min; write the outputs.
// D > 0: a fixed feature count (coordinates in registers); D == 0: any d <= 64.
template <int D>
__global__ __launch_bounds__(kThreads) void finalize_kernel(
    const float *__restrict__ xs1, const float *__restrict__ xs2,
    const unsigned long long *__restrict__ keys, const int64_t *__restrict__ perm1,
    const int64_t *__restrict__ perm2, int64_t pairs, int64_t b1, int64_t b2, int64_t p1,
    int64_t p2, int d, float *__restrict__ out, int64_t *__restrict__ idx1,
    int64_t *__restrict__ idx2) {
    const int64_t pair = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (pair >= pairs) return;
    const int64_t bb = pair / (b1 * b2);
    if (p1 == 0 || p2 == 0) {
        if (lane == 0) {
            out[pair] = 0.0f;
            idx1[pair] = 0;
            idx2[pair] = 0;
        }
        return;
    }
    const PairPtrs P = pair_ptrs(xs1, xs2, pair, b1, b2, p1, p2, d);
    const unsigned long long k = keys[pair];
    const int64_t m = (int64_t)(k & 0xffffffffull);
    const float H = __uint_as_float((uint32_t)(k >> 32));
    float a[D > 0 ? D : 64];
    if constexpr (D > 0) {
#pragma unroll
        for (int t = 0; t < D; ++t) a[t] = P.x1[(int64_t)t * p1 + m];
    } else {
        for (int t = 0; t < d && t < 64; ++t) a[t] = P.x1[(int64_t)t * p1 + m];
    }
    int64_t npos = p2;
    int64_t start = 0;
    if constexpr (D > 0) {
        // four 64-point chunks per step, their ballots taken in order (first hit wins)
        for (; start + 256 <= p2 && npos == p2; start += 256) {
            float dist[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) dist[u] = sqdist_fixed<D>(a, P.x2, p2, start + 64 * u + lane);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const unsigned long long mask = __ballot(dist[u] == H);
                if (mask && npos == p2) npos = start + 64 * u + __builtin_ctzll(mask);
            }
        }
    }
    for (int64_t n0 = start; n0 < p2 && npos == p2; n0 += 64) {
        const int64_t n = n0 + lane;
        float dist = 0.0f;
        if (n < p2) {
            if constexpr (D > 0) dist = sqdist_fixed<D>(a, P.x2, p2, n);
            else dist = sqdist(a, P.x2, p2, n, d);
        }
        const bool hit = n < p2 && dist == H;
        const unsigned long long mask = __ballot(hit);
        if (mask) {
            npos = n0 + __builtin_ctzll(mask);
            break;
        }
    }
    if (lane == 0) {
        out[pair] = sqrt_rn(H);
        idx1[pair] = perm1 ? perm1[bb * p1 + m] : m;
        idx2[pair] = npos < p2 ? (perm2 ? perm2[bb * p2 + npos] : npos) : 0;
    }
}

// Seeds and the final rescan for a fixed feature count D = 1..4, spread over many blocks per
// cloud pair.
//
// seed_select: block (pair, y) takes x1 points [y chunk, (y + 1) chunk) and each wave offers
// the point farthest from x2's bounding box as a candidate, cand[pair][4 y + wave] = (that
// squared distance's bits << 32 | m + 1); 0 = no point.
template <int D>
__global__ __launch_bounds__(kThreads) void seed_select_kernel(const float *__restrict__ xs1,
                                                               const float *__restrict__ bbox2, int64_t b1,
                                                               int64_t b2, int64_t p1, int64_t chunk,
                                                               int64_t ncand,
                                                               unsigned long long *__restrict__ cand) {
    const int64_t pair = blockIdx.x;
    const int64_t per_batch = b1 * b2;
    const int64_t bb = pair / per_batch, rem = pair - bb * per_batch;
    const int64_t i = rem / b2, j = rem - i * b2;
    const float *X1 = xs1 + (bb * b1 + i) * D * p1;
    float box[2 * D];
#pragma unroll
    for (int k = 0; k < 2 * D; ++k) box[k] = bbox2[(bb * b2 + j) * D * 2 + k];
    const int64_t beg = (int64_t)blockIdx.y * chunk;
    const int64_t end = beg + chunk < p1 ? beg + chunk : p1;
    unsigned long long best = 0;
    for (int64_t m = beg + threadIdx.x; m < end; m += kThreads) {
        float L = 0.0f;
#pragma unroll
        for (int k = 0; k < D; ++k) {
            const float v = X1[k * p1 + m];
            const float e = fmaxf(fmaxf(box[2 * k] - v, v - box[2 * k + 1]), 0.0f);
            L = L + e * e;
        }
        const unsigned long long key = ((unsigned long long)__float_as_uint(L) << 32) | (uint64_t)(m + 1);
        best = key > best ? key : best;
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) cand[pair * ncand + blockIdx.y * (kThreads / 64) + (threadIdx.x >> 6)] = best;
}

// seed_pick: one wave per pair takes the kSeeds largest candidate keys (keys are distinct; kSeeds
// rounds, each the largest key below the previous one, every lane holding the same reduced
// value) and writes their positions to seedm[pair][s] (0xffffffff = no candidate left).
__global__ __launch_bounds__(kThreads) void seed_pick_kernel(const unsigned long long *__restrict__ cand,
                                                             int64_t ncand, int64_t pairs,
                                                             uint32_t *__restrict__ seedm) {
    const int64_t pair = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (pair >= pairs) return;
    const int lane = threadIdx.x & 63;
    const unsigned long long *C = cand + pair * ncand;
    unsigned long long prev = ~0ull;
    for (int r = 0; r < kSeeds; ++r) {
        unsigned long long best = 0;
        for (int64_t e = lane; e < ncand; e += 64) {
            const unsigned long long v = C[e];
            if (v < prev && v > best) best = v;
        }
        best = wave_max_u64(best);
        if (lane == 0) seedm[pair * kSeeds + r] = best ? (uint32_t)(best & 0xffffffffull) - 1u : 0xffffffffu;
        prev = best ? best : prev;
    }
}

// Exact mins of listed x1 points, spread over blocks.  list[pair][0..K) holds x1 positions:
// with cnt, the first min(cnt[pair], K) entries; without, every entry but 0xffffffff (entry 0
// is then always valid).  Block (pair, y) takes the x2 points [y chunk, (y + 1) chunk) and, eight
// entries at a time, folds each entry's min over them into lmin[pair][e] (fp32 bits, preset to
// +inf) with atomicMin.
template <int D>
__global__ __launch_bounds__(kThreads) void list_scan_kernel(
    const float *__restrict__ xs1, const float *__restrict__ xs2, const uint32_t *__restrict__ list,
    const uint32_t *__restrict__ cnt, int64_t K, int64_t b1, int64_t b2, int64_t p1, int64_t p2, int64_t chunk,
    uint32_t *__restrict__ lmin) {
    constexpr int kGroup = 8;
    __shared__ float red[kThreads / 64][kGroup];
    const int64_t pair = blockIdx.x;
    const PairPtrs P = pair_ptrs(xs1, xs2, pair, b1, b2, p1, p2, D);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t *L = list + pair * K;
    const int64_t n = cnt ? std::min<int64_t>(cnt[pair], K) : K;
    const int64_t beg = (int64_t)blockIdx.y * chunk;
    const int64_t end = beg + chunk < p2 ? beg + chunk : p2;
    for (int64_t g0 = 0; g0 < n; g0 += kGroup) {
        uint32_t ms[kGroup];
        float a[kGroup][D];
#pragma unroll
        for (int s = 0; s < kGroup; ++s) {
            ms[s] = g0 + s < n ? L[g0 + s] : 0xffffffffu;
            const uint32_t m = ms[s] == 0xffffffffu ? L[g0] : ms[s];  // L[g0] is valid
#pragma unroll
            for (int k = 0; k < D; ++k) a[s][k] = P.x1[k * p1 + m];
        }
        float best[kGroup];
#pragma unroll
        for (int s = 0; s < kGroup; ++s) best[s] = INFINITY;
        // four points per thread and step, their loads in flight together
        for (int64_t q0 = beg + threadIdx.x; q0 < end; q0 += 4 * kThreads) {
            float b[4][D];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t q = q0 + u * kThreads;
                const bool ok = q < end;
                const int64_t qq = ok ? q : q0;
#pragma unroll
                for (int k = 0; k < D; ++k) b[u][k] = P.x2[k * p2 + qq];
                // a missing point: d = inf or NaN, which fminf passes over
                b[u][0] = ok ? b[u][0] : INFINITY;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
#pragma unroll
                for (int s = 0; s < kGroup; ++s) {
                    float acc = 0.0f;
#pragma unroll
                    for (int k = 0; k < D; ++k) {
                        const float diff = a[s][k] - b[u][k];
                        acc = acc + diff * diff;
                    }
                    best[s] = fminf(best[s], acc);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < kGroup; ++s) {
            const float v = wave_min(best[s]);
            if (lane == 0) red[wave][s] = v;
        }
        __syncthreads();
        if (threadIdx.x < kGroup) {
            const int s = threadIdx.x;
            float v = red[0][s];
            for (int w = 1; w < kThreads / 64; ++w) v = fminf(v, red[w][s]);
            if (ms[s] != 0xffffffffu) atomicMin(&lmin[pair * K + g0 + s], __float_as_uint(v));
        }
        __syncthreads();
    }
}

// Each listed point's exact min (the fold of all list_scan blocks) goes into its pair's key.
__global__ void list_fold_kernel(const uint32_t *__restrict__ lmin, const uint32_t *__restrict__ list,
                                 const uint32_t *__restrict__ cnt, int64_t K, int64_t pairs,
                                 unsigned long long *__restrict__ keys) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= pairs * K) return;
    const int64_t pair = t / K, e = t - pair * K;
    const bool valid = cnt ? e < (int64_t)cnt[pair] : list[t] != 0xffffffffu;
    if (valid) fold_key(&keys[pair], __uint_as_float(lmin[t]), list[t]);
}

// Final rescan: block (pair, y) checks the x2 points [y chunk, (y + 1) chunk) against the
// winning m of the pair's key and folds the first position n whose d equals the min into
// first[pair] (preset to all ones) with atomicMin.
template <int D>
__global__ __launch_bounds__(kThreads) void first_hit_kernel(
    const float *__restrict__ xs1, const float *__restrict__ xs2, const unsigned long long *__restrict__ keys,
    int64_t b1, int64_t b2, int64_t p1, int64_t p2, int64_t chunk, unsigned long long *__restrict__ first) {
    __shared__ unsigned long long red[kThreads / 64];
    const int64_t pair = blockIdx.x;
    const PairPtrs P = pair_ptrs(xs1, xs2, pair, b1, b2, p1, p2, D);
    const unsigned long long key = keys[pair];
    const int64_t m = (int64_t)(key & 0xffffffffull);
    const float H = __uint_as_float((uint32_t)(key >> 32));
    float a[D];
#pragma unroll
    for (int k = 0; k < D; ++k) a[k] = P.x1[k * p1 + m];
    const int64_t beg = (int64_t)blockIdx.y * chunk;
    const int64_t end = beg + chunk < p2 ? beg + chunk : p2;
    unsigned long long hit = ~0ull;
    int64_t n = beg + threadIdx.x;
    for (; n + 3 * kThreads < end; n += 4 * kThreads) {
        float dd[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) dd[u] = sqdist_fixed<D>(a, P.x2, p2, n + u * kThreads);
#pragma unroll
        for (int u = 3; u >= 0; --u)
            if (dd[u] == H) hit = (unsigned long long)(n + u * kThreads);
        if (hit != ~0ull) break;
    }
    for (; n < end && hit == ~0ull; n += kThreads)
        if (sqdist_fixed<D>(a, P.x2, p2, n) == H) hit = (unsigned long long)n;
    hit = wave_min_u64(hit);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = hit;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kThreads / 64; ++w) hit = red[w] < hit ? red[w] : hit;
        if (hit != ~0ull) atomicMin(&first[pair], hit);
    }
}

// One thread per pair: sqrt of the winning min, and the (permuted) positions of m and n.
__global__ void write_out_kernel(const unsigned long long *__restrict__ keys,
                                 const unsigned long long *__restrict__ first, const int64_t *__restrict__ perm1,
                                 const int64_t *__restrict__ perm2, int64_t pairs, int64_t b1, int64_t b2,
                                 int64_t p1, int64_t p2, float *__restrict__ out, int64_t *__restrict__ idx1,
                                 int64_t *__restrict__ idx2) {
    const int64_t pair = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (pair >= pairs) return;
    const int64_t bb = pair / (b1 * b2);
    const unsigned long long key = keys[pair];
    const int64_t m = (int64_t)(key & 0xffffffffull);
    const unsigned long long n = first[pair];
    out[pair] = sqrt_rn(__uint_as_float((uint32_t)(key >> 32)));
    idx1[pair] = perm1 ? perm1[bb * p1 + m] : m;
    idx2[pair] = n < (unsigned long long)p2 ? (perm2 ? perm2[bb * p2 + (int64_t)n] : (int64_t)n) : 0;
}

// grad_x1[bb,i,m*,k] += g * (x1[m*,k] - x2[n*,k]) / out, over j in order (one thread per
// (bb, i, k) owns every update of its slice, so the summation order is the reference's).
__global__ void backward_x1_kernel(const float *__restrict__ g, const float *__restrict__ x1,
                                   const float *__restrict__ x2, const float *__restrict__ out,
                                   const int64_t *__restrict__ idx1,
                                   const int64_t *__restrict__ idx2, int64_t batch, int64_t b1,
                                   int64_t p1, int64_t b2, int64_t p2, int64_t d,
                                   float *__restrict__ gx1) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= batch * b1 * d) return;
    const int64_t k = t % d, i = (t / d) % b1, bb = t / (d * b1);
    for (int64_t j = 0; j < b2; ++j) {
        const int64_t pr = (bb * b1 + i) * b2 + j;
        const int64_t m = idx1[pr], n = idx2[pr];
        const float diff = x1[((bb * b1 + i) * p1 + m) * d + k] - x2[((bb * b2 + j) * p2 + n) * d + k];
        float *dst = gx1 + ((bb * b1 + i) * p1 + m) * d + k;
        *dst = *dst + g[pr] * diff / out[pr];
    }
}

__global__ void backward_x2_kernel(const float *__restrict__ g, const float *__restrict__ x1,
                                   const float *__restrict__ x2, const float *__restrict__ out,
                                   const int64_t *__restrict__ idx1,
                                   const int64_t *__restrict__ idx2, int64_t batch, int64_t b1,
                                   int64_t p1, int64_t b2, int64_t p2, int64_t d,
                                   float *__restrict__ gx2) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= batch * b2 * d) return;
    const int64_t k = t % d, j = (t / d) % b2, bb = t / (d * b2);
    for (int64_t i = 0; i < b1; ++i) {
        const int64_t pr = (bb * b1 + i) * b2 + j;
        const int64_t m = idx1[pr], n = idx2[pr];
        const float diff = x2[((bb * b2 + j) * p2 + n) * d + k] - x1[((bb * b1 + i) * p1 + m) * d + k];
        float *dst = gx2 + ((bb * b2 + j) * p2 + n) * d + k;
        *dst = *dst + g[pr] * diff / out[pr];
    }
}

// The scatter with a wave per cloud (x1's clouds, then x2's), for at most 64 clouds on the
// other side, into zero-filled gradients: lane o takes the cloud's o-th pair (x1 cloud
// c = bb b1 + i: pair (c, o); x2 cloud bb b2 + j: pair (bb b1 + o, j)), its target position and,
// per feature, its term g (own - other) / out.  Each lane then adds, over the pairs in order
// from +0, the terms of those with its target, and the last lane of each target stores the sum:
// the sequential loop's additions in its order, so the same bits, with the pairs' loads in
// parallel instead of one dependent round of loads and a read-modify-write per pair.
__global__ __launch_bounds__(256) void backward_wave_kernel(
    const float *__restrict__ g, const float *__restrict__ x1, const float *__restrict__ x2,
    const float *__restrict__ out, const int64_t *__restrict__ idx1, const int64_t *__restrict__ idx2, int64_t batch,
    int64_t b1, int64_t p1, int64_t b2, int64_t p2, int64_t d, float *__restrict__ gx1, float *__restrict__ gx2) {
    const int64_t cy = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t clouds1 = batch * b1;
    if (cy >= clouds1 + batch * b2) return;  // the same in every lane
    const bool side1 = cy < clouds1;
    const int64_t c = side1 ? cy : cy - clouds1;
    const int64_t bb = side1 ? c / b1 : c / b2, j2 = c - bb * b2;
    const int other = (int)(side1 ? b2 : b1);
    const int64_t pr = lane >= other ? 0 : side1 ? c * b2 + lane : (bb * b1 + lane) * b2 + j2;
    const int64_t m = idx1[pr], n = idx2[pr];
    // lanes past the cloud count, and pairs with an index outside its cloud, take no part
    const bool act = lane < other && m >= 0 && m < p1 && n >= 0 && n < p2;
    const int64_t tgt = act ? (side1 ? m : n) : -1;
    const float gv = g[pr], ov = out[pr];
    // own / other rows of the lane's pair
    const float *own = side1 ? x1 + (c * p1 + m) * d : x2 + (c * p2 + n) * d;
    const float *oth = side1 ? x2 + ((bb * b2 + lane) * p2 + n) * d : x1 + ((bb * b1 + lane) * p1 + m) * d;
    float *dst = side1 ? gx1 + (c * p1 + m) * d : gx2 + (c * p2 + n) * d;
    // the last lane of each target stores (every lane runs every shuffle: a shuffle from a lane
    // that is not running returns nothing of use)
    bool last = act;
    for (int o = 0; o < other; ++o) {
        const int64_t to = __shfl(tgt, o, 64);
        last = last && !(o > lane && to == tgt);
    }
    for (int64_t k = 0; k < d; ++k) {
        const float diff = act ? own[k] - oth[k] : 0.0f;
        const float term = gv * diff / ov;
        float acc = 0.0f;
        for (int o = 0; o < other; ++o) {
            const float t = __shfl(term, o, 64);
            if (__shfl(tgt, o, 64) == tgt) acc = acc + t;
        }
        if (last) dst[k] = acc;
    }
}

// ---------------------------------------------------------------------------------------
// Scan with a spatial first guess (D = 1, 2, 3).  Pruning an m needs only one distance below
// T, and an m that is never pruned gets its exact min whatever order x2 is visited in.  Each
// x2 cloud is therefore counting-sorted once by a grid cell (4096 cells over the cloud's
// bounding box; Morton order of 16^3 / 64^2 cells, or 4096 intervals for D = 1), and the scan
// first tries, for every m, the 64 sorted points at m's own cell, which almost always hold
// one within T.  x1 stays in iteration order, so the m that need more (points far from x2,
// with mins near T) are spread evenly over the waves.
constexpr int kCells = 4096;

// The cell scan takes a pair's cells in a scattered order, position (c * 0x9b1) mod 4096 for
// cell c (an odd multiplier: a permutation, which mixes every bit of c into the high bits), so
// that cells that need more work, which cluster in space, spread evenly over its blocks.
// Per-cell data it reads is stored by position, so that its loads stay contiguous.
__device__ __forceinline__ int pos_cell(int c) { return (c * 0x9b1) & (kCells - 1); }


template <int D>
__device__ __forceinline__ uint32_t spread_bits(uint32_t v) {
    if constexpr (D == 3) {  // 4 bits -> every third bit
        v &= 0xfu;
        v = (v | (v << 4)) & 0x0c3u;
        v = (v | (v << 2)) & 0x249u;
        return v;
    } else {  // D == 2: 6 bits -> every second bit
        v &= 0x3fu;
        v = (v | (v << 4)) & 0x30fu;
        v = (v | (v << 2)) & 0x333u;
        v = (v | (v << 1)) & 0x555u;
        return v;
    }
}

// Inverse of spread_bits: every third (D = 3) or second (D = 2) bit back to 4 or 6 bits.
template <int D>
__device__ __forceinline__ uint32_t compact_bits(uint32_t v) {
    if constexpr (D == 3) {
        v &= 0x249u;
        v = (v | (v >> 2)) & 0x0c3u;
        v = (v | (v >> 4)) & 0x00fu;
        return v;
    } else {
        v &= 0x555u;
        v = (v | (v >> 1)) & 0x333u;
        v = (v | (v >> 2)) & 0x30fu;
        v = (v | (v >> 4)) & 0x03fu;
        return v;
    }
}

// Cell of a point in a frame (lo[k], cells per unit[k]); coordinates outside it clamp to the
// nearest boundary cell and NaN goes to cell 0.
template <int D>
__device__ __forceinline__ uint32_t cell_of(const float (&a)[D], const float (&fr)[2 * D]) {
    constexpr int kBits = D == 3 ? 4 : D == 2 ? 6 : 12;
    constexpr float kMax = (float)((1 << kBits) - 1);
    uint32_t c = 0;
#pragma unroll
    for (int k = 0; k < D; ++k) {
        const float q = fminf(fmaxf((a[k] - fr[2 * k]) * fr[2 * k + 1], 0.0f), kMax);
        const uint32_t u = (uint32_t)q;
        if constexpr (D == 1) c = u;
        else c |= spread_bits<D>(u) << k;
    }
    return c;
}

// The frame of an x2 cloud from its bounding box (bbox[k][0..1]).
template <int D>
__device__ __forceinline__ void frame_of(const float *box, float (&fr)[2 * D]) {
    constexpr int kBits = D == 3 ? 4 : D == 2 ? 6 : 12;
#pragma unroll
    for (int k = 0; k < D; ++k) {
        const float lo = box[2 * k], span = box[2 * k + 1] - lo;
        fr[2 * k] = lo == lo ? lo : 0.0f;
        fr[2 * k + 1] = span > 0.0f && span < INFINITY ? (float)(1 << kBits) / span : 0.0f;
    }
}

// One side's clouds for the cell sort: the input as given ([clouds][p][D]; when perm is given,
// iteration position pos of cloud c is row perm[c / cpb][pos]), the records to write
// ([clouds][p]) and the frames (boxes[c / cpf][D][2]).
struct CellSet {
    const float *x;
    const int64_t *perm;
    float4 *rec;
    const float *boxes;
    int64_t clouds, p, cpb, cpf;
};

// Counting sort of one cloud (block) of S by cell into records, with, when given, the cloud's
// cell start offsets (cstart[c][kCells + 1]; cstartT[c][pos(cell)] the same starts in the cell
// scan's order).  Points of one cell land in an unspecified order
// (LDS atomics); nothing depends on it.
template <int D>
__global__ __launch_bounds__(kThreads) void cell_sort_kernel(CellSet S, int32_t *__restrict__ cstart,
                                                             int32_t *__restrict__ cstartT) {
    __shared__ uint32_t cnt[kCells];
    __shared__ uint32_t part[kThreads];
    const int64_t c = blockIdx.x;
    const int64_t p = S.p;
    float fr[2 * D];
    frame_of<D>(S.boxes + (c / S.cpf) * D * 2, fr);
    for (int t = threadIdx.x; t < kCells; t += kThreads) cnt[t] = 0u;
    __syncthreads();
    for (int64_t n = threadIdx.x; n < p; n += kThreads) {
        float a[D];
        point_at<D>(S.x, S.perm, c, S.cpb, p, n, a);
        atomicAdd(&cnt[cell_of<D>(a, fr)], 1u);
    }
    __syncthreads();
    constexpr int kPer = kCells / kThreads;  // exclusive scan: 16 consecutive cells per thread
    uint32_t local = 0;
#pragma unroll
    for (int e = 0; e < kPer; ++e) local += cnt[threadIdx.x * kPer + e];
    part[threadIdx.x] = local;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t run = 0;
        for (int t = 0; t < kThreads; ++t) {
            const uint32_t v = part[t];
            part[t] = run;
            run += v;
        }
    }
    __syncthreads();
    uint32_t run = part[threadIdx.x];
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
        const int cell = threadIdx.x * kPer + e;
        const uint32_t v = cnt[cell];
        cnt[cell] = run;
        if (cstart) cstart[c * (kCells + 1) + cell] = (int32_t)run;
        if (cstartT) cstartT[c * kCells + pos_cell(cell)] = (int32_t)run;
        run += v;
    }
    if (cstart && threadIdx.x == 0) cstart[c * (kCells + 1) + kCells] = (int32_t)p;
    __syncthreads();
    float4 *O = S.rec + c * p;
    for (int64_t n = threadIdx.x; n < p; n += kThreads) {
        float a[D];
        point_at<D>(S.x, S.perm, c, S.cpb, p, n, a);
        const uint32_t slot = atomicAdd(&cnt[cell_of<D>(a, fr)], 1u);
        O[slot] = make_rec<D>(a, (uint32_t)n);
    }
}

// The same counting sort spread over many blocks per cloud, for runs with few clouds (one
// block per cloud would leave most CUs idle), with no global atomics.  Clouds [0, A.clouds)
// come from A, the rest from B; hist[cloud][chunk][cell] holds each chunk's histogram and then
// its first slot in every cell.
//   cell_count: block (cloud, y) histograms positions [y chunk, (y + 1) chunk) in LDS and
//     writes it out;
//   cell_offsets: per cloud, the cell starts (starts[cloud], A's clouds first; A's also in the
//     cell scan's order, startsA_T, when given) and each chunk's first slot in every cell (the
//     start plus the earlier chunks' counts);
//   cell_scatter: block (cloud, y) writes its points from those slots on, the slot within a
//     cell taken with an LDS atomicAdd.
template <int D>
__global__ __launch_bounds__(kThreads) void cell_count_kernel(CellSet A, CellSet B, int64_t chunk, int64_t chunks,
                                                              uint32_t *__restrict__ hist_out) {
    __shared__ uint32_t hist[kCells];
    const int64_t g = blockIdx.x;
    const bool inA = g < A.clouds;
    const CellSet &S = inA ? A : B;
    const int64_t c = inA ? g : g - A.clouds;
    const int64_t beg = (int64_t)blockIdx.y * chunk;
    const int64_t end = beg + chunk < S.p ? beg + chunk : S.p;  // empty when beg >= p
    float fr[2 * D];
    frame_of<D>(S.boxes + (c / S.cpf) * D * 2, fr);
    for (int t = threadIdx.x; t < kCells; t += kThreads) hist[t] = 0u;
    __syncthreads();
    for (int64_t n = beg + threadIdx.x; n < end; n += kThreads) {
        float a[D];
        point_at<D>(S.x, S.perm, c, S.cpb, S.p, n, a);
        atomicAdd(&hist[cell_of<D>(a, fr)], 1u);
    }
    __syncthreads();
    uint32_t *H = hist_out + (g * chunks + blockIdx.y) * kCells;
    for (int t = threadIdx.x; t < kCells; t += kThreads) H[t] = hist[t];
}

constexpr int kOffThreads = 1024;

__global__ __launch_bounds__(kOffThreads) void cell_offsets_kernel(CellSet A, CellSet B, int64_t chunks,
                                                                   uint32_t *__restrict__ hist,
                                                                   int32_t *__restrict__ starts,
                                                                   int32_t *__restrict__ startsA_T) {
    __shared__ uint32_t tot[kCells];
    __shared__ uint32_t wsum[kOffThreads / 64];
    const int64_t g = blockIdx.x;
    const CellSet &S = g < A.clouds ? A : B;
    uint32_t *H = hist + g * chunks * kCells;
    constexpr int kPer = kCells / kOffThreads;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    // per-cell totals: thread t sums cells t + 1024 e over the chunks, four chunks of its four
    // cells in flight at a time
    uint32_t run4[kPer] = {};
    int64_t y = 0;
    for (; y + 4 <= chunks; y += 4) {
        uint32_t v[4][kPer];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < kPer; ++e) v[u][e] = H[(y + u) * kCells + t + e * kOffThreads];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < kPer; ++e) run4[e] += v[u][e];
    }
    for (; y < chunks; ++y)
#pragma unroll
        for (int e = 0; e < kPer; ++e) run4[e] += H[y * kCells + t + e * kOffThreads];
#pragma unroll
    for (int e = 0; e < kPer; ++e) tot[t + e * kOffThreads] = run4[e];
    __syncthreads();
    // exclusive scan over cells: thread t owns cells kPer t .. kPer t + kPer - 1
    uint32_t v[kPer], local = 0;
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
        v[e] = tot[kPer * t + e];
        local += v[e];
    }
    uint32_t incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = (uint32_t)__shfl_up((int)incl, off, 64);
        if (lane >= off) incl += o;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    if (t == 0) {
        uint32_t run = 0;
        for (int w = 0; w < kOffThreads / 64; ++w) {
            const uint32_t x = wsum[w];
            wsum[w] = run;
            run += x;
        }
    }
    __syncthreads();
    uint32_t run = wsum[wave] + incl - local;
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
        tot[kPer * t + e] = run;
        run += v[e];
    }
    __syncthreads();
    // starts, and each chunk's first slot per cell (four chunks of the four cells at a time)
    int32_t *St = starts + g * (kCells + 1);
    uint32_t sl[kPer];
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
        const int cell = t + e * kOffThreads;
        sl[e] = tot[cell];
        St[cell] = (int32_t)sl[e];
        if (startsA_T && g < A.clouds) startsA_T[g * kCells + pos_cell(cell)] = (int32_t)sl[e];
    }
    y = 0;
    for (; y + 4 <= chunks; y += 4) {
        uint32_t v[4][kPer];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < kPer; ++e) v[u][e] = H[(y + u) * kCells + t + e * kOffThreads];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < kPer; ++e) {
                H[(y + u) * kCells + t + e * kOffThreads] = sl[e];
                sl[e] += v[u][e];
            }
    }
    for (; y < chunks; ++y)
#pragma unroll
        for (int e = 0; e < kPer; ++e) {
            const uint32_t n = H[y * kCells + t + e * kOffThreads];
            H[y * kCells + t + e * kOffThreads] = sl[e];
            sl[e] += n;
        }
    if (t == 0) St[kCells] = (int32_t)S.p;
}

template <int D>
__global__ __launch_bounds__(kThreads) void cell_scatter_kernel(CellSet A, CellSet B, int64_t chunk, int64_t chunks,
                                                                const uint32_t *__restrict__ slots) {
    __shared__ uint32_t next[kCells];
    const int64_t g = blockIdx.x;
    const bool inA = g < A.clouds;
    const CellSet &S = inA ? A : B;
    const int64_t c = inA ? g : g - A.clouds;
    const int64_t beg = (int64_t)blockIdx.y * chunk;
    if (beg >= S.p) return;  // the same for the whole block
    const int64_t end = beg + chunk < S.p ? beg + chunk : S.p;
    float fr[2 * D];
    frame_of<D>(S.boxes + (c / S.cpf) * D * 2, fr);
    const uint32_t *H = slots + (g * chunks + blockIdx.y) * kCells;
    for (int t = threadIdx.x; t < kCells; t += kThreads) next[t] = H[t];
    __syncthreads();
    float4 *O = S.rec + c * S.p;
    for (int64_t n = beg + threadIdx.x; n < end; n += kThreads) {
        float a[D];
        point_at<D>(S.x, S.perm, c, S.cpb, S.p, n, a);
        const uint32_t slot = atomicAdd(&next[cell_of<D>(a, fr)], 1u);
        O[slot] = make_rec<D>(a, (uint32_t)n);
    }
}

// ---------------------------------------------------------------------------------------
// Exact nearest-neighbour search over the cell grid, by one wave.  The query's cell c0 (its
// coordinates clamped into the grid, as cell_of does) is visited first, then the rings of cells
// at Chebyshev distance R = 1, 2, ... around it.  A cell is scanned only when a lower bound of
// the squared distance from the query to any point assigned to it is not above the current
// bound; the search ends at the first ring whose lower bound is above it.  Both bounds are
// conservative: a point's cell comes from the rounded (x - lo) * scale (off by far less than the
// 0.01-cell margin taken off every gap), edge cells reach to infinity (clamping), and the bound
// is scaled by 1 - 2^-12 for the rounding of the computed distances.  The ring's cells are
// taken 64 at a time: the candidates among them are scanned together, their points packed 64 to
// a step.  Visiting order does not change a min, so the result is that of a scan of all of x2.
//   kBallPrune: drop the query at the first d < T (returns true); otherwise fold the exact min
//     with position mpos into key (returns false);
//   kBallMin: return the exact min (out_min);
//   kBallFirst: return the smallest position of a point with d == H (all ones if none).
// evals (per lane) is raised by the number of points the lane evaluated.
constexpr int kBallPrune = 0, kBallMin = 1, kBallFirst = 2;

template <int D>
__device__ __forceinline__ constexpr int grid_side() { return D == 3 ? 16 : D == 2 ? 64 : 4096; }

// Offsets of cell t of ring R (0 <= t < ring_count(R)) around the query's cell.
template <int D>
__device__ __forceinline__ int64_t ring_count(int R) {
    if (R == 0) return 1;
    if constexpr (D == 1) return 2;
    else if constexpr (D == 2) return 8 * (int64_t)R;
    else return 24 * (int64_t)R * R + 2;
}
template <int D>
__device__ __forceinline__ void ring_cell(int R, int64_t t, int (&o)[D]) {
    if constexpr (D == 1) {
        o[0] = R == 0 ? 0 : (t == 0 ? -R : R);
    } else if constexpr (D == 2) {
        const int S = 2 * R + 1;
        if (R == 0) {
            o[0] = o[1] = 0;
        } else if (t < 2 * S) {  // bottom and top rows
            o[0] = (int)(t % S) - R;
            o[1] = t < S ? -R : R;
        } else {                 // left and right columns without the corners
            const int64_t u = t - 2 * S;
            o[0] = u < S - 2 ? -R : R;
            o[1] = (int)(u % (S - 2)) - (R - 1);
        }
    } else {
        const int S = 2 * R + 1;
        if (R == 0) {
            o[0] = o[1] = o[2] = 0;
        } else if (t < 2 * (int64_t)S * S) {  // faces z = -R, +R
            const int64_t r = t % ((int64_t)S * S);
            o[0] = (int)(r % S) - R;
            o[1] = (int)(r / S) - R;
            o[2] = t < (int64_t)S * S ? -R : R;
        } else if (t < 2 * (int64_t)S * S + 2 * (int64_t)S * (S - 2)) {  // faces y = -R, +R, |z| < R
            const int64_t u = t - 2 * (int64_t)S * S;
            const int64_t r = u % ((int64_t)S * (S - 2));
            o[0] = (int)(r % S) - R;
            o[1] = u < (int64_t)S * (S - 2) ? -R : R;
            o[2] = (int)(r / S) - (R - 1);
        } else {  // faces x = -R, +R, |y|, |z| < R
            const int64_t u = t - 2 * (int64_t)S * S - 2 * (int64_t)S * (S - 2);
            const int64_t r = u % ((int64_t)(S - 2) * (S - 2));
            o[0] = u < (int64_t)(S - 2) * (S - 2) ? -R : R;
            o[1] = (int)(r % (S - 2)) - (R - 1);
            o[2] = (int)(r / (S - 2)) - (R - 1);
        }
    }
}

template <int D, int MODE>
__device__ unsigned long long wave_ball_query(const float (&q)[D], const float4 *X2, const int32_t *CS,
                                              const float (&fr)[2 * D], float T, unsigned long long *key,
                                              int64_t mpos, float *out_min, uint32_t &evals) {
    constexpr int G = grid_side<D>();
    constexpr float kMargin = 0.01f, kShrink = 1.0f - 0x1p-12f;
    const int lane = threadIdx.x & 63;
    float f[D], inv[D];
    int c0[D];
#pragma unroll
    for (int k = 0; k < D; ++k) {
        f[k] = (q[k] - fr[2 * k]) * fr[2 * k + 1];
        c0[k] = (int)fminf(fmaxf(f[k], 0.0f), (float)(G - 1));
        inv[k] = fr[2 * k + 1] > 0.0f ? 1.0f / fr[2 * k + 1] : 0.0f;  // 0: one cell along k
    }
    float best = INFINITY;                 // per lane, then wave-wide at each ring
    unsigned long long first = ~0ull;      // kBallFirst
    const float bound0 = MODE == kBallFirst ? T : INFINITY;
    for (int R = 0; R < G; ++R) {
        float bound = MODE == kBallFirst ? bound0 : wave_min(best);
        if (R > 0) {
            // every cell of ring R (and beyond) is at least R - 1 cells away along some axis
            float lb = INFINITY;
            bool inside = false;
#pragma unroll
            for (int k = 0; k < D; ++k) {
                if (inv[k] > 0.0f) {
                    const float g = fmaxf((float)(R - 1) - kMargin, 0.0f) * inv[k];
                    lb = fminf(lb, g * g);
                }
                inside = inside || c0[k] - R >= 0 || c0[k] + R <= G - 1;
            }
            if (!inside) break;  // the ring lies outside the grid, and so do the later ones
            if (lb * kShrink > bound) break;
        }
        const int64_t count = ring_count<D>(R);
        for (int64_t t0 = 0; t0 < count; t0 += 64) {
            const int64_t t = t0 + lane;
            int32_t cs = 0, cn = 0;  // the lane's candidate cell: its points (none: cn = 0)
            if (t < count) {
                int o[D];
                ring_cell<D>(R, t, o);
                bool in = true;
                float lbc = 0.0f;
                uint32_t morton = 0;
#pragma unroll
                for (int k = 0; k < D; ++k) {
                    const int c = c0[k] + o[k];
                    in = in && c >= 0 && c <= G - 1;
                    const float lo = c == 0 ? -INFINITY : (float)c;
                    const float hi = c == G - 1 ? INFINITY : (float)(c + 1);
                    const float gap = fmaxf(fmaxf(lo - f[k], f[k] - hi) - kMargin, 0.0f) * inv[k];
                    lbc = lbc + gap * gap;
                    const uint32_t u = (uint32_t)(c < 0 ? 0 : c > G - 1 ? G - 1 : c);  // used only in grid
                    if constexpr (D == 1) morton = u;
                    else morton |= spread_bits<D>(u) << k;
                }
                if (in && !(lbc * kShrink > bound)) {
                    cs = CS[morton];
                    cn = CS[morton + 1] - cs;
                }
            }
            // the candidate cells' points, packed 64 per step: point g of the chunk belongs to
            // the lane r with the largest exclusive prefix of the counts that is <= g (prefixes
            // do not decrease over the lanes; a lane after the owner starts past g)
            uint32_t incl = (uint32_t)cn;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t o = (uint32_t)__shfl_up((int)incl, off, 64);
                if (lane >= off) incl += o;
            }
            const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
            const uint32_t excl = incl - (uint32_t)cn;
            for (uint32_t b0 = 0; b0 < total; b0 += 64) {
                const uint32_t g = b0 + (uint32_t)lane;
                const bool ok = g < total;
                int r = 0;
#pragma unroll
                for (int step = 32; step > 0; step >>= 1)
                    if ((uint32_t)__shfl((int)excl, r + step, 64) <= g) r += step;
                const int32_t n = __shfl(cs, r, 64) + (int32_t)(g - (uint32_t)__shfl((int)excl, r, 64));
                const float4 v = X2[ok ? n : 0];
                const float d = ok ? rec_dist<D>(q, v) : INFINITY;
                evals += ok ? 1u : 0u;
                if constexpr (MODE == kBallPrune) {
                    if (__any(d < T)) return 1ull;
                }
                if constexpr (MODE == kBallFirst) {
                    const unsigned long long pos = rec_pos(v);
                    if (ok && d == T && pos < first) first = pos;
                } else {
                    best = fminf(best, d);
                }
            }
        }
    }
    if constexpr (MODE == kBallFirst) {
        return wave_min_u64(first);
    } else {
        const float mn = wave_min(best);
        if constexpr (MODE == kBallPrune) {
            if (lane == 0) fold_key(key, mn, mpos);
        } else {
            *out_min = mn;
        }
        return 0ull;
    }
}

// Start of m's 64-point window in the sorted x2 of a cloud: its cell's first point, clamped to
// a full window.
template <int D>
__device__ __forceinline__ int64_t window_start(const float (&a)[D], const float (&fr)[2 * D],
                                                const int32_t *CS, int64_t p2) {
    const int64_t wstart = p2 > 64 ? p2 - 64 : 0;
    const int64_t s0 = (int64_t)CS[cell_of<D>(a, fr)];
    return s0 > wstart ? wstart : s0;
}

// Scan of the unsorted mode (x1 in iteration order, SoA; x2 sorted in its cloud's own frame):
// block = 2048 consecutive m of one pair; each wave takes 64 m at a time, one per lane.  A lane
// checks the 64 sorted x2 points of its window, first the head of its own cell (which almost
// always holds a point within T), and stops at the first d < T; the pair's seeds have their
// exact mins in the key already and are skipped.  The lanes left (ballot) are taken in turn by
// the whole wave through a ball query.
template <int D>
__global__ __launch_bounds__(kThreads) void scan_window_kernel(
    const float *__restrict__ xs1, const float4 *__restrict__ xs2r, const int32_t *__restrict__ cstart2,
    const float *__restrict__ boxes, int64_t b1, int64_t b2, int64_t p1, int64_t p2, int64_t m_per_block,
    const uint32_t *__restrict__ seedm, unsigned long long *__restrict__ keys, unsigned long long *__restrict__ counts) {
    const int64_t pair = blockIdx.y;
    const int64_t per_batch = b1 * b2;
    const int64_t bb = pair / per_batch, rem = pair - bb * per_batch;
    const int64_t i = rem / b2, j = rem - i * b2;
    const float *X1 = xs1 + (bb * b1 + i) * D * p1;
    const float4 *X2 = xs2r + (bb * b2 + j) * p2;
    const int32_t *CS = cstart2 + (bb * b2 + j) * (kCells + 1);
    float fr[2 * D];
    frame_of<D>(boxes + (bb * b2 + j) * D * 2, fr);
    const int lane = threadIdx.x & 63;
    const int64_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // the same in every lane
    const int64_t mbeg = (int64_t)blockIdx.x * m_per_block;
    const int64_t mend = mbeg + m_per_block < p1 ? mbeg + m_per_block : p1;
    const int64_t wlen = p2 < 64 ? p2 : 64;
    unsigned long long *key = &keys[pair];
    uint32_t evals = 0;
    // four groups of 64 m per step (m0, m0 + 256, ...), so that their dependent loads (point,
    // cell start, window) overlap
    constexpr int kG = 4;
    for (int64_t m0 = mbeg + 64 * wave; m0 < mend; m0 += kG * kThreads) {
        float a[kG][D];
        int64_t s0[kG];
        bool done[kG];
#pragma unroll
        for (int g = 0; g < kG; ++g) {
            const int64_t m = m0 + g * kThreads + lane;
            const bool valid = m < mend;
#pragma unroll
            for (int k = 0; k < D; ++k) a[g][k] = X1[k * p1 + (valid ? m : mbeg)];  // mbeg < p1
            done[g] = !valid;
        }
#pragma unroll
        for (int g = 0; g < kG; ++g) s0[g] = window_start<D>(a[g], fr, CS, p2);
        const float T = threshold_of(key);
        // two points first (the head of m's own cell), then 8 per step so that their loads are
        // in flight together (fewer in all when p2 < 64)
#pragma unroll
        for (int g = 0; g < kG; ++g) {
            bool hit = false;
            if (!done[g]) {
#pragma unroll
                for (int u = 0; u < 2; ++u)
                    if (u < wlen) hit = hit | (rec_dist<D>(a[g], X2[s0[g] + u]) < T);
                evals += wlen < 2 ? (uint32_t)wlen : 2u;
            }
            done[g] = done[g] || hit || is_seed(seedm, pair, m0 + g * kThreads + lane);
        }
#pragma unroll
        for (int g = 0; g < kG; ++g) {
            for (int64_t t = 2; t < wlen && !done[g]; t += 8) {
                bool hit = false;
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (t + u < wlen) hit = hit | (rec_dist<D>(a[g], X2[s0[g] + t + u]) < T);
                evals += wlen - t < 8 ? (uint32_t)(wlen - t) : 8u;
                done[g] = hit;
            }
        }
#pragma unroll
        for (int g = 0; g < kG; ++g) {
            unsigned long long left = __ballot(!done[g]);
            while (left) {
                const int l = __builtin_ctzll(left);
                left &= left - 1;
                float b[D];
#pragma unroll
                for (int k = 0; k < D; ++k)
                    b[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a[g][k]), l));
                wave_ball_query<D, kBallPrune>(b, X2, CS, fr, threshold_of(key), key, m0 + g * kThreads + l,
                                               nullptr, evals);
            }
        }
    }
    add_counts(counts, evals, 0u);
}

// The m the cell scan left (flag bits), in iteration order: block = 256 words = 8192 m of one
// pair (blocks ordered by x2 cloud), each lane one word; each flagged m is taken by its whole wave through an exact ball
// query (dropped at the first d < T, or folded with its exact min).
template <int D>
__global__ __launch_bounds__(kThreads) void scan_flagged_kernel(
    const float *__restrict__ x1, const int64_t *__restrict__ perm1, const float4 *__restrict__ xs2r,
    const int32_t *__restrict__ cstart2, const float *__restrict__ boxes, int64_t clouds2, int64_t b1, int64_t b2,
    int64_t p1, int64_t p2, unsigned long long *__restrict__ keys, const uint32_t *__restrict__ flagbits,
    unsigned long long *__restrict__ counts) {
    // units ordered (x2 cloud, x1 cloud of the batch, block of m): an XCD reads few x2 clouds
    const int64_t nbx = cdiv_dev(p1, 32 * kThreads);
    const int64_t unit = xcd_unit(clouds2 * b1 * nbx);
    const int64_t g2 = unit / (b1 * nbx);
    const int64_t rest = unit - g2 * b1 * nbx;
    const int64_t i = rest / nbx, bx = rest - i * nbx;
    const int64_t bb = g2 / b2, j = g2 - bb * b2;
    const int64_t pair = (bb * b1 + i) * b2 + j;
    const float4 *X2 = xs2r + g2 * p2;
    const int32_t *CS = cstart2 + g2 * (kCells + 1);
    float fr[2 * D];
    frame_of<D>(boxes + bb * D * 2, fr);
    unsigned long long *key = &keys[pair];
    const int64_t fwords = cdiv_dev(p1, 32);
    const int64_t wi = bx * kThreads + threadIdx.x;
    const uint32_t word = wi < fwords ? flagbits[pair * fwords + wi] : 0u;
    const int64_t wbase = (bx * kThreads + 64 * __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * 32;
    uint32_t evals = 0;
    unsigned long long left = __ballot(word != 0u);
    while (left) {
        const int l = __builtin_ctzll(left);
        left &= left - 1;
        uint32_t bits = (uint32_t)__builtin_amdgcn_readlane((int)word, l);
        while (bits) {
            const int bit = __builtin_ctz(bits);
            bits &= bits - 1;
            const int64_t mm = wbase + 32 * l + bit;  // < p1: only real m are flagged
            float b[D];
            point_at<D>(x1, perm1, bb * b1 + i, b1, p1, mm, b);
            wave_ball_query<D, kBallPrune>(b, X2, CS, fr, threshold_of(key), key, mm, nullptr, evals);
        }
    }
    add_counts(counts, evals, 0u);
}

// Seeds on the cell grid: one wave per (pair, seed s), waves ordered by x2 cloud.  The pair's
// ncand candidate keys (squared distance to x2's box << 32 | x1 position + 1; 0 = none) are
// distinct, so every wave of the pair takes the kSeeds largest in the same order (each round
// the largest key below the previous one) and keeps the s-th: seedm[pair][s] = its position
// (0xffffffff when there are fewer candidates).  The wave finds that point's exact min with a
// ball query and folds it into the pair's key.
template <int D>
__global__ __launch_bounds__(kThreads) void seed_ball_kernel(
    const float *__restrict__ x1, const int64_t *__restrict__ perm1, const float4 *__restrict__ xs2r,
    const int32_t *__restrict__ cstart2, const float *__restrict__ boxes, bool batch_frame,
    const unsigned long long *__restrict__ cand, int64_t ncand, int64_t b1, int64_t b2, int64_t p1, int64_t p2,
    int64_t pairs, uint32_t *__restrict__ seedm, unsigned long long *__restrict__ keys,
    unsigned long long *__restrict__ counts) {
    // waves ordered (x2 cloud, x1 cloud of the batch, seed): an XCD reads few x2 clouds
    const int64_t v = xcd_unit(cdiv_dev(pairs * kSeeds, kThreads / 64)) * (kThreads / 64) + (threadIdx.x >> 6);
    if (v >= pairs * kSeeds) return;  // the same in every lane
    const int64_t g2 = v / (b1 * kSeeds);
    const int64_t vr = v - g2 * b1 * kSeeds;
    const int64_t bb0 = g2 / b2;
    const int64_t pair = (bb0 * b1 + vr / kSeeds) * b2 + (g2 - bb0 * b2);
    const int s = (int)(vr % kSeeds);
    const int64_t t = pair * kSeeds + s;
    const int lane = threadIdx.x & 63;
    const unsigned long long *C = cand + pair * ncand;
    // up to kHeld candidates per lane stay in registers over the rounds (any more are re-read)
    constexpr int kHeld = 4;
    unsigned long long held[kHeld];
#pragma unroll
    for (int h = 0; h < kHeld; ++h) held[h] = lane + 64 * h < ncand ? C[lane + 64 * h] : 0ull;
    unsigned long long prev = ~0ull, pick = 0;
    for (int r = 0; r <= s; ++r) {  // every lane holds the same reduced values
        unsigned long long best = 0;
#pragma unroll
        for (int h = 0; h < kHeld; ++h)
            if (held[h] < prev && held[h] > best) best = held[h];
        for (int64_t e = lane + 64 * kHeld; e < ncand; e += 64) {
            const unsigned long long v = C[e];
            if (v < prev && v > best) best = v;
        }
        pick = wave_max_u64(best);
        if (!pick) break;
        prev = pick;
    }
    const uint32_t m = pick ? (uint32_t)(pick & 0xffffffffull) - 1u : 0xffffffffu;
    if (lane == 0) seedm[t] = m;
    if (m == 0xffffffffu) return;
    const int64_t per_batch = b1 * b2;
    const int64_t bb = pair / per_batch, rem = pair - bb * per_batch;
    const int64_t i = rem / b2, j = rem - i * b2;
    float fr[2 * D];
    frame_of<D>(boxes + (batch_frame ? bb : bb * b2 + j) * D * 2, fr);
    float q[D];
    point_at<D>(x1, perm1, bb * b1 + i, b1, p1, m, q);
    float mn = INFINITY;
    uint32_t evals = 0;
    wave_ball_query<D, kBallMin>(q, xs2r + (bb * b2 + j) * p2, cstart2 + (bb * b2 + j) * (kCells + 1), fr, 0.0f,
                                 nullptr, 0, &mn, evals);
    if (lane == 0) fold_key(&keys[pair], mn, m);
    add_counts(counts, evals, 0u);
}

// Final rescan on the cell grid: one wave per pair finds the smallest position n of an x2 point
// at the winning m's min with a ball query, then writes sqrt of the min and the (permuted)
// positions of m and n.  A pair whose batch holds a value that is not finite (nonfin[bb]), or
// whose winning min is +inf (squared sums that overflow), takes the reference's loop instead
// (hdx::exact_pair on the inputs as given): its early exits on NaN, and the indices it carries
// over from an earlier row when a row never improves on +inf, are no property of the mins that
// pruning could reproduce.
template <int D>
__global__ __launch_bounds__(kThreads) void first_ball_kernel(
    const float *__restrict__ x1, const float *__restrict__ x2, const int64_t *__restrict__ perm1,
    const int64_t *__restrict__ perm2, const float4 *__restrict__ xs2r, const int32_t *__restrict__ cstart2,
    const float *__restrict__ boxes, bool batch_frame, const unsigned long long *__restrict__ keys,
    const uint32_t *__restrict__ nonfin, int64_t b1, int64_t b2, int64_t p1, int64_t p2, int64_t pairs,
    float *__restrict__ out, int64_t *__restrict__ idx1, int64_t *__restrict__ idx2,
    unsigned long long *__restrict__ counts) {
    const int64_t pair = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (pair >= pairs) return;  // the same in every lane
    const int64_t per_batch = b1 * b2;
    const int64_t bb = pair / per_batch, rem = pair - bb * per_batch;
    const int64_t i = rem / b2, j = rem - i * b2;
    const unsigned long long key = keys[pair];
    if (__builtin_amdgcn_readfirstlane(nonfin[bb]) || __uint_as_float((uint32_t)(key >> 32)) == INFINITY) {
        float best;
        int64_t mb, nb;
        hdx::exact_pair<TPW_F32>(x1 + (bb * b1 + i) * p1 * D, x2 + (bb * b2 + j) * p2 * D, p1, p2, D,
                                 perm1 ? perm1 + bb * p1 : nullptr, perm2 ? perm2 + bb * p2 : nullptr, best, mb, nb);
        if ((threadIdx.x & 63) == 0) {
            out[pair] = sqrt_rn(best);
            idx1[pair] = mb;
            idx2[pair] = nb;
        }
        return;
    }
    const int64_t m = (int64_t)(key & 0xffffffffull);
    const float H = __uint_as_float((uint32_t)(key >> 32));
    float fr[2 * D];
    frame_of<D>(boxes + (batch_frame ? bb : bb * b2 + j) * D * 2, fr);
    float q[D];
    point_at<D>(x1, perm1, bb * b1 + i, b1, p1, m, q);
    uint32_t evals = 0;
    const unsigned long long n = wave_ball_query<D, kBallFirst>(
        q, xs2r + (bb * b2 + j) * p2, cstart2 + (bb * b2 + j) * (kCells + 1), fr, H, nullptr, 0, nullptr, evals);
    if ((threadIdx.x & 63) == 0) {
        out[pair] = sqrt_rn(H);
        idx1[pair] = perm1 ? perm1[bb * p1 + m] : m;
        idx2[pair] = n < (unsigned long long)p2 ? (perm2 ? perm2[bb * p2 + (int64_t)n] : (int64_t)n) : 0;
    }
    add_counts(counts, evals, 0u);
}

// The unsorted modes without the cell grid: after the outputs, one wave per pair whose batch
// holds a value that is not finite (nonfin[bb]), or whose winning min is +inf, overwrites them
// with the reference's loop (as first_ball_kernel does).
__global__ __launch_bounds__(kThreads) void exact_fix_kernel(const float *__restrict__ x1, const float *__restrict__ x2,
                                                             const int64_t *__restrict__ perm1,
                                                             const int64_t *__restrict__ perm2,
                                                             const uint32_t *__restrict__ nonfin, int64_t b1,
                                                             int64_t b2, int64_t p1, int64_t p2, int64_t d,
                                                             int64_t pairs, float *__restrict__ out,
                                                             int64_t *__restrict__ idx1, int64_t *__restrict__ idx2,
                                                             const unsigned long long *__restrict__ keys) {
    const int64_t pair = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (pair >= pairs) return;  // the same in every lane
    const int64_t per_batch = b1 * b2;
    const int64_t bb = pair / per_batch, rem = pair - bb * per_batch;
    const int64_t i = rem / b2, j = rem - i * b2;
    if (!__builtin_amdgcn_readfirstlane(nonfin[bb]) && !(__uint_as_float((uint32_t)(keys[pair] >> 32)) == INFINITY))
        return;
    float best;
    int64_t mb, nb;
    hdx::exact_pair<TPW_F32>(x1 + (bb * b1 + i) * p1 * d, x2 + (bb * b2 + j) * p2 * d, p1, p2, d,
                             perm1 ? perm1 + bb * p1 : nullptr, perm2 ? perm2 + bb * p2 : nullptr, best, mb, nb);
    if ((threadIdx.x & 63) == 0) {
        out[pair] = sqrt_rn(best);
        idx1[pair] = mb;
        idx2[pair] = nb;
    }
}

// ---------------------------------------------------------------------------------------
// The sorted mode (d <= 3 and the flag bits fit): x1 and x2 both cell-sorted in each batch's
// frame, read from the inputs as given (no SoA copy):
//   prep: presets, and every cloud's per-chunk min / max of each coordinate;
//   frames: each x2 cloud's box (for the seeds) and each batch's box over both sides;
//   cell sort of both sides (cell_count / cell_offsets / cell_scatter, or cell_sort);
//   cells: the exact box of every x1 cell's points, the seed candidates, and one
//     representative point of every x2 cell;
//   seed_ball: the seeds' exact mins, the first T;
//   cell_scan: whole cells of x1 dropped by one box test, the m of the cells left by their
//     windows; flags;
//   scan_flagged: ball queries for the flagged m;
//   first_ball: the first x2 position at the winner's min, and the outputs.

// Block (g, y): rows [y chunk, (y + 1) chunk) of cloud g (x1's clouds, then x2's; rows in input
// order, which a box does not depend on): part[g][y][k][0..1] = their min and max of coordinate
// k (NaN ignored, as fminf / fmaxf ignore it; +inf / -inf when there is none), and bad[g][y] = 1
// when one of their values is not finite (v - v != 0), else 0.  The grid also writes the
// presets fs.
template <int D>
__global__ __launch_bounds__(kThreads) void prep_kernel(const float *__restrict__ x1, int64_t clouds1, int64_t p1,
                                                        const float *__restrict__ x2, int64_t p2, int64_t chunk,
                                                        int64_t chunks, float *__restrict__ part,
                                                        uint32_t *__restrict__ bad, Fills fs) {
    __shared__ float red[kThreads / 64][2 * D];
    __shared__ uint32_t red_bad[kThreads / 64];
    const int64_t nthr = (int64_t)gridDim.x * gridDim.y * kThreads;
    const int64_t tid = ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * kThreads + threadIdx.x;
    // constant indices only (a dynamically indexed copy of the argument would live in LDS)
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        if (r >= fs.count) break;
        uint32_t *p = fs.f[r].p;
        const int64_t n = fs.f[r].n;
        const uint32_t v0 = fs.f[r].v[0], v1 = fs.f[r].v[1];
        for (int64_t t = tid; t < n; t += nthr) p[t] = (t & 1) ? v1 : v0;
    }
    const int64_t g = blockIdx.x;
    const bool in1 = g < clouds1;
    const int64_t p = in1 ? p1 : p2;
    const float *X = in1 ? x1 + g * p1 * D : x2 + (g - clouds1) * p2 * D;
    const int64_t beg = (int64_t)blockIdx.y * chunk;
    const int64_t end = beg + chunk < p ? beg + chunk : p;
    float lo[D], hi[D];
#pragma unroll
    for (int k = 0; k < D; ++k) {
        lo[k] = INFINITY;
        hi[k] = -INFINITY;
    }
    bool nf = false;  // a value that is not finite
    int64_t n = beg + threadIdx.x;
    for (; n + 3 * kThreads < end; n += 4 * kThreads) {  // four rows in flight
        float v[4][D];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int k = 0; k < D; ++k) v[u][k] = X[(n + u * kThreads) * D + k];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int k = 0; k < D; ++k) {
                lo[k] = fminf(lo[k], v[u][k]);
                hi[k] = fmaxf(hi[k], v[u][k]);
                nf = nf || !(v[u][k] - v[u][k] == 0.0f);
            }
    }
    for (; n < end; n += kThreads)
#pragma unroll
        for (int k = 0; k < D; ++k) {
            const float v = X[n * D + k];
            lo[k] = fminf(lo[k], v);
            hi[k] = fmaxf(hi[k], v);
            nf = nf || !(v - v == 0.0f);
        }
    const bool wave_nf = __ballot(nf) != 0ull;
#pragma unroll
    for (int k = 0; k < D; ++k)
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            lo[k] = fminf(lo[k], __shfl_xor(lo[k], off, 64));
            hi[k] = fmaxf(hi[k], __shfl_xor(hi[k], off, 64));
        }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            red[wave][2 * k] = lo[k];
            red[wave][2 * k + 1] = hi[k];
        }
        red_bad[wave] = wave_nf ? 1u : 0u;
    }
    __syncthreads();
    if (threadIdx.x < 2 * D) {
        const int e = threadIdx.x;
        float v = red[0][e];
        for (int w = 1; w < kThreads / 64; ++w) v = (e & 1) ? fmaxf(v, red[w][e]) : fminf(v, red[w][e]);
        part[(g * chunks + blockIdx.y) * 2 * D + e] = v;
    }
    if (threadIdx.x == 0) {
        uint32_t b = 0;
        for (int w = 0; w < kThreads / 64; ++w) b |= red_bad[w];
        bad[g * chunks + blockIdx.y] = b;
    }
}

// Block g < clouds2: x2 cloud g's box bbox2[g][k][0..1] (the seeds' distance) from its chunk
// partials; block clouds2 + bb: batch bb's box over the partials of its b1 x1 clouds and b2 x2
// clouds, the cell frame boxb[bb][k][0..1], and nonfin[bb] = whether any of its chunks holds a
// value that is not finite.
template <int D>
__global__ __launch_bounds__(kThreads) void frames_kernel(const float *__restrict__ part,
                                                          const uint32_t *__restrict__ bad, int64_t clouds1,
                                                          int64_t clouds2, int64_t b1, int64_t b2, int64_t chunks,
                                                          float *__restrict__ bbox2, float *__restrict__ boxb,
                                                          uint32_t *__restrict__ nonfin) {
    __shared__ float red[kThreads / 64][2 * D];
    __shared__ uint32_t red_bad[kThreads / 64];
    const int64_t g = blockIdx.x;
    // partial rows (row = cloud * chunks + y) [r0, r1) and [r2, r3)
    int64_t r0, r1, r2 = 0, r3 = 0;
    float *dst;
    if (g < clouds2) {
        r0 = (clouds1 + g) * chunks;
        r1 = r0 + chunks;
        dst = bbox2 + g * 2 * D;
    } else {
        const int64_t bb = g - clouds2;
        r0 = bb * b1 * chunks;
        r1 = r0 + b1 * chunks;
        r2 = (clouds1 + bb * b2) * chunks;
        r3 = r2 + b2 * chunks;
        dst = boxb + bb * 2 * D;
    }
    float lo[D], hi[D];
#pragma unroll
    for (int k = 0; k < D; ++k) {
        lo[k] = INFINITY;
        hi[k] = -INFINITY;
    }
    uint32_t nf = 0;
    for (int half = 0; half < 2; ++half) {
        const int64_t a = half ? r2 : r0, b = half ? r3 : r1;
        for (int64_t r = a + threadIdx.x; r < b; r += kThreads) {
#pragma unroll
            for (int k = 0; k < D; ++k) {
                lo[k] = fminf(lo[k], part[r * 2 * D + 2 * k]);
                hi[k] = fmaxf(hi[k], part[r * 2 * D + 2 * k + 1]);
            }
            nf |= bad[r];
        }
    }
    const bool wave_nf = __ballot(nf != 0u) != 0ull;
#pragma unroll
    for (int k = 0; k < D; ++k)
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            lo[k] = fminf(lo[k], __shfl_xor(lo[k], off, 64));
            hi[k] = fmaxf(hi[k], __shfl_xor(hi[k], off, 64));
        }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            red[wave][2 * k] = lo[k];
            red[wave][2 * k + 1] = hi[k];
        }
        red_bad[wave] = wave_nf ? 1u : 0u;
    }
    __syncthreads();
    if (threadIdx.x < 2 * D) {
        const int e = threadIdx.x;
        float v = red[0][e];
        for (int w = 1; w < kThreads / 64; ++w) v = (e & 1) ? fmaxf(v, red[w][e]) : fminf(v, red[w][e]);
        dst[e] = v;
    }
    if (threadIdx.x == 0 && g >= clouds2) {
        uint32_t b = 0;
        for (int w = 0; w < kThreads / 64; ++w) b |= red_bad[w];
        nonfin[g - clouds2] = b;
    }
}

// Per-cell pass over both sides' sorted records, one lane per cell, blocks of 256 cells:
//   x1 clouds, for the x2 clouds j of one group (kCellsJ per group; units ordered by cloud,
//   group, cells): the seed candidates, the kCandPerWave largest keys (squared distance to x2
//   j's box << 32 | position + 1) over the wave's 64 cells, cand[pair][kCandPerWave (c / 64) +
//   r] (0: none).  Group 0 also writes the cell's record range and the exact box of its points,
//   info1[cloud][pos(c)] = {start, end (int bits), lo[0..2], hi[0..2]} (two float4; a cell
//   holding a NaN coordinate gets lo -inf and hi +inf, which no box test passes);
//   x2 clouds (units spread among those): rep2[cloud][pos(c)] = the record of the cell that is
//   nearest to covering the cell's region (least squared distance to the region's farthest
//   corner; any x2 point serves the box test, this one drops the most cells), or, for an empty
//   cell, the point at its start.
// Records are loaded kU at a time (indices past the end repeat the last record, which changes
// no min, max or largest key).
constexpr int kCandPerWave = 4;
constexpr int64_t kCellCand = kCells / 64 * kCandPerWave;
constexpr int kCellsJ = 2;  // x2 clouds per x1 group

template <int D>
__device__ __forceinline__ void x2_rep_cell(const float4 *__restrict__ X, const int32_t *__restrict__ CS,
                                            const float *__restrict__ frame, int c, int64_t p2,
                                            float4 *__restrict__ rep) {
    constexpr int kU = 8;
    const int32_t s = CS[c], e = CS[c + 1];
    float fr[2 * D];
    frame_of<D>(frame, fr);
    float lo[D], hi[D];
#pragma unroll
    for (int k = 0; k < D; ++k) {
        const uint32_t u = D == 1 ? (uint32_t)c : compact_bits<D>((uint32_t)c >> k);
        const float step = fr[2 * k + 1] > 0.0f ? 1.0f / fr[2 * k + 1] : 0.0f;
        lo[k] = fr[2 * k] + (float)u * step;
        hi[k] = lo[k] + step;
    }
    float4 best = X[s < p2 ? s : p2 - 1];
    float bestv = INFINITY;
    for (int32_t n0 = s; n0 < e; n0 += kU) {
        float4 v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) v[u] = X[n0 + u < e ? n0 + u : e - 1];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            float mc = 0.0f;
#pragma unroll
            for (int k = 0; k < D; ++k) {
                const float a = rec_coord(v[u], k);
                const float ek = fmaxf(hi[k] - a, a - lo[k]);
                mc = mc + ek * ek;
            }
            if (mc < bestv) {
                bestv = mc;
                best = v[u];
            }
        }
    }
    *rep = best;
}

template <int D>
__global__ __launch_bounds__(kThreads) void cells_kernel(const float4 *__restrict__ xs1r,
                                                         const float4 *__restrict__ xs2r,
                                                         const int32_t *__restrict__ cstart,
                                                         const float *__restrict__ bbox2,
                                                         const float *__restrict__ boxb, int64_t clouds1,
                                                         int64_t clouds2, int64_t b1, int64_t b2, int64_t p1,
                                                         int64_t p2, float4 *__restrict__ info1,
                                                         float4 *__restrict__ rep2,
                                                         unsigned long long *__restrict__ cand) {
    constexpr int kJ = kCellsJ, kU = 8;
    constexpr int64_t kBlocksPerCloud = kCells / kThreads;
    const int64_t groups = cdiv_dev(b2, kJ);
    const int64_t units1 = clouds1 * groups * kBlocksPerCloud, units2 = clouds2 * kBlocksPerCloud;
    const int64_t total = units1 + units2;
    // the x2 units spread evenly among the x1 units (n2(p) of them before place p), so that
    // every XCD's range holds its share of both
    const int64_t place = xcd_unit(total);
    const int64_t n2 = place * units2 / total;
    if ((place + 1) * units2 / total > n2) {  // the same in every lane
        const int64_t g2 = n2 / kBlocksPerCloud;
        const int c = (int)(n2 - g2 * kBlocksPerCloud) * kThreads + threadIdx.x;
        x2_rep_cell<D>(xs2r + g2 * p2, cstart + g2 * (kCells + 1), boxb + (g2 / b2) * 2 * D, c, p2,
                       rep2 + g2 * kCells + pos_cell(c));
        return;
    }
    const int64_t unit = place - n2;
    const int64_t g1 = unit / (groups * kBlocksPerCloud);
    const int64_t rest = unit - g1 * groups * kBlocksPerCloud;
    const int64_t z = rest / kBlocksPerCloud;
    const int64_t bb = g1 / b1;
    const int64_t j0 = z * kJ;
    const bool first = z == 0;
    const int c = (int)(rest - z * kBlocksPerCloud) * kThreads + threadIdx.x;
    const int lane = threadIdx.x & 63;
    const int32_t *CS = cstart + (clouds2 + g1) * (kCells + 1);
    const int32_t s = CS[c], e = CS[c + 1];
    const float4 *X = xs1r + g1 * p1;
    float box[kJ][2 * D];
#pragma unroll
    for (int jj = 0; jj < kJ; ++jj)
#pragma unroll
        for (int k = 0; k < 2 * D; ++k) box[jj][k] = j0 + jj < b2 ? bbox2[(bb * b2 + j0 + jj) * 2 * D + k] : 0.0f;
    float lo[D], hi[D];
#pragma unroll
    for (int k = 0; k < D; ++k) {
        lo[k] = INFINITY;
        hi[k] = -INFINITY;
    }
    bool nan = false;
    unsigned long long best[kJ];
#pragma unroll
    for (int jj = 0; jj < kJ; ++jj) best[jj] = 0;
    for (int32_t n0 = s; n0 < e; n0 += kU) {
        float4 v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) v[u] = X[n0 + u < e ? n0 + u : e - 1];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            float a[D];
#pragma unroll
            for (int k = 0; k < D; ++k) a[k] = rec_coord(v[u], k);
            if (first) {
#pragma unroll
                for (int k = 0; k < D; ++k) {
                    nan = nan || a[k] != a[k];
                    lo[k] = fminf(lo[k], a[k]);
                    hi[k] = fmaxf(hi[k], a[k]);
                }
            }
            const uint64_t pos1 = (uint64_t)rec_pos(v[u]) + 1;
#pragma unroll
            for (int jj = 0; jj < kJ; ++jj) {
                float L = 0.0f;
#pragma unroll
                for (int k = 0; k < D; ++k) {
                    const float ex = fmaxf(fmaxf(box[jj][2 * k] - a[k], a[k] - box[jj][2 * k + 1]), 0.0f);
                    L = L + ex * ex;
                }
                const unsigned long long key = ((unsigned long long)__float_as_uint(L) << 32) | pos1;
                best[jj] = key > best[jj] ? key : best[jj];
            }
        }
    }
#pragma unroll
    for (int jj = 0; jj < kJ; ++jj) {
        if (j0 + jj >= b2) break;  // the same in every lane
        unsigned long long *C = cand + (g1 * b2 + j0 + jj) * kCellCand + (c / 64) * kCandPerWave;
        unsigned long long mine = best[jj];
        for (int r = 0; r < kCandPerWave; ++r) {
            const unsigned long long mx = wave_max_u64(mine);
            if (lane == 0) C[r] = mx;
            if (mine == mx) mine = 0;  // keys of distinct points differ
        }
    }
    if (first) {
        float f[8] = {__int_as_float(s), __int_as_float(e), 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < D; ++k) {
            f[2 + k] = nan ? -INFINITY : lo[k];
            f[5 + k] = nan ? INFINITY : hi[k];
        }
        float4 *I = info1 + (g1 * kCells + pos_cell(c)) * 2;
        I[0] = make_float4(f[0], f[1], f[2], f[3]);
        I[1] = make_float4(f[4], f[5], f[6], f[7]);
    }
}

__device__ __forceinline__ unsigned long long wave_or_u64(unsigned long long v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v |= shfl_xor_u64(v, off);
    return v;
}

// One cell by the whole wave: lane = window point W (the cell's 64-point window of sorted x2,
// from x2's start of the cell clamped to a full window; lanes past wlen repeat its last
// point), R = the cell's records in lanes 0 .. cnt - 1 (cnt <= 64).  Each lane tests every m_i
// (broadcast, four at a time) against its point and keeps bit i when d(m_i, point) < T; the OR
// over the wave marks the m some window point drops, the test a lane-per-m scan of the window
// makes.  An m left, not a seed, sets bit (its iteration position) of the pair's flag bits
// (preset to 0) for scan_flagged_kernel.
template <int D>
__device__ __forceinline__ void window_check(const float4 &W, const float4 &R, int cnt, float T, int64_t wlen,
                                             int64_t pair, const uint32_t *seedm, uint32_t *flagbits, int64_t fwords,
                                             uint32_t &evals) {
    const int lane = threadIdx.x & 63;
    float w[D];
#pragma unroll
    for (int k = 0; k < D; ++k) w[k] = rec_coord(W, k);
    unsigned long long mine = 0;
    for (int i0 = 0; i0 < cnt; i0 += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = i0 + u < cnt ? i0 + u : cnt - 1;  // a repeated m sets a bit it already sets
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < D; ++k) {
                const float mk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rec_coord(R, k)), i));
                const float diff = mk - w[k];
                s = s + diff * diff;
            }
            mine |= (unsigned long long)(s < T) << i;
        }
    }
    const unsigned long long hits = wave_or_u64(mine);
    if (lane == 0) evals += (uint32_t)(cnt * wlen);
    if (lane < cnt && !((hits >> lane) & 1ull)) {
        const uint32_t mpos = rec_pos(R);
        if (!is_seed(seedm, pair, mpos)) atomicOr(&flagbits[pair * fwords + (mpos >> 5)], 1u << (mpos & 31));
    }
}

// Scan of the sorted mode: block = kScanCells cells of one pair (positions pos(c); kScanCols
// per lane), 16 waves; blocks ordered (x2 cloud, x1 cloud of the batch, block) so that an XCD
// reads few x2 clouds.  The x1 points of cell c are the records start .. end (x1 is sorted in
// the batch frame x2 shares), inside the exact box of info1.  First each lane tests that box
// against x2's representative point q of cell c (rep2, an x2 point): when the box's farthest
// corner from q, computed as d is (coordinate differences, squared and summed in order in
// fp32), is below T, every m of the cell has d(m, q) < T and the whole cell is dropped.  That
// holds bit for bit: rounding is monotone, so each |fl(a_k - q_k)| is at most the corner's
// rounded difference, and the squares and the in-order sums keep that order.  Special values
// (inf, NaN; a NaN cell's box) make the corner's value inf or NaN, which drops nothing.  The
// cells left go to a list in LDS (their record range and window start), and the block's waves
// then take them in turn, two at a time so that their loads overlap (window_check).
constexpr int kScanThreads = 1024;
#ifndef TPW_SCAN_COLS
#define TPW_SCAN_COLS 1
#endif
constexpr int kScanCols = TPW_SCAN_COLS;
constexpr int kScanCells = kScanThreads * kScanCols;
constexpr int kScanBlocksPerPair = kCells / kScanCells;

template <int D>
__global__ __launch_bounds__(kScanThreads) void cell_scan_kernel(
    const float4 *__restrict__ xs1r, const float4 *__restrict__ xs2r, const int32_t *__restrict__ cstT,
    const float4 *__restrict__ info1, const float4 *__restrict__ rep2, int64_t clouds2, int64_t b1, int64_t b2,
    int64_t p1, int64_t p2, const uint32_t *__restrict__ seedm, unsigned long long *__restrict__ keys,
    uint32_t *__restrict__ flagbits, unsigned long long *__restrict__ counts) {
    __shared__ int32_t lst[kScanCells][3];  // start, count, window start of each cell left
    __shared__ uint32_t nlst;
    // the index math is 32-bit (pairs <= 65535)
    const uint32_t ub1 = (uint32_t)b1, ub2 = (uint32_t)b2;
    const uint32_t unit = (uint32_t)xcd_unit(clouds2 * b1 * kScanBlocksPerPair);
    const uint32_t g2 = unit / (ub1 * kScanBlocksPerPair);
    const uint32_t rest = unit - g2 * ub1 * kScanBlocksPerPair;
    const uint32_t i = rest / kScanBlocksPerPair, blk = rest - i * kScanBlocksPerPair;
    const uint32_t bb = g2 / ub2, j = g2 - bb * ub2;
    const uint32_t g1 = bb * ub1 + i;
    const int64_t pair = (int64_t)g1 * ub2 + j;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (threadIdx.x == 0) nlst = 0;
    __syncthreads();
    unsigned long long *key = &keys[pair];
    float T = threshold_of(key);
    const int64_t wlen = p2 < 64 ? p2 : 64;
    uint32_t evals = 0, tests = 0;
#pragma unroll
    for (int h = 0; h < kScanCols; ++h) {
        const int t = (int)blk * kScanCells + h * kScanThreads + threadIdx.x;  // position of a cell
        const float4 A = info1[((int64_t)g1 * kCells + t) * 2], Bq = info1[((int64_t)g1 * kCells + t) * 2 + 1];
        const float4 q = rep2[(int64_t)g2 * kCells + t];
        const int32_t s2 = cstT[(int64_t)g2 * kCells + t];
        const float f[6] = {A.z, A.w, Bq.x, Bq.y, Bq.z, Bq.w};
        const int32_t s1 = __float_as_int(A.x), e1 = __float_as_int(A.y);
        bool todo = e1 > s1;
        if (todo) {
            float mc = 0.0f;
#pragma unroll
            for (int k = 0; k < D; ++k) {
                const float qk = rec_coord(q, k);
                const float ek = fmaxf(f[3 + k] - qk, qk - f[k]);
                mc = mc + ek * ek;
            }
            todo = !(mc < T);
            ++tests;
        }
        const unsigned long long left = __ballot(todo);
        if (left) {  // the same in every lane
            uint32_t base = 0;
            if (lane == 0) base = atomicAdd(&nlst, (uint32_t)__popcll(left));  // LDS
            base = __builtin_amdgcn_readfirstlane(base);
            if (todo) {
                const uint32_t e = base + __popcll(left & ((1ull << lane) - 1ull));
                lst[e][0] = s1;
                lst[e][1] = e1 - s1;
                lst[e][2] = s2 < p2 - wlen ? s2 : (int32_t)(p2 - wlen);
            }
        }
    }
    __syncthreads();
    const uint32_t n = nlst;
    if (n) T = threshold_of(key);
    const int wl = lane < wlen ? lane : (int)wlen - 1;
    const int64_t fwords = cdiv_dev(p1, 32);
    const float4 *X1 = xs1r + (int64_t)g1 * p1;
    const float4 *X2 = xs2r + (int64_t)g2 * p2;
    constexpr uint32_t kWaves = kScanThreads / 64;
    for (uint32_t e0 = wave; e0 < n; e0 += 2 * kWaves) {
        const bool two = e0 + kWaves < n;
        int32_t cs[2], cn[2];
        float4 W[2], R[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t e = u && two ? e0 + kWaves : e0;
            cs[u] = __builtin_amdgcn_readfirstlane(lst[e][0]);
            cn[u] = __builtin_amdgcn_readfirstlane(lst[e][1]);
            const int32_t cw = __builtin_amdgcn_readfirstlane(lst[e][2]);
            W[u] = X2[cw + wl];
            R[u] = X1[cs[u] + (lane < cn[u] ? lane : cn[u] - 1)];
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (u == 1 && !two) break;  // the same in every lane
            window_check<D>(W[u], R[u], cn[u] < 64 ? cn[u] : 64, T, wlen, pair, seedm, flagbits, fwords, evals);
            for (int32_t off = 64; off < cn[u]; off += 64) {
                const int32_t rem = cn[u] - off;
                const float4 r = X1[cs[u] + off + (lane < rem ? lane : rem - 1)];
                window_check<D>(W[u], r, rem < 64 ? rem : 64, T, wlen, pair, seedm, flagbits, fwords, evals);
            }
        }
    }
    add_counts(counts, evals, tests);
}

// The sorted mode keeps one flag bit per (pair, m): up to 32 MiB of them.
inline bool sorted_mode(int64_t pairs, int64_t p1) { return pairs * p1 <= ((int64_t)1 << 28); }

int64_t round_up(int64_t v, int64_t q) { return cdiv(v, q) * q; }

// How a run is split; a function of the sizes only (the workspace size depends on it).
struct Plan {
    int64_t batch = 0, pairs = 0, clouds1 = 0, clouds2 = 0;
    bool active = false;      // points and features on both sides
    bool fast = false;        // d = 1..4: seeds and final rescan spread over blocks
    bool cells = false;       // d <= 3 and int32 cell starts: the cell-sorted scan
    bool sorted = false;      // cells and the flags fit: x1 sorted too, in a shared frame
    bool multi_sort = false;  // few clouds to sort: the counting sort spread over blocks
    int64_t box_rows1 = 0, box_rows2 = 0, box_chunk = 1, box_chunks = 0;  // unsorted boxes
    int64_t prep_chunk = 1, prep_chunks = 0;  // sorted boxes: rows per prep block
    int64_t chunk1 = 1, ncand = 0;   // x1 points per seed_select block; candidates per pair
    int64_t chunk2 = 1, nch2 = 0;    // x2 points per first_hit block
    int64_t chunkL = 1, nchL = 0;    // x2 points per list_scan block of the seeds
    int64_t sort_clouds = 0, sort_chunk = 1, sort_chunks = 0;
};

Plan make_plan(int64_t batch, int64_t b1, int64_t p1, int64_t b2, int64_t p2, int64_t d) {
    Plan P;
    P.batch = batch;
    P.pairs = batch * b1 * b2;
    P.clouds1 = batch * b1;
    P.clouds2 = batch * b2;
    P.active = P.pairs > 0 && p1 > 0 && p2 > 0 && d > 0;
    if (!P.active) return P;
    P.fast = d <= 4;
    P.cells = d <= 3 && p2 < (int64_t)0x7fffffff - 64;
    P.sorted = P.cells && sorted_mode(P.pairs, p1);
    const int64_t pmax = std::max(p1, p2);
    if (P.sorted) {
        P.prep_chunk = std::max<int64_t>(2048, round_up(cdiv(pmax, kMaxGridYZ), kThreads));
        P.prep_chunks = cdiv(pmax, P.prep_chunk);
        P.ncand = kCellCand;
    } else {
        P.box_rows2 = P.clouds2 * d;
        P.box_chunk = std::max<int64_t>(8192, round_up(cdiv(p2, kMaxGridYZ), kThreads));
        P.box_chunks = cdiv(p2, P.box_chunk);
        // at most 64 seed_select blocks (256 candidates) per pair, at least 4096 points each
        P.chunk1 = std::max<int64_t>(4096, round_up(cdiv(p1, 64), kThreads));
        P.ncand = cdiv(p1, P.chunk1) * (kThreads / 64);
    }
    P.chunk2 = std::max<int64_t>(4096, round_up(cdiv(p2, kMaxGridYZ), kThreads));
    P.nch2 = cdiv(p2, P.chunk2);
    P.chunkL = std::max<int64_t>(16384, round_up(cdiv(p2, kMaxGridYZ), kThreads));
    P.nchL = cdiv(p2, P.chunkL);
    if (P.cells) {
        P.sort_clouds = P.clouds2 + (P.sorted ? P.clouds1 : 0);
        P.multi_sort = P.sort_clouds <= 2048;
        // chunks of >= 4096 points, at most 4096 (cloud, chunk) histograms (64 MiB)
        const int64_t psort = P.sorted ? pmax : p2;
        const int64_t most = std::max<int64_t>(1, 4096 / std::max<int64_t>(1, P.sort_clouds));
        P.sort_chunks = std::min<int64_t>(cdiv(psort, 4096), most);
        P.sort_chunk = round_up(cdiv(psort, P.sort_chunks), kThreads);
        P.sort_chunks = cdiv(psort, P.sort_chunk);
    }
    return P;
}

struct Workspace {
    float *xs1, *xs2, *bbox, *boxb, *part;
    float4 *xs2r, *xs1r, *info1, *rep2;
    unsigned long long *keys, *cand, *first;
    int32_t *cstart2, *cstT;
    int *boxkeys;
    uint32_t *seedmin, *seedm, *cellhist;
    uint32_t *flagbits, *nonfin, *chunkbad;
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// [keys | non-finite flags per batch, per prep chunk (sorted) | x2 boxes | x1, x2 SoA (unsorted) | box keys (unsorted) | box partials, batch boxes
//  (sorted) | seeds, candidates, first hits (fast) | x2 records, cell starts (cells; x2's,
//  then x1's when sorted) | x1 records, x1 cell ranges and boxes, x2 representatives and cell
//  starts in the cell scan's order, flag bits (sorted) | per-chunk cell histograms
//  (multi_sort)]
Workspace carve(void *ws, const Plan &P, int64_t p1, int64_t p2, int64_t d, size_t *total = nullptr) {
    char *base = static_cast<char *>(ws), *p = base;
    auto take = [&](bool on, size_t bytes) {
        char *r = p;
        if (on) p += align256(bytes);
        return on ? r : nullptr;
    };
    const bool uns = !P.sorted;
    Workspace w;
    w.keys = reinterpret_cast<unsigned long long *>(take(true, 8 * P.pairs));
    w.nonfin = reinterpret_cast<uint32_t *>(take(P.active, 4 * P.batch));
    w.chunkbad = reinterpret_cast<uint32_t *>(take(P.sorted, 4 * (P.clouds1 + P.clouds2) * P.prep_chunks));
    w.bbox = reinterpret_cast<float *>(take(true, 4 * P.clouds2 * d * 2));
    w.xs1 = reinterpret_cast<float *>(take(uns, 4 * P.clouds1 * p1 * d));
    w.xs2 = reinterpret_cast<float *>(take(uns, 4 * P.clouds2 * p2 * d));
    w.boxkeys = reinterpret_cast<int *>(take(uns && P.active, 4 * P.box_rows2 * 2));
    w.part = reinterpret_cast<float *>(take(P.sorted, 4 * (P.clouds1 + P.clouds2) * P.prep_chunks * d * 2));
    w.boxb = reinterpret_cast<float *>(take(P.sorted, 4 * P.batch * d * 2));
    w.seedmin = reinterpret_cast<uint32_t *>(take(P.fast, 4 * P.pairs * kSeeds));
    w.seedm = reinterpret_cast<uint32_t *>(take(P.fast, 4 * P.pairs * kSeeds));
    w.cand = reinterpret_cast<unsigned long long *>(take(P.fast, 8 * P.pairs * P.ncand));
    w.first = reinterpret_cast<unsigned long long *>(take(P.fast, 8 * P.pairs));
    w.xs2r = reinterpret_cast<float4 *>(take(P.cells, 16 * P.clouds2 * p2));
    w.cstart2 = reinterpret_cast<int32_t *>(take(P.cells, 4 * P.sort_clouds * (kCells + 1)));
    w.xs1r = reinterpret_cast<float4 *>(take(P.sorted, 16 * P.clouds1 * p1));
    w.info1 = reinterpret_cast<float4 *>(take(P.sorted, 32 * P.clouds1 * kCells));
    w.rep2 = reinterpret_cast<float4 *>(take(P.sorted, 16 * P.clouds2 * kCells));
    w.cstT = reinterpret_cast<int32_t *>(take(P.sorted, 4 * P.clouds2 * kCells));
    w.flagbits = reinterpret_cast<uint32_t *>(take(P.sorted, 4 * P.pairs * cdiv(p1, 32)));
    w.cellhist = reinterpret_cast<uint32_t *>(take(P.multi_sort, 4 * P.sort_clouds * P.sort_chunks * kCells));
    if (total) *total = (size_t)(p - base);
    return w;
}

// Host side of the measurement counters: armed on one device, whose device address of
// g_hd_counts the kernels get (null otherwise); launches of the forward are counted on the host.
struct Counters {
    std::mutex mu;
    bool armed = false;
    int device = -1;
    unsigned long long *ptr = nullptr;
    unsigned long long launches = 0;
};
Counters g_counters;

unsigned long long *counts_arg() {
    if (!__atomic_load_n(&g_counters.armed, __ATOMIC_RELAXED)) return nullptr;
    std::lock_guard<std::mutex> lk(g_counters.mu);
    int dev = -1;
    if (!g_counters.armed || hipGetDevice(&dev) != hipSuccess || dev != g_counters.device) return nullptr;
    return g_counters.ptr;
}

void note_launch() {
    if (!__atomic_load_n(&g_counters.armed, __ATOMIC_RELAXED)) return;
    std::lock_guard<std::mutex> lk(g_counters.mu);
    int dev = -1;
    if (g_counters.armed && hipGetDevice(&dev) == hipSuccess && dev == g_counters.device) ++g_counters.launches;
}

#define HD_LAUNCH(...)                    \
    do {                                  \
        hipLaunchKernelGGL(__VA_ARGS__);  \
        note_launch();                    \
    } while (0)

// Counting sort into records: x2's clouds (sets S2), then, when S1 has clouds, x1's; cell starts
// of every sorted cloud in that order.
template <int D>
void launch_sort(const Plan &P, const Workspace &w, const CellSet &S2, const CellSet &S1, hipStream_t s) {
    if (P.multi_sort) {
        const dim3 grid((unsigned)P.sort_clouds, (unsigned)P.sort_chunks);
        HD_LAUNCH(cell_count_kernel<D>, grid, dim3(kThreads), 0, s, S2, S1, P.sort_chunk, P.sort_chunks, w.cellhist);
        HD_LAUNCH(cell_offsets_kernel, dim3((unsigned)P.sort_clouds), dim3(kOffThreads), 0, s, S2, S1,
                  P.sort_chunks, w.cellhist, w.cstart2, w.cstT);
        HD_LAUNCH(cell_scatter_kernel<D>, grid, dim3(kThreads), 0, s, S2, S1, P.sort_chunk, P.sort_chunks,
                  static_cast<const uint32_t *>(w.cellhist));
    } else {
        HD_LAUNCH(cell_sort_kernel<D>, dim3((unsigned)S2.clouds), dim3(kThreads), 0, s, S2, w.cstart2, w.cstT);
        if (S1.clouds > 0)
            HD_LAUNCH(cell_sort_kernel<D>, dim3((unsigned)S1.clouds), dim3(kThreads), 0, s, S1,
                      w.cstart2 + S2.clouds * (kCells + 1), static_cast<int32_t *>(nullptr));
    }
}

// The sorted mode, every launch (d <= 3).
template <int D>
int launch_sorted(const Plan &P, const Workspace &w, const float *x1, const float *x2, int64_t b1, int64_t p1,
                  int64_t b2, int64_t p2, const int64_t *perm1, const int64_t *perm2, float *out, int64_t *idx1,
                  int64_t *idx2, hipStream_t s) {
    unsigned long long *counts = counts_arg();
    Fills fs{};
    fs.f[fs.count++] = Fill{reinterpret_cast<uint32_t *>(w.keys), 2 * P.pairs, {0u, 0u}};
    fs.f[fs.count++] = Fill{w.flagbits, P.pairs * cdiv(p1, 32), {0u, 0u}};
    HD_LAUNCH(prep_kernel<D>, dim3((unsigned)(P.clouds1 + P.clouds2), (unsigned)P.prep_chunks), dim3(kThreads), 0,
              s, x1, P.clouds1, p1, x2, p2, P.prep_chunk, P.prep_chunks, w.part, w.chunkbad, fs);
    HD_LAUNCH(frames_kernel<D>, dim3((unsigned)(P.clouds2 + P.batch)), dim3(kThreads), 0, s, w.part, w.chunkbad,
              P.clouds1, P.clouds2, b1, b2, P.prep_chunks, w.bbox, w.boxb, w.nonfin);
    int rc = check_launch("hausdorff frames");
    if (rc) return rc;
    const CellSet S2{x2, perm2, w.xs2r, w.boxb, P.clouds2, p2, b2, b2};
    const CellSet S1{x1, perm1, w.xs1r, w.boxb, P.clouds1, p1, b1, b1};
    launch_sort<D>(P, w, S2, S1, s);
    HD_LAUNCH(cells_kernel<D>,
              dim3((unsigned)((P.clouds1 * cdiv(b2, kCellsJ) + P.clouds2) * (kCells / kThreads))), dim3(kThreads),
              0, s, w.xs1r, w.xs2r, w.cstart2, w.bbox, w.boxb, P.clouds1, P.clouds2, b1, b2, p1, p2, w.info1, w.rep2,
              w.cand);
    HD_LAUNCH(seed_ball_kernel<D>, dim3((unsigned)cdiv(P.pairs * kSeeds, kThreads / 64)), dim3(kThreads), 0, s, x1,
              perm1, w.xs2r, w.cstart2, w.boxb, true, w.cand, P.ncand, b1, b2, p1, p2, P.pairs, w.seedm, w.keys,
              counts);
    rc = check_launch("hausdorff seeds");
    if (rc) return rc;
    HD_LAUNCH(cell_scan_kernel<D>, dim3((unsigned)(P.pairs * kScanBlocksPerPair)), dim3(kScanThreads), 0, s, w.xs1r,
              w.xs2r, w.cstT, w.info1, w.rep2, P.clouds2, b1, b2, p1, p2, w.seedm, w.keys, w.flagbits, counts);
    HD_LAUNCH(scan_flagged_kernel<D>, dim3((unsigned)(cdiv(p1, 32 * kThreads) * P.pairs)), dim3(kThreads), 0, s, x1,
              perm1, w.xs2r, w.cstart2, w.boxb, P.clouds2, b1, b2, p1, p2, w.keys, w.flagbits, counts);
    HD_LAUNCH(first_ball_kernel<D>, dim3((unsigned)cdiv(P.pairs, kThreads / 64)), dim3(kThreads), 0, s, x1, x2,
              perm1, perm2, w.xs2r, w.cstart2, w.boxb, true, w.keys, w.nonfin, b1, b2, p1, p2, P.pairs, out, idx1,
              idx2, counts);
    return check_launch("hausdorff scan");
}

// d = 1..4 in the unsorted modes, after the relayout and the boxes: (cell sort of x2,) seeds,
// scan, final rescan, outputs.
template <int D>
int launch_fast(const Plan &P, const Workspace &w, const float *x1, const float *x2, int64_t b1, int64_t p1,
                int64_t b2, int64_t p2,
                const int64_t *perm1, const int64_t *perm2, float *out, int64_t *idx1, int64_t *idx2,
                hipStream_t s) {
    constexpr bool kCellsOk = D <= 3;
    const bool cells = kCellsOk && P.cells;
    unsigned long long *counts = counts_arg();
    const unsigned per_wave_blocks = (unsigned)cdiv(P.pairs, kThreads / 64);
    if constexpr (kCellsOk) {
        if (cells) {
            const CellSet S2{x2, perm2, w.xs2r, w.bbox, P.clouds2, p2, b2, 1};
            const CellSet none{nullptr, nullptr, nullptr, w.bbox, 0, 1, 1, 1};
            launch_sort<D>(P, w, S2, none, s);
        }
    }
    HD_LAUNCH(seed_select_kernel<D>, dim3((unsigned)P.pairs, (unsigned)cdiv(p1, P.chunk1)), dim3(kThreads), 0, s,
              w.xs1, w.bbox, b1, b2, p1, P.chunk1, P.ncand, w.cand);
    if constexpr (kCellsOk) {
        if (cells)
            HD_LAUNCH(seed_ball_kernel<D>, dim3((unsigned)cdiv(P.pairs * kSeeds, kThreads / 64)), dim3(kThreads), 0,
                      s, x1, perm1, w.xs2r, w.cstart2, w.bbox, false, w.cand,
                      P.ncand, b1, b2, p1, p2, P.pairs, w.seedm, w.keys, counts);
    }
    if (!cells) {
        HD_LAUNCH(seed_pick_kernel, dim3(per_wave_blocks), dim3(kThreads), 0, s, w.cand, P.ncand, P.pairs, w.seedm);
        HD_LAUNCH(list_scan_kernel<D>, dim3((unsigned)P.pairs, (unsigned)P.nchL), dim3(kThreads), 0, s, w.xs1, w.xs2,
                  w.seedm, static_cast<const uint32_t *>(nullptr), (int64_t)kSeeds, b1, b2, p1, p2, P.chunkL,
                  w.seedmin);
        HD_LAUNCH(list_fold_kernel, dim3((unsigned)cdiv(P.pairs * kSeeds, 256)), dim3(256), 0, s, w.seedmin, w.seedm,
                  static_cast<const uint32_t *>(nullptr), (int64_t)kSeeds, P.pairs, w.keys);
    }
    int rc = check_launch("hausdorff seeds");
    if (rc) return rc;
    if constexpr (kCellsOk) {
        if (cells) {
            const int64_t m_per_block = 2048;
            HD_LAUNCH(scan_window_kernel<D>, dim3((unsigned)cdiv(p1, m_per_block), (unsigned)P.pairs),
                      dim3(kThreads), 0, s, w.xs1, w.xs2r, w.cstart2, w.bbox, b1, b2, p1, p2, m_per_block, w.seedm,
                      w.keys, counts);
            HD_LAUNCH(first_ball_kernel<D>, dim3(per_wave_blocks), dim3(kThreads), 0, s, x1, x2, perm1, perm2,
                      w.xs2r, w.cstart2, w.bbox, false, w.keys, w.nonfin, b1, b2, p1, p2, P.pairs, out, idx1, idx2,
                      counts);
        }
    }
    if (!cells) {
        const int64_t m_per_block = 2048;
        const int64_t lds_points = (kLdsFloats / D) / 64 * 64;
        HD_LAUNCH(scan_kernel<D>, dim3((unsigned)cdiv(p1, m_per_block), (unsigned)P.pairs), dim3(kThreads), 0, s,
                  w.xs1, w.xs2, b1, b2, p1, p2, m_per_block, lds_points, w.seedm, w.keys);
        HD_LAUNCH(first_hit_kernel<D>, dim3((unsigned)P.pairs, (unsigned)P.nch2), dim3(kThreads), 0, s, w.xs1, w.xs2,
                  w.keys, b1, b2, p1, p2, P.chunk2, w.first);
        HD_LAUNCH(write_out_kernel, dim3((unsigned)cdiv(P.pairs, 256)), dim3(256), 0, s, w.keys, w.first, perm1,
                  perm2, P.pairs, b1, b2, p1, p2, out, idx1, idx2);
        HD_LAUNCH(exact_fix_kernel, dim3(per_wave_blocks), dim3(kThreads), 0, s, x1, x2, perm1, perm2, w.nonfin, b1,
                  b2, p1, p2, (int64_t)D, P.pairs, out, idx1, idx2, w.keys);
    }
    return check_launch("hausdorff scan");
}

}  // namespace
}  // namespace tpw

using namespace tpw;

extern "C" size_t tpw_hausdorff_workspace_size(int64_t batch, int64_t b1, int64_t p1, int64_t b2,
                                               int64_t p2, int64_t d) {
    if (batch < 0 || b1 < 0 || b2 < 0 || p1 < 0 || p2 < 0 || d < 0) return 0;
    size_t total = 0;
    carve(nullptr, make_plan(batch, b1, p1, b2, p2, d), p1, p2, d, &total);
    return total;
}

extern "C" int tpw_hausdorff_counters(int arm, unsigned long long *out) {
    std::lock_guard<std::mutex> lk(g_counters.mu);
    if (arm) {
        int dev = -1;
        TPW_REQUIRE(hipGetDevice(&dev) == hipSuccess, "no current HIP device");
        void *ptr = nullptr;
        TPW_REQUIRE(hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_hd_counts)) == hipSuccess && ptr,
                    "hipGetSymbolAddress failed");
        TPW_REQUIRE(hipDeviceSynchronize() == hipSuccess, "hipDeviceSynchronize failed");
        TPW_REQUIRE(hipMemset(ptr, 0, sizeof(g_hd_counts)) == hipSuccess, "hipMemset failed");
        TPW_REQUIRE(hipDeviceSynchronize() == hipSuccess, "hipDeviceSynchronize failed");
        g_counters.device = dev;
        g_counters.ptr = static_cast<unsigned long long *>(ptr);
        g_counters.launches = 0;
        __atomic_store_n(&g_counters.armed, true, __ATOMIC_RELAXED);
        return TPW_OK;
    }
    TPW_REQUIRE(out, "null pointer");
    TPW_REQUIRE(g_counters.armed, "the counters are not armed");
    __atomic_store_n(&g_counters.armed, false, __ATOMIC_RELAXED);
    int dev = -1;
    TPW_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev == g_counters.device,
                "read the counters with the device they were armed on current");
    TPW_REQUIRE(hipDeviceSynchronize() == hipSuccess, "hipDeviceSynchronize failed");
    unsigned long long c[2] = {0, 0};
    TPW_REQUIRE(hipMemcpy(c, g_counters.ptr, sizeof(c), hipMemcpyDeviceToHost) == hipSuccess, "hipMemcpy failed");
    out[0] = c[0];
    out[1] = c[1];
    out[2] = g_counters.launches;
    return TPW_OK;
}

extern "C" int tpw_directed_hausdorff(const float *x1, const float *x2, int64_t batch, int64_t b1,
                                      int64_t p1, int64_t b2, int64_t p2, int64_t d,
                                      const int64_t *perm1, const int64_t *perm2, float *out,
                                      int64_t *idx1, int64_t *idx2, void *workspace,
                                      void *stream) {
    TPW_REQUIRE(batch >= 0 && b1 >= 0 && b2 >= 0 && p1 >= 0 && p2 >= 0 && d >= 0, "invalid sizes");
    TPW_REQUIRE(d <= 64, "directed_hausdorff supports at most 64 features on the GPU (got %lld)",
                (long long)d);
    TPW_REQUIRE(p1 < (int64_t)0xffffffffLL, "too many points in x1 (%lld)", (long long)p1);
    const int64_t pairs = batch * b1 * b2;
    if (pairs == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out && idx1 && idx2 && workspace, "null pointer");
    TPW_REQUIRE(pairs <= kMaxGridYZ, "too many cloud pairs (%lld)", (long long)pairs);
    hipStream_t s = as_stream(stream);
    const Plan P = make_plan(batch, b1, p1, b2, p2, d);
    const Workspace w = carve(workspace, P, p1, p2, d);
    if (P.sorted) {
        switch (d) {
            case 1: return launch_sorted<1>(P, w, x1, x2, b1, p1, b2, p2, perm1, perm2, out, idx1, idx2, s);
            case 2: return launch_sorted<2>(P, w, x1, x2, b1, p1, b2, p2, perm1, perm2, out, idx1, idx2, s);
            default: return launch_sorted<3>(P, w, x1, x2, b1, p1, b2, p2, perm1, perm2, out, idx1, idx2, s);
        }
    }
    // presets: keys 0, non-finite flags 0, box keys (+inf, -inf), seed mins +inf, first hits all ones
    Fills fs{};
    int64_t most = 0;
    auto add = [&](void *ptr, int64_t words, uint32_t v0, uint32_t v1) {
        if (!ptr || words <= 0) return;
        fs.f[fs.count++] = Fill{static_cast<uint32_t *>(ptr), words, {v0, v1}};
        most = std::max(most, words);
    };
    add(w.keys, 2 * pairs, 0u, 0u);
    add(w.nonfin, batch, 0u, 0u);
    add(w.boxkeys, 2 * P.box_rows2, kOrderedPosInf, kOrderedNegInf);
    add(w.seedmin, pairs * kSeeds, 0x7f800000u, 0x7f800000u);
    add(w.first, 2 * pairs, 0xffffffffu, 0xffffffffu);
    HD_LAUNCH(fill_kernel, dim3((unsigned)std::min<int64_t>(cdiv(most, 256), 2048)), dim3(256), 0, s, fs);
    int rc = check_launch("hausdorff presets");
    if (rc) return rc;
    if (P.active) {
        HD_LAUNCH(soa_kernel, dim3((unsigned)cdiv(batch * b1 * p1, 256)), dim3(256), 0, s, x1, perm1, batch * b1, b1,
                  p1, (int)d, w.xs1, w.nonfin);
        HD_LAUNCH(soa_kernel, dim3((unsigned)cdiv(batch * b2 * p2, 256)), dim3(256), 0, s, x2, perm2, batch * b2, b2,
                  p2, (int)d, w.xs2, w.nonfin);
        HD_LAUNCH(bbox_rows_kernel, dim3((unsigned)P.box_rows2, (unsigned)P.box_chunks), dim3(kThreads), 0, s,
                  w.xs1, (int64_t)0, p1, w.xs2, p2, P.box_chunk, w.boxkeys);
        HD_LAUNCH(box_finish_kernel, dim3((unsigned)cdiv(P.box_rows2, 256)), dim3(256), 0, s, w.boxkeys,
                  (int64_t)0, P.box_rows2, static_cast<float *>(nullptr), w.bbox, batch, b1, b2, (int)d,
                  static_cast<float *>(nullptr));
        rc = check_launch("hausdorff prologue");
        if (rc) return rc;
        if (P.fast) {
            switch (d) {
                case 1: return launch_fast<1>(P, w, x1, x2, b1, p1, b2, p2, perm1, perm2, out, idx1, idx2, s);
                case 2: return launch_fast<2>(P, w, x1, x2, b1, p1, b2, p2, perm1, perm2, out, idx1, idx2, s);
                case 3: return launch_fast<3>(P, w, x1, x2, b1, p1, b2, p2, perm1, perm2, out, idx1, idx2, s);
                default: return launch_fast<4>(P, w, x1, x2, b1, p1, b2, p2, perm1, perm2, out, idx1, idx2, s);
            }
        }
        HD_LAUNCH(seed_kernel<0>, dim3((unsigned)pairs), dim3(kThreads), 0, s, w.xs1, w.xs2, w.bbox, b1, b2, p1, p2,
                  (int)d, w.keys);
        HD_LAUNCH(scan_kernel_any, dim3((unsigned)cdiv(p1, 2048), (unsigned)pairs), dim3(kThreads), 0, s, w.xs1,
                  w.xs2, b1, b2, p1, p2, (int)d, (int64_t)2048, w.keys);
        rc = check_launch("hausdorff scan_kernel_any");
        if (rc) return rc;
    }
    HD_LAUNCH(finalize_kernel<0>, dim3((unsigned)cdiv(pairs, kThreads / 64)), dim3(kThreads), 0, s, w.xs1, w.xs2,
              w.keys, perm1, perm2, pairs, b1, b2, p1, p2, (int)d, out, idx1, idx2);
    if (P.active)
        HD_LAUNCH(exact_fix_kernel, dim3((unsigned)cdiv(pairs, kThreads / 64)), dim3(kThreads), 0, s, x1, x2, perm1,
                  perm2, w.nonfin, b1, b2, p1, p2, d, pairs, out, idx1, idx2, w.keys);
    return check_launch("hausdorff finalize_kernel");
}

extern "C" int tpw_directed_hausdorff_backward(const float *grad, const float *x1,
                                               const float *x2, const float *out,
                                               const int64_t *idx1, const int64_t *idx2,
                                               int64_t batch, int64_t b1, int64_t p1, int64_t b2,
                                               int64_t p2, int64_t d, float *grad_x1,
                                               float *grad_x2, void *stream) {
    TPW_REQUIRE(batch >= 0 && b1 >= 0 && b2 >= 0 && p1 >= 0 && p2 >= 0 && d >= 0, "invalid sizes");
    if (batch * b1 * b2 == 0 || d == 0 || p1 == 0 || p2 == 0) return TPW_OK;
    TPW_REQUIRE(grad && x1 && x2 && out && idx1 && idx2 && grad_x1 && grad_x2, "null pointer");
    hipStream_t s = as_stream(stream);
    const int64_t n1 = batch * b1 * p1 * d, n2 = batch * b2 * p2 * d;
    // a fill of both gradients, then the scatter: a wave per cloud for at most 64 clouds per side
    // (C5: 16), else one thread per (cloud, feature) passing over the other side's clouds
    Fills fs{};
    fs.f[fs.count++] = Fill{reinterpret_cast<uint32_t *>(grad_x1), n1, {0u, 0u}};
    fs.f[fs.count++] = Fill{reinterpret_cast<uint32_t *>(grad_x2), n2, {0u, 0u}};
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)std::min<int64_t>(cdiv(std::max(n1, n2), 256), 2048)), dim3(256),
                       0, s, fs);
    if (b1 <= 64 && b2 <= 64) {
        hipLaunchKernelGGL(backward_wave_kernel, dim3((unsigned)cdiv(batch * (b1 + b2), 4)), dim3(256), 0, s, grad,
                           x1, x2, out, idx1, idx2, batch, b1, p1, b2, p2, d, grad_x1, grad_x2);
        return check_launch("hausdorff backward");
    }
    hipLaunchKernelGGL(backward_x1_kernel, dim3((unsigned)cdiv(batch * b1 * d, 256)), dim3(256), 0,
                       s, grad, x1, x2, out, idx1, idx2, batch, b1, p1, b2, p2, d, grad_x1);
    hipLaunchKernelGGL(backward_x2_kernel, dim3((unsigned)cdiv(batch * b2 * d, 256)), dim3(256), 0,
                       s, grad, x1, x2, out, idx1, idx2, batch, b1, p1, b2, p2, d, grad_x2);
    return check_launch("hausdorff backward");
}
