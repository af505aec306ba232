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
//      flags fit (pairs x p1 bytes <= 256 MiB), x1 is sorted by cell too, in a frame shared
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
// (value, m position) exactly.
#include "common.hpp"

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

// xs[c][k][pos] = x[c][perm ? perm[batch_of(c)][pos] : pos][k]
__global__ void soa_kernel(const float *__restrict__ x, const int64_t *__restrict__ perm,
                           int64_t clouds, int64_t clouds_per_batch, int64_t p, int d,
                           float *__restrict__ xs) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= clouds * p) return;
    const int64_t c = t / p, pos = t - c * p;
    const int64_t src = perm ? perm[(c / clouds_per_batch) * p + pos] : pos;
    const float *s = x + (c * p + src) * d;
    float *o = xs + c * d * p + pos;
    for (int k = 0; k < d; ++k) o[(int64_t)k * p] = s[k];
}

// bbox[c][k][0] = min, [1] = max over the points of cloud c (SoA input)
__global__ void bbox_kernel(const float *__restrict__ xs, int64_t p, int d,
                            float *__restrict__ bbox) {
    __shared__ float red[2][kThreads];
    const int64_t c = blockIdx.x;
    for (int k = 0; k < d; ++k) {
        const float *row = xs + (c * d + k) * p;
        float lo = INFINITY, hi = -INFINITY;
        for (int64_t n = threadIdx.x; n < p; n += kThreads) {
            const float v = row[n];
            lo = fminf(lo, v);
            hi = fmaxf(hi, v);
        }
        red[0][threadIdx.x] = lo;
        red[1][threadIdx.x] = hi;
        __syncthreads();
        for (int s = kThreads / 2; s > 0; s >>= 1) {
            if (threadIdx.x < s) {
                red[0][threadIdx.x] = fminf(red[0][threadIdx.x], red[0][threadIdx.x + s]);
                red[1][threadIdx.x] = fmaxf(red[1][threadIdx.x], red[1][threadIdx.x + s]);
            }
            __syncthreads();
        }
        if (threadIdx.x == 0) {
            bbox[(c * d + k) * 2 + 0] = red[0][0];
            bbox[(c * d + k) * 2 + 1] = red[1][0];
        }
        __syncthreads();
    }
}

__global__ void zero_keys_kernel(unsigned long long *keys, int64_t count) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < count) keys[t] = 0ull;
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

// ---------------------------------------------------------------------------------------
// Scan with a spatial first guess (D = 1, 2, 3).  Pruning an m needs only one distance below
// T, and an m that is never pruned gets its exact min whatever order x2 is visited in.  Each
// x2 cloud is therefore counting-sorted once by a grid cell (4096 cells over the cloud's
// bounding box; Morton order of 16^3 / 64^2 cells, or 4096 intervals for D = 1), and the scan
// first tries, for every m, the 64 sorted points at m's own cell, which almost always hold
// one within T.  x1 stays in iteration order, so the m that need more (points far from x2,
// with mins near T) are spread evenly over the waves.
constexpr int kCells = 4096;

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

// Counting sort of one cloud (block) by cell, in the frame of boxes[c / clouds_per_box], into
// xs_sorted (SoA), with, when given, each sorted point's iteration position (pos) and the
// cloud's cell start offsets (cstart, kCells + 1).  Points of one cell land in an unspecified order (LDS
// atomics); nothing depends on it.
template <int D>
__global__ __launch_bounds__(kThreads) void cell_sort_kernel(const float *__restrict__ xs, int64_t p,
                                                             const float *__restrict__ boxes,
                                                             int64_t clouds_per_box,
                                                             float *__restrict__ xs_sorted,
                                                             uint32_t *__restrict__ pos,
                                                             int32_t *__restrict__ cstart) {
    __shared__ uint32_t cnt[kCells];
    __shared__ uint32_t part[kThreads];
    const int64_t c = blockIdx.x;
    const float *X = xs + c * D * p;
    float fr[2 * D];
    frame_of<D>(boxes + (c / clouds_per_box) * D * 2, fr);
    for (int t = threadIdx.x; t < kCells; t += kThreads) cnt[t] = 0u;
    __syncthreads();
    for (int64_t n = threadIdx.x; n < p; n += kThreads) {
        float a[D];
#pragma unroll
        for (int k = 0; k < D; ++k) a[k] = X[k * p + n];
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
        run += v;
    }
    if (cstart && threadIdx.x == 0) cstart[c * (kCells + 1) + kCells] = (int32_t)p;
    __syncthreads();
    float *O = xs_sorted + c * D * p;
    for (int64_t n = threadIdx.x; n < p; n += kThreads) {
        float a[D];
#pragma unroll
        for (int k = 0; k < D; ++k) a[k] = X[k * p + n];
        const uint32_t slot = atomicAdd(&cnt[cell_of<D>(a, fr)], 1u);
#pragma unroll
        for (int k = 0; k < D; ++k) O[k * p + slot] = a[k];
        if (pos) pos[c * p + slot] = (uint32_t)n;
    }
}

// The whole wave scans all of x2 (sorted) for one m with coordinates b, circularly from st,
// four 64-point steps in flight, and drops m at the first d < T; an m never dropped folds its
// exact min with its iteration position mpos.
template <int D>
__device__ __forceinline__ void wave_full_scan(const float (&b)[D], const float *X2, int64_t p2, int64_t st,
                                               unsigned long long *key, int64_t mpos) {
    const int lane = threadIdx.x & 63;
    float T = threshold_of(key);
    float best = INFINITY;
    int64_t t0 = 0;
    for (; t0 + 256 <= p2; t0 += 256) {
        float dd[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            int64_t n = st + t0 + 64 * u + lane;
            if (n >= p2) n -= p2;
            dd[u] = sqdist_fixed<D>(b, X2, p2, n);
        }
        const float dmin = fminf(fminf(dd[0], dd[1]), fminf(dd[2], dd[3]));
        if (__any(dmin < T)) return;
        best = fminf(best, dmin);
        if ((t0 & 4095) == 3840) T = threshold_of(key);
    }
    for (; t0 < p2; t0 += 64) {
        const int64_t t = t0 + lane;
        int64_t n = st + t;
        if (n >= p2) n -= p2;
        const float dd = t < p2 ? sqdist_fixed<D>(b, X2, p2, n) : INFINITY;
        if (__any(dd < T)) return;
        best = fminf(best, dd);
    }
    const float mn = wave_min(best);
    if (lane == 0) fold_key(key, mn, mpos);
}

// Start of m's 64-point window in the sorted x2 of a cloud: 32 before its cell's first point,
// clamped to a full window.
template <int D>
__device__ __forceinline__ int64_t window_start(const float (&a)[D], const float (&fr)[2 * D],
                                                const int32_t *CS, int64_t p2) {
    const int64_t wstart = p2 > 64 ? p2 - 64 : 0;
    int64_t s0 = (int64_t)CS[cell_of<D>(a, fr)] - 32;
    s0 = s0 > wstart ? wstart : s0;
    return s0 < 0 ? 0 : s0;
}

// Block = 2048 consecutive m of one pair; each wave takes 64 m at a time, one per lane.  A
// lane checks the 64 sorted x2 points of its window and stops at the first d < T.
//   SORTED (x1 sorted by cell in the batch frame, pos1 = iteration positions): neighbouring
//     lanes share windows, so the loads coalesce; each lane writes flag[pair][m position] =
//     "not dropped", and scan_flagged_kernel scans those m in iteration order.
//   otherwise (x1 in iteration order, x2 sorted in its cloud's own frame): the lanes left
//     (ballot) are scanned in turn by the whole wave (wave_full_scan).
template <int D, bool SORTED>
__global__ __launch_bounds__(kThreads) void scan_window_kernel(
    const float *__restrict__ xs1, const uint32_t *__restrict__ pos1, const float *__restrict__ xs2s,
    const int32_t *__restrict__ cstart2, const float *__restrict__ boxes, int64_t b1, int64_t b2,
    int64_t p1, int64_t p2, int64_t m_per_block, unsigned long long *__restrict__ keys,
    uint8_t *__restrict__ flags) {
    const int64_t pair = blockIdx.y;
    const int64_t per_batch = b1 * b2;
    const int64_t bb = pair / per_batch, rem = pair - bb * per_batch;
    const int64_t i = rem / b2, j = rem - i * b2;
    const float *X1 = xs1 + (bb * b1 + i) * D * p1;
    const float *X2 = xs2s + (bb * b2 + j) * D * p2;
    const int32_t *CS = cstart2 + (bb * b2 + j) * (kCells + 1);
    float fr[2 * D];
    frame_of<D>(boxes + (SORTED ? bb : bb * b2 + j) * D * 2, fr);
    const int lane = threadIdx.x & 63;
    const int64_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // the same in every lane
    const int64_t mbeg = (int64_t)blockIdx.x * m_per_block;
    const int64_t mend = mbeg + m_per_block < p1 ? mbeg + m_per_block : p1;
    const int64_t wlen = p2 < 64 ? p2 : 64;
    unsigned long long *key = &keys[pair];
    for (int64_t m0 = mbeg + 64 * wave; m0 < mend; m0 += 64 * (kThreads / 64)) {
        const int64_t m = m0 + lane;
        const bool valid = m < mend;
        float a[D];
#pragma unroll
        for (int k = 0; k < D; ++k) a[k] = valid ? X1[k * p1 + m] : 0.0f;
        const int64_t s0 = window_start<D>(a, fr, CS, p2);
        const float T = threshold_of(key);
        // the window (fewer points when p2 < 64), 8 per step so that their loads are in flight
        // together
        bool done = !valid;
        for (int64_t t = 0; t < wlen && !done; t += 8) {
            bool hit = false;
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (t + u < wlen) hit = hit | (sqdist_fixed<D>(a, X2, p2, s0 + t + u) < T);
            done = hit;
        }
        if constexpr (SORTED) {
            if (valid) flags[pair * p1 + pos1[(bb * b1 + i) * p1 + m]] = done ? 0 : 1;
        } else {
            unsigned long long left = __ballot(!done);
            while (left) {
                const int l = __builtin_ctzll(left);
                left &= left - 1;
                float b[D];
#pragma unroll
                for (int k = 0; k < D; ++k)
                    b[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a[k]), l));
                const int64_t st = (int64_t)(uint32_t)__builtin_amdgcn_readlane((int)s0, l);
                wave_full_scan<D>(b, X2, p2, st, key, m0 + l);
            }
        }
    }
}

// The m the window pass of the sorted mode left (flags), in iteration order: each wave takes
// 64 consecutive m, and the flagged ones are scanned in turn by the whole wave.  The m far from
// x2 cluster in the sorted order; here they are spread over the grid.
template <int D>
__global__ __launch_bounds__(kThreads) void scan_flagged_kernel(
    const float *__restrict__ xs1, const float *__restrict__ xs2s, const int32_t *__restrict__ cstart2,
    const float *__restrict__ boxes, int64_t b1, int64_t b2, int64_t p1, int64_t p2,
    unsigned long long *__restrict__ keys, const uint8_t *__restrict__ flags) {
    const int64_t pair = blockIdx.y;
    const int64_t per_batch = b1 * b2;
    const int64_t bb = pair / per_batch, rem = pair - bb * per_batch;
    const int64_t i = rem / b2, j = rem - i * b2;
    const float *X1 = xs1 + (bb * b1 + i) * D * p1;
    const float *X2 = xs2s + (bb * b2 + j) * D * p2;
    const int32_t *CS = cstart2 + (bb * b2 + j) * (kCells + 1);
    float fr[2 * D];
    frame_of<D>(boxes + bb * D * 2, fr);
    const int lane = threadIdx.x & 63;
    const int64_t m0 = (int64_t)blockIdx.x * kThreads + 64 * __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t m = m0 + lane;
    const bool flagged = m < p1 && flags[pair * p1 + m] != 0;
    unsigned long long left = __ballot(flagged);
    while (left) {
        const int l = __builtin_ctzll(left);
        left &= left - 1;
        float b[D];
#pragma unroll
        for (int k = 0; k < D; ++k) b[k] = X1[k * p1 + m0 + l];
        wave_full_scan<D>(b, X2, p2, window_start<D>(b, fr, CS, p2), &keys[pair], m0 + l);
    }
}

// bbox of each batch over both sides' cloud bounding boxes (the shared frame of the sorted mode)
__global__ void batch_box_kernel(const float *__restrict__ bbox1, const float *__restrict__ bbox2,
                                 int64_t batch, int64_t b1, int64_t b2, int d, float *__restrict__ boxb) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= batch * d) return;
    const int64_t bb = t / d;
    const int k = (int)(t - bb * d);
    float lo = INFINITY, hi = -INFINITY;
    for (int64_t c = 0; c < b1; ++c) {
        lo = fminf(lo, bbox1[((bb * b1 + c) * d + k) * 2]);
        hi = fmaxf(hi, bbox1[((bb * b1 + c) * d + k) * 2 + 1]);
    }
    for (int64_t c = 0; c < b2; ++c) {
        lo = fminf(lo, bbox2[((bb * b2 + c) * d + k) * 2]);
        hi = fmaxf(hi, bbox2[((bb * b2 + c) * d + k) * 2 + 1]);
    }
    boxb[t * 2] = lo;
    boxb[t * 2 + 1] = hi;
}

// The sorted mode keeps one flag byte per (pair, m): up to 256 MiB of them.
inline bool sorted_mode(int64_t pairs, int64_t p1) { return pairs * p1 <= ((int64_t)1 << 28); }

struct Workspace {
    float *xs1, *xs2, *bbox, *xs2s, *bbox1, *boxb, *xs1s;
    unsigned long long *keys;
    int32_t *cstart2;
    uint32_t *pos1;
    uint8_t *flags;
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// [keys | x2 bboxes | x1 SoA | x2 SoA | sorted x2 | x2 cell starts | x1 bboxes | batch boxes |
//  sorted x1 | x1 positions | flags]; from sorted x2 on only for d <= 3, from x1 bboxes on only
// in the sorted mode.
Workspace carve(void *ws, int64_t batch, int64_t b1, int64_t p1, int64_t b2, int64_t p2, int64_t d,
                size_t *total = nullptr) {
    char *base = static_cast<char *>(ws), *p = base;
    auto take = [&](size_t bytes) {
        char *r = p;
        p += align256(bytes);
        return r;
    };
    const int64_t pairs = batch * b1 * b2;
    Workspace w;
    w.keys = reinterpret_cast<unsigned long long *>(take(sizeof(unsigned long long) * pairs));
    w.bbox = reinterpret_cast<float *>(take(sizeof(float) * batch * b2 * d * 2));
    w.xs1 = reinterpret_cast<float *>(take(sizeof(float) * batch * b1 * p1 * d));
    w.xs2 = reinterpret_cast<float *>(take(sizeof(float) * batch * b2 * p2 * d));
    const bool cells = d >= 1 && d <= 3;
    const bool sorted = cells && sorted_mode(pairs, p1);
    w.xs2s = reinterpret_cast<float *>(take(cells ? sizeof(float) * batch * b2 * p2 * d : 0));
    w.cstart2 = reinterpret_cast<int32_t *>(take(cells ? sizeof(int32_t) * batch * b2 * (kCells + 1) : 0));
    w.bbox1 = reinterpret_cast<float *>(take(sorted ? sizeof(float) * batch * b1 * d * 2 : 0));
    w.boxb = reinterpret_cast<float *>(take(sorted ? sizeof(float) * batch * d * 2 : 0));
    w.xs1s = reinterpret_cast<float *>(take(sorted ? sizeof(float) * batch * b1 * p1 * d : 0));
    w.pos1 = reinterpret_cast<uint32_t *>(take(sorted ? sizeof(uint32_t) * batch * b1 * p1 : 0));
    w.flags = reinterpret_cast<uint8_t *>(take(sorted ? (size_t)(pairs * p1) : 0));
    if (total) *total = (size_t)(p - base);
    return w;
}

// Steps 3-4 for d <= 3 (see the kernels): cell sort of x2 (and, in the sorted mode, of x1),
// then the window pass and the scan of the m it leaves.
template <int D>
int launch_cells(const Workspace &w, int64_t batch, int64_t b1, int64_t p1, int64_t b2, int64_t p2,
                 hipStream_t s) {
    const int64_t pairs = batch * b1 * b2;
    const int64_t m_per_block = 2048;
    const dim3 grid((unsigned)cdiv(p1, m_per_block), (unsigned)pairs);
    if (sorted_mode(pairs, p1)) {
        hipLaunchKernelGGL(bbox_kernel, dim3((unsigned)(batch * b1)), dim3(kThreads), 0, s, w.xs1, p1, D,
                           w.bbox1);
        hipLaunchKernelGGL(batch_box_kernel, dim3((unsigned)cdiv(batch * D, 256)), dim3(256), 0, s, w.bbox1,
                           w.bbox, batch, b1, b2, D, w.boxb);
        hipLaunchKernelGGL(cell_sort_kernel<D>, dim3((unsigned)(batch * b2)), dim3(kThreads), 0, s, w.xs2, p2,
                           w.boxb, b2, w.xs2s, static_cast<uint32_t *>(nullptr), w.cstart2);
        hipLaunchKernelGGL(cell_sort_kernel<D>, dim3((unsigned)(batch * b1)), dim3(kThreads), 0, s, w.xs1, p1,
                           w.boxb, b1, w.xs1s, w.pos1, static_cast<int32_t *>(nullptr));
        hipLaunchKernelGGL((scan_window_kernel<D, true>), grid, dim3(kThreads), 0, s, w.xs1s, w.pos1, w.xs2s,
                           w.cstart2, w.boxb, b1, b2, p1, p2, m_per_block, w.keys, w.flags);
        hipLaunchKernelGGL(scan_flagged_kernel<D>, dim3((unsigned)cdiv(p1, kThreads), (unsigned)pairs),
                           dim3(kThreads), 0, s, w.xs1, w.xs2s, w.cstart2, w.boxb, b1, b2, p1, p2, w.keys,
                           w.flags);
    } else {
        hipLaunchKernelGGL(cell_sort_kernel<D>, dim3((unsigned)(batch * b2)), dim3(kThreads), 0, s, w.xs2, p2,
                           w.bbox, (int64_t)1, w.xs2s, static_cast<uint32_t *>(nullptr), w.cstart2);
        hipLaunchKernelGGL((scan_window_kernel<D, false>), grid, dim3(kThreads), 0, s, w.xs1,
                           static_cast<const uint32_t *>(nullptr), w.xs2s, w.cstart2, w.bbox, b1, b2, p1, p2,
                           m_per_block, w.keys, static_cast<uint8_t *>(nullptr));
    }
    return check_launch("hausdorff cell scan");
}

}  // namespace
}  // namespace tpw

using namespace tpw;

extern "C" size_t tpw_hausdorff_workspace_size(int64_t batch, int64_t b1, int64_t p1, int64_t b2,
                                               int64_t p2, int64_t d) {
    size_t total = 0;
    carve(nullptr, batch, b1, p1, b2, p2, d, &total);
    return total;
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
    Workspace w = carve(workspace, batch, b1, p1, b2, p2, d);
    hipLaunchKernelGGL(zero_keys_kernel, dim3((unsigned)cdiv(pairs, 256)), dim3(256), 0, s, w.keys,
                       pairs);
    int rc = check_launch("zero_keys_kernel");
    if (rc) return rc;
    if (p1 > 0 && p2 > 0 && d > 0) {
        hipLaunchKernelGGL(soa_kernel, dim3((unsigned)cdiv(batch * b1 * p1, 256)), dim3(256), 0, s,
                           x1, perm1, batch * b1, b1, p1, (int)d, w.xs1);
        hipLaunchKernelGGL(soa_kernel, dim3((unsigned)cdiv(batch * b2 * p2, 256)), dim3(256), 0, s,
                           x2, perm2, batch * b2, b2, p2, (int)d, w.xs2);
        hipLaunchKernelGGL(bbox_kernel, dim3((unsigned)(batch * b2)), dim3(kThreads), 0, s, w.xs2,
                           p2, (int)d, w.bbox);
        auto seed = d == 1 ? seed_kernel<1> : d == 2 ? seed_kernel<2> : d == 3 ? seed_kernel<3>
                  : d == 4 ? seed_kernel<4> : seed_kernel<0>;
        hipLaunchKernelGGL(seed, dim3((unsigned)pairs), dim3(kThreads), 0, s, w.xs1, w.xs2,
                           w.bbox, b1, b2, p1, p2, (int)d, w.keys);
        rc = check_launch("hausdorff prologue");
        if (rc) return rc;
        if (d <= 3 && p2 < (int64_t)0x7fffffff - 64) {  // cell starts are int32
            rc = d == 1 ? launch_cells<1>(w, batch, b1, p1, b2, p2, s)
               : d == 2 ? launch_cells<2>(w, batch, b1, p1, b2, p2, s)
                        : launch_cells<3>(w, batch, b1, p1, b2, p2, s);
            if (rc) return rc;
        } else {
        const int64_t m_per_block = 2048;
        dim3 grid((unsigned)cdiv(p1, m_per_block), (unsigned)pairs);
        const int64_t lds_points = (kLdsFloats / d) / 64 * 64;
        switch (d) {
            case 1: hipLaunchKernelGGL(scan_kernel<1>, grid, dim3(kThreads), 0, s, w.xs1, w.xs2, b1, b2, p1, p2, m_per_block, lds_points, w.keys); break;
            case 2: hipLaunchKernelGGL(scan_kernel<2>, grid, dim3(kThreads), 0, s, w.xs1, w.xs2, b1, b2, p1, p2, m_per_block, lds_points, w.keys); break;
            case 3: hipLaunchKernelGGL(scan_kernel<3>, grid, dim3(kThreads), 0, s, w.xs1, w.xs2, b1, b2, p1, p2, m_per_block, lds_points, w.keys); break;
            case 4: hipLaunchKernelGGL(scan_kernel<4>, grid, dim3(kThreads), 0, s, w.xs1, w.xs2, b1, b2, p1, p2, m_per_block, lds_points, w.keys); break;
            default: hipLaunchKernelGGL(scan_kernel_any, grid, dim3(kThreads), 0, s, w.xs1, w.xs2, b1, b2, p1, p2, (int)d, m_per_block, w.keys); break;
        }
        rc = check_launch("hausdorff scan_kernel");
        if (rc) return rc;
        }
    }
    auto fin = d == 1 ? finalize_kernel<1> : d == 2 ? finalize_kernel<2> : d == 3 ? finalize_kernel<3>
             : d == 4 ? finalize_kernel<4> : finalize_kernel<0>;
    hipLaunchKernelGGL(fin, dim3((unsigned)cdiv(pairs, kThreads / 64)), dim3(kThreads),
                       0, s, w.xs1, w.xs2, w.keys, perm1, perm2, pairs, b1, b2, p1, p2, (int)d, out,
                       idx1, idx2);
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
    hipLaunchKernelGGL(backward_x1_kernel, dim3((unsigned)cdiv(batch * b1 * d, 256)), dim3(256), 0,
                       s, grad, x1, x2, out, idx1, idx2, batch, b1, p1, b2, p2, d, grad_x1);
    hipLaunchKernelGGL(backward_x2_kernel, dim3((unsigned)cdiv(batch * b2 * d, 256)), dim3(256), 0,
                       s, grad, x1, x2, out, idx1, idx2, batch, b1, p1, b2, p2, d, grad_x2);
    return check_launch("hausdorff backward");
}
