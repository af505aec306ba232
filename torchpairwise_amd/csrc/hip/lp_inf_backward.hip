// Backward of _ppminkowski / _wminkowski at p = +inf (max over k) and p = -inf (min over k)
// (reference: csrc/ops/cpu/ppminkowski_kernel.cpp:171-208, cpu/wminkowski_kernel.cpp:214-265;
// its CUDA kernels use atomics, cuda/ppminkowski_kernel.cu:182-218, wminkowski_kernel.cu:224-265).
//
// Per pair (i, j) the reference takes the first k with the largest (smallest) |d_k| (times
// w_k), d = x1[i] - x2[j], keeping k = 0 unless a later value compares strictly greater
// (smaller), so a NaN is never taken over, and scatters
//     grad_x1[i][k] += g[i,j] (* w[k]) * sgn(d_k),   grad_x2[j][k] += g[i,j] (* w[k]) * -sgn(d_k),
//     grad_w[k]     += g[i,j] * |d_k|                (weighted only)
// with sgn(NaN) = sgn(0) = 0.  Here one wave owns one row of the side being differentiated and
// walks the other side in index order, 64 partners per step (one per lane); the lanes' terms
// are then added to the row's accumulator one lane at a time in partner order, which is the
// reference's order for grad_x1 (j ascending) and grad_x2 (i ascending), without atomics.  The
// weight gradient is summed per row of x1 (j ascending) and the rows are then added in order.
// The accumulator is the row's LDS slice while four waves' rows fit in LDS; past that (GACC) it
// is the wave's own output row in global memory (and its wrows row), which no other wave
// touches, so lane 0 alone zeroes it and adds into it in the same order: any d, same bits.
#include "common.hpp"

#pragma clang fp contract(off)

namespace tpw {
namespace {

constexpr int kWaves = 4;

__device__ __forceinline__ float signum(float v) { return (float)((0.0f < v) - (v < 0.0f)); }

// COLS = false: rows of x1 (output grad_x1, and per-row weight-gradient partials when W);
// COLS = true: rows of x2 (output grad_x2), walking x1.
template <bool NEG, bool W, bool COLS, bool GACC>
__global__ __launch_bounds__(kWaves * 64) void lp_inf_grad_kernel(
    const float *__restrict__ g, const float *__restrict__ x1, const float *__restrict__ x2,
    const float *__restrict__ w, int64_t n, int64_t m, int64_t d, float *__restrict__ out,
    float *__restrict__ wrows) {
    extern __shared__ float lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t b = blockIdx.y;
    const int64_t own_rows = COLS ? m : n, other_rows = COLS ? n : m;
    const int64_t r = (int64_t)blockIdx.x * kWaves + wave;
    if (r >= own_rows) return;  // a whole wave: no block-wide barrier follows
    float *dst = out + (b * own_rows + r) * d;
    float *wdst = W && !COLS ? wrows + (b * n + r) * d : nullptr;
    // LDS slices, or (GACC) the wave's own rows of out / wrows
    float *acc = GACC ? dst : lds + (int64_t)wave * (W && !COLS ? 2 : 1) * d;
    float *gacc = GACC ? wdst : acc + d;  // weight-gradient partial of this row (W, rows pass)
    if constexpr (GACC) {
        // one lane zeroes and later updates the rows, so every access to them is in its order
        if (lane == 0)
            for (int64_t k = 0; k < d; ++k) {
                acc[k] = 0.0f;
                if constexpr (W && !COLS) gacc[k] = 0.0f;
            }
    } else {
        for (int64_t k = lane; k < d; k += 64) {
            acc[k] = 0.0f;
            if constexpr (W && !COLS) gacc[k] = 0.0f;
        }
    }
    const float *own = (COLS ? x2 + b * m * d : x1 + b * n * d) + r * d;
    const float *oth = COLS ? x1 + b * n * d : x2 + b * m * d;
    const float *wb = W ? w + b * d : nullptr;
    const float *G = g + b * n * m;
    for (int64_t p0 = 0; p0 < other_rows; p0 += 64) {
        const int64_t p = p0 + lane;
        const bool ok = p < other_rows;
        const float *q = oth + (ok ? p : 0) * d;
        // d_k = x1 - x2 whichever side this wave owns
        float a0 = COLS ? q[0] : own[0], c0 = COLS ? own[0] : q[0];
        float best_d = a0 - c0, best_a = fabsf(best_d);
        float best_v = W ? best_a * wb[0] : best_a;
        int64_t best_k = 0;
        for (int64_t k = 1; k < d; ++k) {
            const float a = COLS ? q[k] : own[k], c = COLS ? own[k] : q[k];
            const float t = a - c, ta = fabsf(t);
            const float tv = W ? ta * wb[k] : ta;
            const bool take = NEG ? (tv < best_v) : (tv > best_v);
            if (take) {
                best_d = t;
                best_a = ta;
                best_v = tv;
                best_k = k;
            }
        }
        const float gv = ok ? G[COLS ? p * m + r : r * m + p] : 0.0f;
        const float sg = COLS ? -signum(best_d) : signum(best_d);
        const float term = W ? (gv * wb[best_k]) * sg : gv * sg;
        const float gterm = W && !COLS ? gv * best_a : 0.0f;
        // add the 64 partners' terms in partner order (lane order)
        const int64_t valid = other_rows - p0 < 64 ? other_rows - p0 : 64;
        for (int l = 0; l < valid; ++l) {
            const int kk = __shfl((int)best_k, l, 64);
            const float t = __shfl(term, l, 64);
            const float gt = __shfl(gterm, l, 64);
            if (lane == 0) {
                acc[kk] += t;
                if constexpr (W && !COLS) gacc[kk] += gt;
            }
        }
    }
    if constexpr (!GACC)
        for (int64_t k = lane; k < d; k += 64) {
            dst[k] = acc[k];
            if constexpr (W && !COLS) wdst[k] = gacc[k];
        }
}

// Largest feature count whose per-row accumulators (four waves' rows) live in LDS.
int64_t lds_max_features(bool weighted) { return weighted ? 2048 : 4096; }

template <bool NEG, bool W, bool COLS>
int launch(const float *g, const float *x1, const float *x2, const float *w, int64_t batch, int64_t n,
           int64_t m, int64_t d, float *out, float *wrows, hipStream_t s) {
    const int64_t rows = COLS ? m : n;
    const dim3 grid((unsigned)cdiv(rows, kWaves), (unsigned)batch);
    if (d <= lds_max_features(W)) {
        const size_t lds = (size_t)kWaves * (W && !COLS ? 2 : 1) * d * sizeof(float);
        hipLaunchKernelGGL((lp_inf_grad_kernel<NEG, W, COLS, false>), grid, dim3(kWaves * 64), lds, s, g, x1, x2,
                           w, n, m, d, out, wrows);
    } else {
        hipLaunchKernelGGL((lp_inf_grad_kernel<NEG, W, COLS, true>), grid, dim3(kWaves * 64), 0, s, g, x1, x2, w,
                           n, m, d, out, wrows);
    }
    return check_launch("lp_inf_grad_kernel");
}

template <bool NEG, bool W>
int run(const float *g, const float *x1, const float *x2, const float *w, int64_t batch, int64_t n, int64_t m,
        int64_t d, float *gx1, float *gx2, float *wrows, hipStream_t s) {
    int rc = launch<NEG, W, false>(g, x1, x2, w, batch, n, m, d, gx1, wrows, s);
    if (rc != TPW_OK) return rc;
    return launch<NEG, W, true>(g, x1, x2, w, batch, n, m, d, gx2, nullptr, s);
}

}  // namespace

// grad_x1 [batch, n, d], grad_x2 [batch, m, d] and, with w, the per-row weight-gradient
// partials wrows [batch, n, d] (summed over rows by the caller); every element written.
int lp_inf_backward(const float *g, const float *x1, const float *x2, const float *w, int64_t batch, int64_t n,
                    int64_t m, int64_t d, bool neg, float *gx1, float *gx2, float *wrows, hipStream_t s) {
    TPW_REQUIRE(batch <= kMaxGridYZ && cdiv(n > m ? n : m, kWaves) <= 0x7fffffffLL, "sizes exceed the launch grid");
    if (w) return neg ? run<true, true>(g, x1, x2, w, batch, n, m, d, gx1, gx2, wrows, s)
                      : run<false, true>(g, x1, x2, w, batch, n, m, d, gx1, gx2, wrows, s);
    return neg ? run<true, false>(g, x1, x2, nullptr, batch, n, m, d, gx1, gx2, nullptr, s)
               : run<false, false>(g, x1, x2, nullptr, batch, n, m, d, gx1, gx2, nullptr, s);
}

}  // namespace tpw
