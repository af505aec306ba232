// The reference's directed Hausdorff loop (cpu/hausdorff_kernel.cpp:12-100,
// cuda/hausdorff_kernel.cu:16-105) for one cloud pair, executed by one wave in the loop's own
// order:
//
//   best = 0
//   for m in (shuffled) order:                       row_min = inf
//       for n in (shuffled) order:                   s = sum_k (x1[m,k] - x2[n,k])^2
//           if s < best: break                       (early exit: this m cannot raise best)
//           if s < row_min: row_min = s, (m_c, n_c) = (m, n)
//       if row_min >= best and s >= best: best = row_min, (m_best, n_best) = (m_c, n_c)
//   out = sqrt(best), indices (m_best, n_best)
//
// The wave takes the n loop 64 points at a time: each lane forms one point's s, a ballot finds
// the first lane that breaks, and the strict running minimum over the lanes before it is the
// chunk's minimum with its first lane, which is what the sequential loop records.  The state
// (best, row_min, the last s, the candidate indices, which carry over from one m to the next as
// in the loop) is the same in every lane, so the result equals the CPU loop's bit for bit, ties,
// NaN and overflowing sums included.  Arithmetic follows the element type as c10 does: double in
// double, float in float, half with every difference, square and sum computed in float and
// rounded to half (c10::Half's operators).  Shared by the exact kernel (float64, float16, and
// float32 as a cross-check) and, for inputs holding NaN or inf, the float32 pruned pipeline.
#pragma once

#include "common.hpp"

#pragma clang fp contract(off)

namespace tpw {
namespace hdx {

// Element arithmetic of each dtype: load to the accumulation type, and round a result as the
// element type would hold it.
template <int DT>
struct HdT;
template <>
struct HdT<TPW_F64> {
    using S = double;
    using A = double;
    static __device__ __forceinline__ A ld(S v) { return v; }
    static __device__ __forceinline__ A rn(A v) { return v; }
    static __device__ __forceinline__ S st(A v) { return v; }
    static __device__ __forceinline__ A root(A v) { return sqrt(v); }
};
template <>
struct HdT<TPW_F32> {
    using S = float;
    using A = float;
    static __device__ __forceinline__ A ld(S v) { return v; }
    static __device__ __forceinline__ A rn(A v) { return v; }
    static __device__ __forceinline__ S st(A v) { return v; }
    static __device__ __forceinline__ A root(A v) { return sqrt_rn(v); }
};
template <>
struct HdT<TPW_F16> {
    using S = _Float16;
    using A = float;
    static __device__ __forceinline__ A ld(S v) { return (float)v; }
    static __device__ __forceinline__ A rn(A v) { return (float)(_Float16)v; }
    static __device__ __forceinline__ S st(A v) { return (_Float16)v; }
    static __device__ __forceinline__ A root(A v) { return sqrt_rn(v); }
};

template <typename A>
__device__ __forceinline__ A wave_min_ordered(A v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const A o = __shfl_xor(v, off, 64);
        v = o < v ? o : v;
    }
    return v;
}

// One pair by the calling wave: P, Q the pair's clouds ([p1][d], [p2][d]); perm1 / perm2 its
// batch's iteration orders (null: natural order).  Every lane returns best (the squared value)
// and the indices.
template <int DT>
__device__ void exact_pair(const typename HdT<DT>::S *__restrict__ P, const typename HdT<DT>::S *__restrict__ Q,
                           int64_t p1, int64_t p2, int64_t d, const int64_t *__restrict__ perm1,
                           const int64_t *__restrict__ perm2, typename HdT<DT>::A &best_out, int64_t &m_out,
                           int64_t &n_out) {
    using H = HdT<DT>;
    using A = typename H::A;
    const int lane = threadIdx.x & 63;
    const A inf = (A)INFINITY;
    A best = 0, s_last = 0;
    int64_t m_best = 0, n_best = 0, m_c = 0, n_c = 0;
    for (int64_t mp = 0; mp < p1; ++mp) {
        const int64_t mi = perm1 ? perm1[mp] : mp;
        const typename H::S *u = P + mi * d;
        A row_min = inf;
        for (int64_t base = 0; base < p2; base += 64) {
            const int64_t np = base + lane;
            const bool act = np < p2;
            const int64_t ni = act ? (perm2 ? perm2[np] : np) : 0;
            const typename H::S *v = Q + ni * d;
            A s = 0;
            for (int64_t k = 0; k < d; ++k) {
                const A diff = H::rn(H::ld(u[k]) - H::ld(v[k]));
                s = H::rn(s + H::rn(diff * diff));
            }
            const uint64_t brk = __ballot(act && s < best);
            const int nact = p2 - base < 64 ? (int)(p2 - base) : 64;
            const int limit = brk ? __builtin_ctzll(brk) : nact;
            // candidates: the lanes the loop reaches whose s improves on the row's minimum; the
            // chunk's smallest candidate, first lane on ties, is the loop's last strict update
            const bool cand = lane < limit && s < row_min;
            const A cmin = wave_min_ordered(cand ? s : inf);
            if (cmin < row_min) {
                const uint64_t hit = __ballot(cand && s == cmin);
                const int fl = __builtin_ctzll(hit);
                row_min = cmin;
                m_c = mi;
                n_c = __shfl(ni, fl, 64);
            }
            s_last = __shfl(s, brk ? limit : nact - 1, 64);
            if (brk) break;
        }
        if (row_min >= best && s_last >= best) {
            best = row_min;
            m_best = m_c;
            n_best = n_c;
        }
    }
    best_out = best;
    m_out = m_best;
    n_out = n_best;
}

}  // namespace hdx
}  // namespace tpw
