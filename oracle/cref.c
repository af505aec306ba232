/*
 * C restatement of the reference's CPU loops — TEST INFRASTRUCTURE ONLY (the checker and
 * the timed CPU baseline; the product never calls it).
 *
 *  - oracle_directed_hausdorff: the sequential early-break max-min loop of
 *    _directed_hausdorff_forward_kernel_impl / _shuffled_ (csrc/ops/cpu/hausdorff_kernel.cpp:
 *    12-53, 55-100), one (b, i, j) per OpenMP iteration.
 *  - oracle_bool_reduce: the one-output-per-iteration loop of
 *    pairwise_binary_reduction_forward_kernel_impl (csrc/ops/cpu/pairwise_binary_kernels.cpp:
 *    28-49) on bool bytes, float accumulator, Mean divides by float(d).
 *  - oracle_jaccard: jaccard_distances as the reference runs it — pwxor_sum pass, pwor_sum
 *    pass, then prf_div(.., .., "zero") (csrc/ops/pairwise_metrics.cpp:215-222).
 *
 * Built with -O2 -ffp-contract=off (the reference's x86-64 build has no -march, so no FMA).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

void oracle_directed_hausdorff(const float *x1, const float *x2, int64_t batch, int64_t b1,
                               int64_t p1, int64_t b2, int64_t p2, int64_t d,
                               const int64_t *perm1, const int64_t *perm2, float *out,
                               int64_t *idx1, int64_t *idx2, int threads) {
    const int64_t total = batch * b1 * b2;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (int64_t t = 0; t < total; ++t) {
        const int64_t j = t % b2, i = (t / b2) % b1, b = t / (b1 * b2);
        const float *A = x1 + (b * b1 + i) * p1 * d;
        const float *Bp = x2 + (b * b2 + j) * p2 * d;
        float best_max = 0.0f, row_min = 0.0f, s = 0.0f;
        int64_t m_best = 0, n_best = 0, m_cand = 0, n_cand = 0;
        for (int64_t mpos = 0; mpos < p1; ++mpos) {
            const int64_t m = perm1 ? perm1[b * p1 + mpos] : mpos;
            row_min = INFINITY;
            for (int64_t npos = 0; npos < p2; ++npos) {
                const int64_t n = perm2 ? perm2[b * p2 + npos] : npos;
                s = 0.0f;
                for (int64_t k = 0; k < d; ++k) {
                    const float diff = A[m * d + k] - Bp[n * d + k];
                    s += diff * diff;
                }
                if (s < best_max) break;
                if (s < row_min) {
                    row_min = s;
                    m_cand = m;
                    n_cand = n;
                }
            }
            if (row_min >= best_max && s >= best_max) {
                best_max = row_min;
                m_best = m_cand;
                n_best = n_cand;
            }
        }
        out[t] = sqrtf(best_max);
        idx1[t] = m_best;
        idx2[t] = n_best;
    }
}

/* op: 0 and, 1 or, 2 xor, 3 eq, 4 ne; mean != 0 divides by float(d) */
void oracle_bool_reduce(const uint8_t *x1, const uint8_t *x2, int64_t batch, int64_t n,
                        int64_t m, int64_t d, int op, int mean, float *out, int threads) {
    const int64_t total = batch * n * m;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t t = 0; t < total; ++t) {
        const int64_t j = t % m, i = (t / m) % n, b = t / (n * m);
        const uint8_t *a = x1 + (b * n + i) * d;
        const uint8_t *c = x2 + (b * m + j) * d;
        float acc = 0.0f;
        for (int64_t k = 0; k < d; ++k) {
            const int u = a[k] != 0, v = c[k] != 0;
            int r;
            switch (op) {
                case 0: r = u & v; break;
                case 1: r = u | v; break;
                case 2: r = u ^ v; break;
                case 3: r = u == v; break;
                default: r = u != v; break;
            }
            acc += (float)r;
        }
        if (mean) acc /= (float)d;
        out[t] = acc;
    }
}

void oracle_jaccard(const uint8_t *x1, const uint8_t *x2, int64_t batch, int64_t n, int64_t m,
                    int64_t d, float *out, float *scratch, int threads) {
    oracle_bool_reduce(x1, x2, batch, n, m, d, 2, 0, out, threads);
    oracle_bool_reduce(x1, x2, batch, n, m, d, 1, 0, scratch, threads);
    const int64_t total = batch * n * m;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t t = 0; t < total; ++t) out[t] = scratch[t] != 0.0f ? out[t] / scratch[t] : 0.0f;
}
