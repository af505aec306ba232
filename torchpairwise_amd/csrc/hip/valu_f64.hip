// float64 kernels of the reference's VALU metric family (_ppminkowski, _wminkowski, _canberra,
// _braycurtis, _additive_chi2_kernel, _sqjensenshannon) and of _haversine, forward and
// backward.  The reference serves double on the GPU for all of them
// (cuda/{ppminkowski,wminkowski,canberra,braycurtis,additive_chi2_kernel,sqjensenshannon,
// haversine}_kernel.cu dispatch AT_DISPATCH_FLOATING_TYPES_AND*).  float64 is not a hot-path
// dtype, so these kernels keep the reference's per-pair arithmetic rather than chase speed:
//
// * forward: 32 x 32 outputs per 256-thread block, the two operands' rows staged through LDS in
//   32-feature chunks, 2 x 2 outputs per thread, each output summed over k = 0..d-1 in order with
//   the reference CPU loop's per-term expression;
// * backward: one pass of per-pair factors (the wminkowski root factor S^(1/p-1), Bray-Curtis
//   1/ss and sd/ss^2, the first arg-extremum feature at p = +-inf), then grad_x1 as one thread per
//   (b, i, k) summing j = 0..m-1 in order and grad_x2 as one thread per (b, j, k) summing i in
//   order, as the CPU loops do; grad_w as per-(b, i, k) sums over j, then over i in order.
//   No atomics anywhere, so the gradients are deterministic.
//
// Floating-point contraction is off in this file: every product and sum is rounded as the CPU
// loops round it (the remaining differences are the last bits of pow / log / sin from the
// device's math library).
#include "common.hpp"

#include <math.h>

#pragma clang fp contract(off)

namespace tpw {
namespace {

constexpr int kT = 32;   // output tile edge (rows and columns)
constexpr int kKC = 32;  // features per LDS chunk

__device__ __forceinline__ double sgn64(double v) { return (double)((0.0 < v) - (v < 0.0)); }

// rel_entr of cpu/rel_entr.h
__device__ __forceinline__ double rel_entr64(double x, double y) {
    if (isnan(x)) return x;
    if (x > 0.0 && y > 0.0) return x * log(x / y);
    if (x == 0.0 && y >= 0.0) return 0.0;
    return INFINITY;
}

// One output's running state: `a` the sum (or the extremum), `c` Bray-Curtis's denominator.
struct Acc {
    double a, c;
};

// Adds feature k (global index gk) of the pair (u from x1, v from x2) to the output's state
// (cpu/{ppminkowski,wminkowski,canberra,braycurtis,additive_chi2,sqjensenshannon}_kernel.cpp
// forward loops).
template <int F>
__device__ __forceinline__ void fwd_term(Acc &s, double u, double v, double wk, int64_t gk, double p,
                                         bool inf, bool neg) {
    if constexpr (F == TPW_FAM_PPMINKOWSKI || F == TPW_FAM_WMINKOWSKI) {
        if (inf) {
            double t = fabs(u - v);
            if constexpr (F == TPW_FAM_WMINKOWSKI) t *= wk;
            if (gk == 0 || (neg ? t < s.a : t > s.a)) s.a = t;
        } else {
            double t = pow(fabs(u - v), p);
            if constexpr (F == TPW_FAM_WMINKOWSKI) t *= wk;
            s.a += t;
        }
    } else if constexpr (F == TPW_FAM_CANBERRA) {
        const double den = fabs(u) + fabs(v);
        if (den != 0.0) s.a += fabs(u - v) / den;
    } else if constexpr (F == TPW_FAM_CHI2) {
        const double nom = u + v;
        if (nom != 0.0) {
            const double den = u - v;
            s.a -= den * den / nom;
        }
    } else if constexpr (F == TPW_FAM_JS) {
        const double mid = (u + v) / 2.0;
        s.a += rel_entr64(u, mid) + rel_entr64(v, mid);
    } else {  // Bray-Curtis
        s.a += fabs(u - v);
        s.c += fabs(u + v);
    }
}

template <int F>
__device__ __forceinline__ double fwd_final(const Acc &s, double p, bool inf) {
    if constexpr (F == TPW_FAM_WMINKOWSKI) return inf ? s.a : pow(s.a, 1.0 / p);
    else if constexpr (F == TPW_FAM_JS) return s.a / p;
    else if constexpr (F == TPW_FAM_BRAYCURTIS) return s.a / s.c;
    else return s.a;
}

// out[b, i, j] for a 32 x 32 tile; thread (ty, tx) owns rows ty, ty + 16 and columns tx, tx + 16.
template <int F>
__global__ __launch_bounds__(256) void fam64_forward_kernel(const double *__restrict__ x1,
                                                            const double *__restrict__ x2,
                                                            const double *__restrict__ w, int64_t n,
                                                            int64_t m, int64_t d, double p,
                                                            double *__restrict__ out) {
    __shared__ double sa[kT][kKC + 1], sb[kT][kKC + 1], sw[kKC];
    const int64_t b = blockIdx.z, i0 = (int64_t)blockIdx.y * kT, j0 = (int64_t)blockIdx.x * kT;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const double *A = x1 + b * n * d, *Bm = x2 + b * m * d;
    const bool inf = isinf(p), neg = p < 0.0;
    Acc acc[2][2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[r][c] = Acc{0.0, 0.0};
    for (int64_t k0 = 0; k0 < d; k0 += kKC) {
        for (int e = threadIdx.x; e < kT * kKC; e += 256) {
            const int r = e / kKC, c = e % kKC;
            const int64_t gk = k0 + c, gi = i0 + r, gj = j0 + r;
            sa[r][c] = (gi < n && gk < d) ? A[gi * d + gk] : 0.0;
            sb[r][c] = (gj < m && gk < d) ? Bm[gj * d + gk] : 0.0;
        }
        if constexpr (F == TPW_FAM_WMINKOWSKI)
            if (threadIdx.x < kKC) sw[threadIdx.x] = k0 + threadIdx.x < d ? w[b * d + k0 + threadIdx.x] : 0.0;
        __syncthreads();
        const int kc = (int)(d - k0 < kKC ? d - k0 : kKC);
        for (int k = 0; k < kc; ++k) {
            const double wk = F == TPW_FAM_WMINKOWSKI ? sw[k] : 1.0;
            const double u0 = sa[ty][k], u1 = sa[ty + 16][k], v0 = sb[tx][k], v1 = sb[tx + 16][k];
            fwd_term<F>(acc[0][0], u0, v0, wk, k0 + k, p, inf, neg);
            fwd_term<F>(acc[0][1], u0, v1, wk, k0 + k, p, inf, neg);
            fwd_term<F>(acc[1][0], u1, v0, wk, k0 + k, p, inf, neg);
            fwd_term<F>(acc[1][1], u1, v1, wk, k0 + k, p, inf, neg);
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int64_t i = i0 + ty + 16 * r, j = j0 + tx + 16 * c;
            if (i < n && j < m) out[(b * n + i) * m + j] = fwd_final<F>(acc[r][c], p, inf);
        }
}

// Per-pair factors of the backward (cpu/*_kernel.cpp backward loops): f1 = S^(1/p - 1)
// (wminkowski), f1 = 1 / ss and f2 = sd / ss^2 (Bray-Curtis), kstar = the first feature reaching
// the max (min) of w |diff| at p = +-inf.
template <int F>
__global__ __launch_bounds__(256) void fam64_pair_kernel(const double *__restrict__ x1,
                                                         const double *__restrict__ x2,
                                                         const double *__restrict__ w, int64_t B,
                                                         int64_t n, int64_t m, int64_t d, double p,
                                                         double *__restrict__ f1,
                                                         double *__restrict__ f2,
                                                         int *__restrict__ kstar) {
    const int64_t at = blockIdx.x * (int64_t)256 + threadIdx.x;
    if (at >= B * n * m) return;
    const int64_t j = at % m, i = (at / m) % n, b = at / (n * m);
    const double *u = x1 + (b * n + i) * d, *v = x2 + (b * m + j) * d;
    const bool inf = isinf(p), neg = p < 0.0;
    if constexpr (F == TPW_FAM_PPMINKOWSKI || F == TPW_FAM_WMINKOWSKI) {
        if (inf) {
            double best = 0.0;
            int kb = 0;
            for (int64_t k = 0; k < d; ++k) {
                double t = fabs(u[k] - v[k]);
                if constexpr (F == TPW_FAM_WMINKOWSKI) t *= w[b * d + k];
                if (k == 0 || (neg ? t < best : t > best)) best = t, kb = (int)k;
            }
            kstar[at] = kb;
        } else if constexpr (F == TPW_FAM_WMINKOWSKI) {
            double s = 0.0;
            for (int64_t k = 0; k < d; ++k) s += pow(fabs(u[k] - v[k]), p) * w[b * d + k];
            f1[at] = pow(s, 1.0 / p - 1.0);
        }
    } else if constexpr (F == TPW_FAM_BRAYCURTIS) {
        double sd = 0.0, ss = 0.0;
        for (int64_t k = 0; k < d; ++k) {
            sd += fabs(u[k] - v[k]);
            ss += fabs(u[k] + v[k]);
        }
        f1[at] = 1.0 / ss;
        f2[at] = sd / ss / ss;
    }
}

// d(out)/d(x) for the pair (x, y), x the differentiated side's value (the same expression for
// both sides, as the reference's loops use it).
template <int F>
__device__ __forceinline__ double bwd_term(double x, double y, double wk, const double *f1,
                                           const double *f2, const int *kstar, int64_t at, int64_t k,
                                           double p, bool inf) {
    const double diff = x - y;
    if constexpr (F == TPW_FAM_PPMINKOWSKI || F == TPW_FAM_WMINKOWSKI) {
        if (inf) return k == kstar[at] ? wk * sgn64(diff) : 0.0;
        if constexpr (F == TPW_FAM_PPMINKOWSKI) return pow(fabs(diff), p - 1.0) * sgn64(diff) * p;
        else return pow(fabs(diff), p - 1.0) * sgn64(diff) * wk * f1[at];
    } else if constexpr (F == TPW_FAM_CANBERRA) {
        const double nom = fabs(x) + fabs(y);
        return sgn64(diff) / nom - sgn64(x) * fabs(diff) / nom / nom;
    } else if constexpr (F == TPW_FAM_CHI2) {
        const double nom = x + y;
        return nom != 0.0 ? diff * diff / (nom * nom) - 2.0 * diff / nom : 0.0;
    } else if constexpr (F == TPW_FAM_JS) {
        const double sum = x + y, mid = sum / 2.0;
        double t = 0.0;
        if (mid > 0.0) {
            if (x > 0.0) t += (y + sum * log(x / mid)) / sum;
            if (y > 0.0) t += -y / sum;
        }
        return t;
    } else {
        return sgn64(diff) * f1[at] - sgn64(x + y) * f2[at];
    }
}

// grad of side SIDE (0: x1, rows n, others m; 1: x2, rows m, others n): one thread per
// (b, row, k), the other side's rows summed in order.
template <int F, int SIDE>
__global__ __launch_bounds__(256) void fam64_grad_kernel(
    const double *__restrict__ g, const double *__restrict__ x1, const double *__restrict__ x2,
    const double *__restrict__ w, const double *__restrict__ f1, const double *__restrict__ f2,
    const int *__restrict__ kstar, int64_t B, int64_t n, int64_t m, int64_t d, double p,
    double *__restrict__ gout) {
    const int64_t rows = SIDE == 0 ? n : m, others = SIDE == 0 ? m : n;
    const int64_t t = blockIdx.x * (int64_t)256 + threadIdx.x;
    if (t >= B * rows * d) return;
    const int64_t k = t % d, r = (t / d) % rows, b = t / (d * rows);
    const double *X = SIDE == 0 ? x1 : x2, *Y = SIDE == 0 ? x2 : x1;
    const double x = X[t];
    const double wk = F == TPW_FAM_WMINKOWSKI ? w[b * d + k] : 1.0;
    const bool inf = isinf(p);
    double s = 0.0;
    for (int64_t o = 0; o < others; ++o) {
        const int64_t at = SIDE == 0 ? (b * n + r) * m + o : (b * n + o) * m + r;
        s += g[at] * bwd_term<F>(x, Y[(b * others + o) * d + k], wk, f1, f2, kstar, at, k, p, inf);
    }
    gout[t] = F == TPW_FAM_JS ? s / p : s;
}

// grad_w of wminkowski: part[b, i, k] = sum_j g * (|diff|^p / p * f1, or |diff| at kstar).
__global__ __launch_bounds__(256) void wmink64_wpart_kernel(
    const double *__restrict__ g, const double *__restrict__ x1, const double *__restrict__ x2,
    const double *__restrict__ f1, const int *__restrict__ kstar, int64_t B, int64_t n, int64_t m,
    int64_t d, double p, double *__restrict__ part) {
    const int64_t t = blockIdx.x * (int64_t)256 + threadIdx.x;
    if (t >= B * n * d) return;
    const int64_t k = t % d, i = (t / d) % n, b = t / (d * n);
    const double x = x1[t];
    const bool inf = isinf(p);
    double s = 0.0;
    for (int64_t j = 0; j < m; ++j) {
        const int64_t at = (b * n + i) * m + j;
        const double diff = x2[(b * m + j) * d + k] - x;
        if (inf) {
            if (k == kstar[at]) s += g[at] * fabs(diff);
        } else {
            s += g[at] * pow(fabs(diff), p) / p * f1[at];
        }
    }
    part[t] = s;
}

__global__ __launch_bounds__(256) void wmink64_wsum_kernel(const double *__restrict__ part, int64_t B,
                                                           int64_t n, int64_t d,
                                                           double *__restrict__ gw) {
    const int64_t t = blockIdx.x * (int64_t)256 + threadIdx.x;
    if (t >= B * d) return;
    const int64_t k = t % d, b = t / d;
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) s += part[(b * n + i) * d + k];
    gw[t] = s;
}

__global__ void fill64_kernel(double *__restrict__ p, int64_t len, double v) {
    const int64_t t = blockIdx.x * (int64_t)256 + threadIdx.x;
    if (t < len) p[t] = v;
}

int fill64(double *p, int64_t len, double v, hipStream_t s) {
    if (len <= 0) return TPW_OK;
    TPW_REQUIRE(p, "null pointer");
    hipLaunchKernelGGL(fill64_kernel, dim3((unsigned)cdiv(len, 256)), dim3(256), 0, s, p, len, v);
    return check_launch("fill64_kernel");
}

// ------------------------------------------------------------------ haversine
// out = 2 asin(sqrt(sa^2 + cos(la) cos(lb) so^2)) (cpu/haversine_kernel.cpp:13-27)
__global__ __launch_bounds__(256) void haversine64_kernel(const double *__restrict__ x1,
                                                          const double *__restrict__ x2, int64_t B,
                                                          int64_t n, int64_t m,
                                                          double *__restrict__ out) {
    const int64_t t = blockIdx.x * (int64_t)256 + threadIdx.x;
    if (t >= B * n * m) return;
    const int64_t j = t % m, i = (t / m) % n, b = t / (n * m);
    const double la = x1[2 * (b * n + i)], lo = x1[2 * (b * n + i) + 1];
    const double lb = x2[2 * (b * m + j)], lob = x2[2 * (b * m + j) + 1];
    const double sa = sin((la - lb) / 2.0), so = sin((lo - lob) / 2.0);
    out[t] = 2.0 * asin(sqrt(sa * sa + cos(la) * cos(lb) * so * so));
}

// per pair: g / (sqrt(val) sqrt(1 - val)) (cpu/haversine_kernel.cpp:88-93)
__device__ __forceinline__ double hav64_weight(double g, double la, double lo, double lb, double lob) {
    const double sa = sin((la - lb) / 2.0), so = sin((lo - lob) / 2.0);
    const double val = sa * sa + cos(la) * cos(lb) * so * so;
    return g / (sqrt(val) * sqrt(1.0 - val));
}

// grad of side SIDE: one thread per point, the other side's points in order
// (cpu/haversine_kernel.cpp:111-116 for x1, 138-143 for x2).
template <int SIDE>
__global__ __launch_bounds__(256) void haversine64_grad_kernel(const double *__restrict__ g,
                                                               const double *__restrict__ x1,
                                                               const double *__restrict__ x2,
                                                               int64_t B, int64_t n, int64_t m,
                                                               double *__restrict__ gout) {
    const int64_t rows = SIDE == 0 ? n : m, others = SIDE == 0 ? m : n;
    const int64_t r = blockIdx.x * (int64_t)256 + threadIdx.x;
    if (r >= B * rows) return;
    const int64_t b = r / rows, own = r % rows;
    const double *X = SIDE == 0 ? x1 : x2, *Y = SIDE == 0 ? x2 : x1;
    const double xa = X[2 * r], xo = X[2 * r + 1];
    double dlat = 0.0, dlon = 0.0;
    for (int64_t o = 0; o < others; ++o) {
        const double ya = Y[2 * (b * others + o)], yo = Y[2 * (b * others + o) + 1];
        const int64_t at = SIDE == 0 ? (b * n + own) * m + o : (b * n + o) * m + own;
        if constexpr (SIDE == 0) {
            const double wv = hav64_weight(g[at], xa, xo, ya, yo);
            const double so = sin((xo - yo) / 2.0);
            dlat += wv * (-sin(xa) * so * so * cos(ya) + sin(xa - ya) / 2.0);
            dlon += wv * (so * cos(xa) * cos(ya) * cos((xo - yo) / 2.0));
        } else {
            const double wv = hav64_weight(g[at], ya, yo, xa, xo);
            const double so = sin((yo - xo) / 2.0);
            dlat += wv * (-sin(xa) * so * so * cos(ya) - sin(ya - xa) / 2.0);
            dlon += wv * (-so * cos(ya) * cos(xa) * cos((yo - xo) / 2.0));
        }
    }
    gout[2 * r] = dlat;
    gout[2 * r + 1] = dlon;
}

// ------------------------------------------------------------------ host side
struct Layout64 {
    size_t f1, f2, kstar, part, total;
};

inline size_t round256(size_t v) { return (v + 255) & ~(size_t)255; }

Layout64 layout64(int metric, int64_t B, int64_t n, int64_t m, int64_t d, double p) {
    const size_t pairs = (size_t)(B * n * m);
    const bool mink = metric == TPW_FAM_PPMINKOWSKI || metric == TPW_FAM_WMINKOWSKI;
    const bool inf = isinf(p);
    Layout64 l{};
    l.f1 = (metric == TPW_FAM_WMINKOWSKI && !inf) || metric == TPW_FAM_BRAYCURTIS ? round256(8 * pairs) : 0;
    l.f2 = metric == TPW_FAM_BRAYCURTIS ? round256(8 * pairs) : 0;
    l.kstar = mink && inf ? round256(4 * pairs) : 0;
    l.part = metric == TPW_FAM_WMINKOWSKI ? round256(8 * (size_t)(B * n * d)) : 0;
    l.total = l.f1 + l.f2 + l.kstar + l.part + 256;
    return l;
}

inline unsigned blocks_of(int64_t len) { return (unsigned)cdiv(len, 256); }

template <int F>
int forward64(const double *x1, const double *x2, const double *w, int64_t B, int64_t n, int64_t m,
              int64_t d, double p, double *out, hipStream_t s) {
    hipLaunchKernelGGL(fam64_forward_kernel<F>, dim3((unsigned)cdiv(m, kT), (unsigned)cdiv(n, kT), (unsigned)B),
                       dim3(256), 0, s, x1, x2, w, n, m, d, p, out);
    return check_launch("fam64_forward_kernel");
}

template <int F>
int backward64(const double *g, const double *x1, const double *x2, const double *w, int64_t B,
               int64_t n, int64_t m, int64_t d, double p, double *gx1, double *gx2, double *gw,
               char *ws, hipStream_t s) {
    const Layout64 l = layout64(F, B, n, m, d, p);
    double *f1 = l.f1 ? reinterpret_cast<double *>(ws) : nullptr;
    double *f2 = l.f2 ? reinterpret_cast<double *>(ws + l.f1) : nullptr;
    int *kstar = l.kstar ? reinterpret_cast<int *>(ws + l.f1 + l.f2) : nullptr;
    double *part = l.part ? reinterpret_cast<double *>(ws + l.f1 + l.f2 + l.kstar) : nullptr;
    if (f1 || f2 || kstar) {
        hipLaunchKernelGGL(fam64_pair_kernel<F>, dim3(blocks_of(B * n * m)), dim3(256), 0, s, x1, x2, w, B, n,
                           m, d, p, f1, f2, kstar);
        const int rc = check_launch("fam64_pair_kernel");
        if (rc != TPW_OK) return rc;
    }
    hipLaunchKernelGGL((fam64_grad_kernel<F, 0>), dim3(blocks_of(B * n * d)), dim3(256), 0, s, g, x1, x2, w,
                       f1, f2, kstar, B, n, m, d, p, gx1);
    int rc = check_launch("fam64_grad_kernel");
    if (rc != TPW_OK) return rc;
    hipLaunchKernelGGL((fam64_grad_kernel<F, 1>), dim3(blocks_of(B * m * d)), dim3(256), 0, s, g, x1, x2, w,
                       f1, f2, kstar, B, n, m, d, p, gx2);
    rc = check_launch("fam64_grad_kernel");
    if (rc != TPW_OK || F != TPW_FAM_WMINKOWSKI) return rc;
    hipLaunchKernelGGL(wmink64_wpart_kernel, dim3(blocks_of(B * n * d)), dim3(256), 0, s, g, x1, x2, f1, kstar,
                       B, n, m, d, p, part);
    rc = check_launch("wmink64_wpart_kernel");
    if (rc != TPW_OK) return rc;
    hipLaunchKernelGGL(wmink64_wsum_kernel, dim3(blocks_of(B * d)), dim3(256), 0, s, part, B, n, d, gw);
    return check_launch("wmink64_wsum_kernel");
}

}  // namespace
}  // namespace tpw

using namespace tpw;

extern "C" int tpw_family_f64(int metric, const double *x1, const double *x2, const double *w,
                              int64_t batch, int64_t n, int64_t m, int64_t d, double p, double *out,
                              void *stream) {
    TPW_REQUIRE(metric >= TPW_FAM_PPMINKOWSKI && metric <= TPW_FAM_JS, "unknown metric %d", metric);
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    TPW_REQUIRE(cdiv(n, kT) <= kMaxGridYZ && batch <= kMaxGridYZ, "too many rows or batches");
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out && (metric != TPW_FAM_WMINKOWSKI || w), "null pointer");
    hipStream_t s = as_stream(stream);
    const bool mink = metric == TPW_FAM_PPMINKOWSKI || metric == TPW_FAM_WMINKOWSKI;
    if (mink && p == 0.0)  // ppminkowski_kernel.cpp:90-91, wminkowski_kernel.cpp:101-102
        return fill64(out, batch * n * m, (double)d, s);
    switch (metric) {
        case TPW_FAM_PPMINKOWSKI: return forward64<TPW_FAM_PPMINKOWSKI>(x1, x2, w, batch, n, m, d, p, out, s);
        case TPW_FAM_WMINKOWSKI: return forward64<TPW_FAM_WMINKOWSKI>(x1, x2, w, batch, n, m, d, p, out, s);
        case TPW_FAM_CANBERRA: return forward64<TPW_FAM_CANBERRA>(x1, x2, w, batch, n, m, d, p, out, s);
        case TPW_FAM_BRAYCURTIS: return forward64<TPW_FAM_BRAYCURTIS>(x1, x2, w, batch, n, m, d, p, out, s);
        case TPW_FAM_CHI2: return forward64<TPW_FAM_CHI2>(x1, x2, w, batch, n, m, d, p, out, s);
        default: return forward64<TPW_FAM_JS>(x1, x2, w, batch, n, m, d, p, out, s);
    }
}

extern "C" size_t tpw_family_f64_backward_workspace_size(int metric, int64_t batch, int64_t n, int64_t m,
                                                         int64_t d, double p) {
    return layout64(metric, batch, n, m, d, p).total;
}

extern "C" int tpw_family_f64_backward(int metric, const double *grad, const double *x1, const double *x2,
                                       const double *w, int64_t batch, int64_t n, int64_t m, int64_t d,
                                       double p, double *grad_x1, double *grad_x2, double *grad_w,
                                       void *workspace, void *stream) {
    TPW_REQUIRE(metric >= TPW_FAM_PPMINKOWSKI && metric <= TPW_FAM_JS, "unknown metric %d", metric);
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    TPW_REQUIRE(d < ((int64_t)1 << 31), "too many features");
    if (batch == 0 || d == 0) return TPW_OK;
    hipStream_t s = as_stream(stream);
    const bool wm = metric == TPW_FAM_WMINKOWSKI;
    const bool mink = metric == TPW_FAM_PPMINKOWSKI || wm;
    if ((mink && p == 0.0) || n == 0 || m == 0) {  // nothing to sum: zero gradients
        int rc = fill64(grad_x1, batch * n * d, 0.0, s);
        if (rc == TPW_OK) rc = fill64(grad_x2, batch * m * d, 0.0, s);
        if (rc == TPW_OK && wm) rc = fill64(grad_w, batch * d, 0.0, s);
        return rc;
    }
    TPW_REQUIRE(grad && x1 && x2 && grad_x1 && grad_x2 && (!wm || (w && grad_w)), "null pointer");
    const Layout64 l = layout64(metric, batch, n, m, d, p);
    TPW_REQUIRE(workspace, "workspace of %zu bytes required", l.total);
    char *ws = static_cast<char *>(workspace);
    switch (metric) {
        case TPW_FAM_PPMINKOWSKI:
            return backward64<TPW_FAM_PPMINKOWSKI>(grad, x1, x2, w, batch, n, m, d, p, grad_x1, grad_x2, grad_w, ws, s);
        case TPW_FAM_WMINKOWSKI:
            return backward64<TPW_FAM_WMINKOWSKI>(grad, x1, x2, w, batch, n, m, d, p, grad_x1, grad_x2, grad_w, ws, s);
        case TPW_FAM_CANBERRA:
            return backward64<TPW_FAM_CANBERRA>(grad, x1, x2, w, batch, n, m, d, p, grad_x1, grad_x2, grad_w, ws, s);
        case TPW_FAM_BRAYCURTIS:
            return backward64<TPW_FAM_BRAYCURTIS>(grad, x1, x2, w, batch, n, m, d, p, grad_x1, grad_x2, grad_w, ws, s);
        case TPW_FAM_CHI2:
            return backward64<TPW_FAM_CHI2>(grad, x1, x2, w, batch, n, m, d, p, grad_x1, grad_x2, grad_w, ws, s);
        default:
            return backward64<TPW_FAM_JS>(grad, x1, x2, w, batch, n, m, d, p, grad_x1, grad_x2, grad_w, ws, s);
    }
}

extern "C" int tpw_haversine_f64(const double *x1, const double *x2, int64_t batch, int64_t n, int64_t m,
                                 double *out, void *stream) {
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0, "invalid sizes");
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    hipLaunchKernelGGL(haversine64_kernel, dim3(blocks_of(batch * n * m)), dim3(256), 0, as_stream(stream), x1,
                       x2, batch, n, m, out);
    return check_launch("haversine64_kernel");
}

extern "C" int tpw_haversine_f64_backward(const double *grad, const double *x1, const double *x2,
                                          int64_t batch, int64_t n, int64_t m, double *grad_x1,
                                          double *grad_x2, void *stream) {
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0, "invalid sizes");
    if (batch == 0 || (n == 0 && m == 0)) return TPW_OK;
    hipStream_t s = as_stream(stream);
    if (n == 0 || m == 0) return fill64(n ? grad_x1 : grad_x2, 2 * batch * (n ? n : m), 0.0, s);
    TPW_REQUIRE(grad && x1 && x2 && grad_x1 && grad_x2, "null pointer");
    hipLaunchKernelGGL(haversine64_grad_kernel<0>, dim3(blocks_of(batch * n)), dim3(256), 0, s, grad, x1, x2,
                       batch, n, m, grad_x1);
    const int rc = check_launch("haversine64_grad_kernel");
    if (rc != TPW_OK) return rc;
    hipLaunchKernelGGL(haversine64_grad_kernel<1>, dim3(blocks_of(batch * m)), dim3(256), 0, s, grad, x1, x2,
                       batch, n, m, grad_x2);
    return check_launch("haversine64_grad_kernel");
}
