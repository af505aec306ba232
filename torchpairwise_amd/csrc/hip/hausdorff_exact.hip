// Directed Hausdorff distance for float64 and float16 (and float32, where it cross-checks the
// pruned cell-grid pipeline of hausdorff.hip): the reference's loop
// (cpu/hausdorff_kernel.cpp:12-100, cuda/hausdorff_kernel.cu:16-105) executed in its own order,
// one wave per cloud pair (exact_pair, hausdorff_exact.hpp).
//
// The backward follows the CPU loop too (cpu/hausdorff_kernel.cpp:187-235): one thread per
// (cloud, k) owns that feature column of its cloud's gradient and adds g * diff / out for every
// cloud pair in order, so there are no atomics and the sums are the loop's.
#include "hausdorff_exact.hpp"

#include <math.h>

#pragma clang fp contract(off)

namespace tpw {
namespace {

using hdx::HdT;

template <int DT>
__global__ __launch_bounds__(256) void hd_exact_kernel(
    const typename HdT<DT>::S *__restrict__ x1, const typename HdT<DT>::S *__restrict__ x2, int64_t pairs,
    int64_t b1, int64_t p1, int64_t b2, int64_t p2, int64_t d, const int64_t *__restrict__ perm1,
    const int64_t *__restrict__ perm2, typename HdT<DT>::S *__restrict__ out, int64_t *__restrict__ idx1,
    int64_t *__restrict__ idx2) {
    using H = HdT<DT>;
    const int64_t pair = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (pair >= pairs) return;  // the whole wave leaves together
    const int64_t j = pair % b2, i = (pair / b2) % b1, bb = pair / (b1 * b2);
    typename H::A best;
    int64_t m_best, n_best;
    hdx::exact_pair<DT>(x1 + (bb * b1 + i) * p1 * d, x2 + (bb * b2 + j) * p2 * d, p1, p2, d,
                        perm1 ? perm1 + bb * p1 : nullptr, perm2 ? perm2 + bb * p2 : nullptr, best, m_best, n_best);
    if (lane == 0) {
        out[pair] = H::st(H::root(best));
        idx1[pair] = m_best;
        idx2[pair] = n_best;
    }
}

template <typename S>
__global__ void hd_zero_kernel(S *__restrict__ p, int64_t len) {
    const int64_t t = blockIdx.x * (int64_t)256 + threadIdx.x;
    if (t < len) p[t] = (S)0;
}

// SIDE 0: thread (bb, i, k) adds g * (x1[m] - x2[n]) / out into grad_x1[bb, i, m, k] for every
// j in order; SIDE 1: thread (bb, j, k) adds g * (x2[n] - x1[m]) / out into grad_x2 for every i.
template <int DT, int SIDE>
__global__ __launch_bounds__(256) void hd_exact_grad_kernel(
    const typename HdT<DT>::S *__restrict__ g, const typename HdT<DT>::S *__restrict__ x1,
    const typename HdT<DT>::S *__restrict__ x2, const typename HdT<DT>::S *__restrict__ out,
    const int64_t *__restrict__ idx1, const int64_t *__restrict__ idx2, int64_t B, int64_t b1, int64_t p1,
    int64_t b2, int64_t p2, int64_t d, typename HdT<DT>::S *__restrict__ gout) {
    using H = HdT<DT>;
    using A = typename H::A;
    const int64_t clouds = SIDE == 0 ? b1 : b2, others = SIDE == 0 ? b2 : b1;
    const int64_t t = blockIdx.x * (int64_t)256 + threadIdx.x;
    if (t >= B * clouds * d) return;
    const int64_t k = t % d, c = (t / d) % clouds, bb = t / (d * clouds);
    for (int64_t o = 0; o < others; ++o) {
        const int64_t pr = SIDE == 0 ? (bb * b1 + c) * b2 + o : (bb * b1 + o) * b2 + c;
        const int64_t a1 = ((bb * b1 + (SIDE == 0 ? c : o)) * p1 + idx1[pr]) * d + k;
        const int64_t a2 = ((bb * b2 + (SIDE == 0 ? o : c)) * p2 + idx2[pr]) * d + k;
        const A diff = SIDE == 0 ? H::rn(H::ld(x1[a1]) - H::ld(x2[a2])) : H::rn(H::ld(x2[a2]) - H::ld(x1[a1]));
        const A q = H::rn(H::rn(H::ld(g[pr]) * diff) / H::ld(out[pr]));
        const int64_t at = SIDE == 0 ? a1 : a2;
        gout[at] = H::st(H::ld(gout[at]) + q);
    }
}

inline unsigned nblocks(int64_t len) { return (unsigned)cdiv(len, 256); }

template <int DT>
int launch_exact(const void *x1, const void *x2, int64_t B, int64_t b1, int64_t p1, int64_t b2, int64_t p2,
                 int64_t d, const int64_t *perm1, const int64_t *perm2, void *out, int64_t *idx1, int64_t *idx2,
                 hipStream_t s) {
    using S = typename HdT<DT>::S;
    const int64_t pairs = B * b1 * b2;
    hipLaunchKernelGGL(hd_exact_kernel<DT>, dim3((unsigned)cdiv(pairs, 4)), dim3(256), 0, s,
                       static_cast<const S *>(x1), static_cast<const S *>(x2), pairs, b1, p1, b2, p2, d, perm1,
                       perm2, static_cast<S *>(out), idx1, idx2);
    return check_launch("hd_exact_kernel");
}

template <int DT>
int launch_exact_backward(const void *g, const void *x1, const void *x2, const void *out, const int64_t *idx1,
                          const int64_t *idx2, int64_t B, int64_t b1, int64_t p1, int64_t b2, int64_t p2,
                          int64_t d, void *gx1, void *gx2, hipStream_t s) {
    using S = typename HdT<DT>::S;
    const int64_t n1 = B * b1 * p1 * d, n2 = B * b2 * p2 * d;
    if (n1 > 0) {
        hipLaunchKernelGGL(hd_zero_kernel<S>, dim3(nblocks(n1)), dim3(256), 0, s, static_cast<S *>(gx1), n1);
        const int rc = check_launch("hd_zero_kernel");
        if (rc != TPW_OK) return rc;
    }
    if (n2 > 0) {
        hipLaunchKernelGGL(hd_zero_kernel<S>, dim3(nblocks(n2)), dim3(256), 0, s, static_cast<S *>(gx2), n2);
        const int rc = check_launch("hd_zero_kernel");
        if (rc != TPW_OK) return rc;
    }
    if (B * b1 * b2 == 0 || p1 == 0 || p2 == 0 || d == 0) return TPW_OK;
    const S *G = static_cast<const S *>(g), *X1 = static_cast<const S *>(x1), *X2 = static_cast<const S *>(x2);
    const S *O = static_cast<const S *>(out);
    hipLaunchKernelGGL((hd_exact_grad_kernel<DT, 0>), dim3(nblocks(B * b1 * d)), dim3(256), 0, s, G, X1, X2, O,
                       idx1, idx2, B, b1, p1, b2, p2, d, static_cast<S *>(gx1));
    const int rc = check_launch("hd_exact_grad_kernel");
    if (rc != TPW_OK) return rc;
    hipLaunchKernelGGL((hd_exact_grad_kernel<DT, 1>), dim3(nblocks(B * b2 * d)), dim3(256), 0, s, G, X1, X2, O,
                       idx1, idx2, B, b1, p1, b2, p2, d, static_cast<S *>(gx2));
    return check_launch("hd_exact_grad_kernel");
}

}  // namespace
}  // namespace tpw

using namespace tpw;

extern "C" int tpw_directed_hausdorff_exact(int dtype, const void *x1, const void *x2, int64_t batch,
                                            int64_t b1, int64_t p1, int64_t b2, int64_t p2, int64_t d,
                                            const int64_t *perm1, const int64_t *perm2, void *out,
                                            int64_t *idx1, int64_t *idx2, void *stream) {
    TPW_REQUIRE(dtype == TPW_F64 || dtype == TPW_F32 || dtype == TPW_F16, "unsupported dtype %d", dtype);
    TPW_REQUIRE(batch >= 0 && b1 >= 0 && p1 >= 0 && b2 >= 0 && p2 >= 0 && d >= 0, "invalid sizes");
    const int64_t pairs = batch * b1 * b2;
    if (pairs == 0) return TPW_OK;
    TPW_REQUIRE(cdiv(pairs, 4) <= 0x7fffffffLL, "too many cloud pairs");
    TPW_REQUIRE(x1 && x2 && out && idx1 && idx2, "null pointer");
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case TPW_F64: return launch_exact<TPW_F64>(x1, x2, batch, b1, p1, b2, p2, d, perm1, perm2, out, idx1, idx2, s);
        case TPW_F32: return launch_exact<TPW_F32>(x1, x2, batch, b1, p1, b2, p2, d, perm1, perm2, out, idx1, idx2, s);
        default: return launch_exact<TPW_F16>(x1, x2, batch, b1, p1, b2, p2, d, perm1, perm2, out, idx1, idx2, s);
    }
}

extern "C" int tpw_directed_hausdorff_exact_backward(int dtype, const void *grad, const void *x1,
                                                     const void *x2, const void *out, const int64_t *idx1,
                                                     const int64_t *idx2, int64_t batch, int64_t b1,
                                                     int64_t p1, int64_t b2, int64_t p2, int64_t d,
                                                     void *grad_x1, void *grad_x2, void *stream) {
    TPW_REQUIRE(dtype == TPW_F64 || dtype == TPW_F32 || dtype == TPW_F16, "unsupported dtype %d", dtype);
    TPW_REQUIRE(batch >= 0 && b1 >= 0 && p1 >= 0 && b2 >= 0 && p2 >= 0 && d >= 0, "invalid sizes");
    const int64_t n1 = batch * b1 * p1 * d, n2 = batch * b2 * p2 * d;
    if (n1 == 0 && n2 == 0) return TPW_OK;
    TPW_REQUIRE((n1 == 0 || grad_x1) && (n2 == 0 || grad_x2), "null pointer");
    if (batch * b1 * b2 > 0 && p1 > 0 && p2 > 0 && d > 0)
        TPW_REQUIRE(grad && x1 && x2 && out && idx1 && idx2, "null pointer");
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case TPW_F64:
            return launch_exact_backward<TPW_F64>(grad, x1, x2, out, idx1, idx2, batch, b1, p1, b2, p2, d,
                                                  grad_x1, grad_x2, s);
        case TPW_F32:
            return launch_exact_backward<TPW_F32>(grad, x1, x2, out, idx1, idx2, batch, b1, p1, b2, p2, d,
                                                  grad_x1, grad_x2, s);
        default:
            return launch_exact_backward<TPW_F16>(grad, x1, x2, out, idx1, idx2, batch, b1, p1, b2, p2, d,
                                                  grad_x1, grad_x2, s);
    }
}
