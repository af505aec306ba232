// CPU implementations of the custom internal ops, for CPU tensors (the reference runs these
// on the CPU too).  They keep the reference's arithmetic: float accumulators for the pairwise
// reductions (csrc/ops/cpu/pairwise_binary_kernels.cpp:28-49), the early-break max-min loop
// for Hausdorff (csrc/ops/cpu/hausdorff_kernel.cpp:12-100, 187-235), parallel over outputs
// with ATen's intra-op pool (the prf_div family is in prf_div.cpp).  GPU tensors never reach
// this file.
#include <ATen/Dispatch.h>
#include <ATen/Parallel.h>

#include <cmath>
#include <limits>

#include "tpw_common.h"

namespace tpw_ext {
namespace {

// ---------------------------------------------------------------- pairwise reductions
template <int OP, bool MEAN>
at::Tensor pw_reduce_cpu(const at::Tensor &x1, const at::Tensor &x2) {
    const bool unbatched = x1.dim() == 2;
    TORCH_CHECK(unbatched || x1.dim() == 3, "x1 must be 2-D (unbatched) or 3-D (batched) tensor.")
    TORCH_CHECK(unbatched || x2.dim() == 3, "x2 must be 2-D (unbatched) or 3-D (batched) tensor.")
    TORCH_CHECK(unbatched || x1.size(0) == x2.size(0), "batch_size of x1 and x2 do not match.")
    TORCH_CHECK(x1.size(-1) == x2.size(-1), "feature dimension of x1 and x2 do not match.")
    const auto common = at::result_type(x1, x2);
    pw_check_dispatch(OP, common, "pairwise_binary_reduction_forward_cpu");
    auto a = as3(x1.to(common)), b = as3(x2.to(common));
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options().dtype(at::kFloat));
    float *o = out.data_ptr<float>();
    AT_DISPATCH_ALL_TYPES_AND3(at::kBool, at::kHalf, at::kBFloat16, common, "pw_reduce_cpu", [&] {
        const scalar_t *A = a.data_ptr<scalar_t>();
        const scalar_t *Bp = b.data_ptr<scalar_t>();
        at::parallel_for(0, B * n * m, 256, [&](int64_t beg, int64_t end) {
            for (int64_t t = beg; t < end; ++t) {
                const int64_t j = t % m, i = (t / m) % n, bb = t / (n * m);
                const scalar_t *u = A + (bb * n + i) * d;
                const scalar_t *v = Bp + (bb * m + j) * d;
                float acc = 0.0f;
                for (int64_t k = 0; k < d; ++k) {
                    bool hit;
                    if constexpr (OP == TPW_BIT_AND) hit = (bool)u[k] && (bool)v[k];
                    else if constexpr (OP == TPW_BIT_OR) hit = (bool)u[k] || (bool)v[k];
                    else if constexpr (OP == TPW_BIT_XOR) hit = (bool)u[k] != (bool)v[k];
                    else if constexpr (OP == TPW_BIT_EQ) hit = u[k] == v[k];
                    else hit = u[k] != v[k];
                    acc += (float)hit;
                }
                if (MEAN) acc /= (float)d;
                o[t] = acc;
            }
        });
    });
    return unbatched ? out.squeeze(0) : out;
}

at::Tensor jaccard_cpu(const at::Tensor &x1, const at::Tensor &x2) {
    // pairwise_metrics.cpp:215-222: prf_div(pwxor_sum, pwor_sum) ("zero" mode)
    auto a = x1.to(at::kBool), b = x2.to(at::kBool);
    return prf_div_cpu(pw_reduce_cpu<TPW_BIT_XOR, false>(a, b), pw_reduce_cpu<TPW_BIT_OR, false>(a, b),
                       "zero");
}

// ---------------------------------------------------------------- Hausdorff
template <typename scalar_t>
void hausdorff_forward_loop(const scalar_t *x1, const scalar_t *x2, int64_t B, int64_t b1, int64_t p1,
                            int64_t b2, int64_t p2, int64_t d, const int64_t *perm1,
                            const int64_t *perm2, scalar_t *out, int64_t *idx1, int64_t *idx2) {
    at::parallel_for(0, B * b1 * b2, 1, [&](int64_t beg, int64_t end) {
        for (int64_t t = beg; t < end; ++t) {
            const int64_t j = t % b2, i = (t / b2) % b1, bb = t / (b1 * b2);
            const scalar_t *A = x1 + (bb * b1 + i) * p1 * d;
            const scalar_t *Bq = x2 + (bb * b2 + j) * p2 * d;
            scalar_t best = 0, row_min = 0, s = 0;
            int64_t m_best = 0, n_best = 0, m_c = 0, n_c = 0;
            for (int64_t mp = 0; mp < p1; ++mp) {
                const int64_t mi = perm1 ? perm1[bb * p1 + mp] : mp;
                row_min = std::numeric_limits<scalar_t>::infinity();
                for (int64_t np = 0; np < p2; ++np) {
                    const int64_t ni = perm2 ? perm2[bb * p2 + np] : np;
                    s = 0;
                    for (int64_t k = 0; k < d; ++k) {
                        const scalar_t diff = A[mi * d + k] - Bq[ni * d + k];
                        s += diff * diff;
                    }
                    if (s < best) break;
                    if (s < row_min) {
                        row_min = s;
                        m_c = mi;
                        n_c = ni;
                    }
                }
                if (row_min >= best && s >= best) {
                    best = row_min;
                    m_best = m_c;
                    n_best = n_c;
                }
            }
            out[t] = std::sqrt(best);
            idx1[t] = m_best;
            idx2[t] = n_best;
        }
    });
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> hausdorff_cpu_run(
    const at::Tensor &x1, const at::Tensor &x2, bool shuffle, c10::optional<at::Generator> gen) {
    check_hausdorff_shapes(x1, x2);
    auto a = x1.dim() == 3 ? x1.unsqueeze(0).contiguous() : x1.contiguous();
    auto b = x2.dim() == 3 ? x2.unsqueeze(0).contiguous() : x2.contiguous();
    const int64_t B = a.size(0), b1 = a.size(1), p1 = a.size(2), d = a.size(3);
    const int64_t b2 = b.size(1), p2 = b.size(2);
    auto out = at::empty({B, b1, b2}, a.options());
    auto i1 = at::empty({B, b1, b2}, a.options().dtype(at::kLong));
    auto i2 = at::empty({B, b1, b2}, a.options().dtype(at::kLong));
    at::Tensor perm1, perm2;
    if (shuffle) std::tie(perm1, perm2) = hausdorff_perms(B, p1, p2, a.options(), gen);
    AT_DISPATCH_FLOATING_TYPES_AND_HALF(a.scalar_type(), "_directed_hausdorff_forward_cpu", [&] {
        hausdorff_forward_loop<scalar_t>(a.data_ptr<scalar_t>(), b.data_ptr<scalar_t>(), B, b1, p1,
                                         b2, p2, d, shuffle ? perm1.data_ptr<int64_t>() : nullptr,
                                         shuffle ? perm2.data_ptr<int64_t>() : nullptr,
                                         out.data_ptr<scalar_t>(), i1.data_ptr<int64_t>(),
                                         i2.data_ptr<int64_t>());
    });
    return {a, b, out, i1, i2};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> directed_hausdorff_cpu(
    const at::Tensor &x1, const at::Tensor &x2, bool shuffle, c10::optional<at::Generator> gen) {
    auto r = hausdorff_cpu_run(x1, x2, shuffle, gen);
    auto out = std::get<2>(r), i1 = std::get<3>(r), i2 = std::get<4>(r);
    if (x1.dim() == 3) return {out.squeeze(0), i1.squeeze(0), i2.squeeze(0)};
    return {out, i1, i2};
}

std::tuple<at::Tensor, at::Tensor> directed_hausdorff_backward_cpu(
    const at::Tensor &grad, const at::Tensor &x1, const at::Tensor &x2, bool shuffle,
    c10::optional<at::Generator> gen) {
    auto r = hausdorff_cpu_run(x1, x2, shuffle, gen);
    auto a = std::get<0>(r), b = std::get<1>(r), out = std::get<2>(r);
    auto i1 = std::get<3>(r), i2 = std::get<4>(r);
    const int64_t B = a.size(0), b1 = a.size(1), p1 = a.size(2), d = a.size(3);
    const int64_t b2 = b.size(1), p2 = b.size(2);
    auto g = grad.to(a.scalar_type()).reshape({B, b1, b2}).contiguous();
    auto gx1 = at::zeros_like(a), gx2 = at::zeros_like(b);
    AT_DISPATCH_FLOATING_TYPES_AND_HALF(a.scalar_type(), "_directed_hausdorff_backward_cpu", [&] {
        const scalar_t *X1 = a.data_ptr<scalar_t>(), *X2 = b.data_ptr<scalar_t>();
        const scalar_t *G = g.data_ptr<scalar_t>(), *O = out.data_ptr<scalar_t>();
        const int64_t *M = i1.data_ptr<int64_t>(), *N = i2.data_ptr<int64_t>();
        scalar_t *GX1 = gx1.data_ptr<scalar_t>(), *GX2 = gx2.data_ptr<scalar_t>();
        at::parallel_for(0, B * b1 * d, 1, [&](int64_t beg, int64_t end) {
            for (int64_t t = beg; t < end; ++t) {
                const int64_t k = t % d, i = (t / d) % b1, bb = t / (d * b1);
                for (int64_t j = 0; j < b2; ++j) {
                    const int64_t pr = (bb * b1 + i) * b2 + j;
                    const scalar_t diff = X1[((bb * b1 + i) * p1 + M[pr]) * d + k] -
                                          X2[((bb * b2 + j) * p2 + N[pr]) * d + k];
                    GX1[((bb * b1 + i) * p1 + M[pr]) * d + k] += G[pr] * diff / O[pr];
                }
            }
        });
        at::parallel_for(0, B * b2 * d, 1, [&](int64_t beg, int64_t end) {
            for (int64_t t = beg; t < end; ++t) {
                const int64_t k = t % d, j = (t / d) % b2, bb = t / (d * b2);
                for (int64_t i = 0; i < b1; ++i) {
                    const int64_t pr = (bb * b1 + i) * b2 + j;
                    const scalar_t diff = X2[((bb * b2 + j) * p2 + N[pr]) * d + k] -
                                          X1[((bb * b1 + i) * p1 + M[pr]) * d + k];
                    GX2[((bb * b2 + j) * p2 + N[pr]) * d + k] += G[pr] * diff / O[pr];
                }
            }
        });
    });
    if (x1.dim() == 3) return {gx1.squeeze(0), gx2.squeeze(0)};
    return {gx1, gx2};
}

}  // namespace

// Bool mask of each row's `count` smallest entries: the first `count` positions of a stable
// ascending argsort (NaN last), the order the HIP kernel implements.
at::Tensor row_smallest_mask_cpu(const at::Tensor &dist, int64_t count) {
    TORCH_CHECK(dist.dim() == 2, "_row_smallest_mask: expected a 2-D tensor");
    TORCH_CHECK(count >= 0, "_row_smallest_mask: count must be non-negative, got ", count);
    auto mask = at::zeros(dist.sizes(), dist.options().dtype(at::kBool));
    const int64_t c = std::min(count, dist.size(1));
    if (dist.numel() == 0 || c == 0) return mask;
    auto inds = at::argsort(dist, /*stable=*/true, /*dim=*/1, /*descending=*/false).slice(1, 0, c);
    mask.scatter_(1, inds, true);
    return mask;
}

namespace {

// out[b, i, j, k] = op(x1[b, i, k], x2[b, j, k]) (cpu/pairwise_binary_kernels.cpp:12-26),
// parallel over (b, i) rows.
template <int OP, typename T>
bool pw_apply(T x, T y) {
    if constexpr (OP == TPW_BIT_AND || OP == TPW_BIT_OR || OP == TPW_BIT_XOR) {
        const bool p = static_cast<bool>(x), q = static_cast<bool>(y);
        return OP == TPW_BIT_AND ? (p && q) : OP == TPW_BIT_OR ? (p || q) : (p != q);
    } else if constexpr (OP == TPW_BIT_EQ) {
        return x == y;
    } else if constexpr (OP == TPW_BIT_NE) {
        return x != y;
    } else if constexpr (OP == TPW_CMP_LT) {
        return x < y;
    } else if constexpr (OP == TPW_CMP_GT) {
        return x > y;
    } else if constexpr (OP == TPW_CMP_LE) {
        return x <= y;
    } else {
        return x >= y;
    }
}

template <int OP>
at::Tensor pw_binary_cpu(const at::Tensor &x1, const at::Tensor &x2) {
    auto r = pw_binary_prepare(OP, x1, x2, "pairwise_binary_forward_cpu");
    const int64_t B = r.a.size(0), n = r.a.size(1), m = r.b.size(1), d = r.a.size(2);
    auto out = at::empty({B, n, m, d}, r.a.options().dtype(at::kBool));
    bool *O = out.data_ptr<bool>();
    AT_DISPATCH_ALL_TYPES_AND3(at::kHalf, at::kBFloat16, at::kBool, r.a.scalar_type(), "pw_binary_cpu", [&] {
        const scalar_t *A = r.a.data_ptr<scalar_t>(), *Bp = r.b.data_ptr<scalar_t>();
        at::parallel_for(0, B * n, 1, [&](int64_t lo, int64_t hi) {
            for (int64_t bi = lo; bi < hi; ++bi) {
                const int64_t b = bi / n;
                for (int64_t j = 0; j < m; ++j)
                    for (int64_t k = 0; k < d; ++k)
                        O[(bi * m + j) * d + k] = pw_apply<OP, scalar_t>(A[bi * d + k], Bp[(b * m + j) * d + k]);
            }
        });
    });
    return out.view(r.out_shape);
}

}  // namespace

TORCH_LIBRARY_IMPL(torchpairwise, CPU, m) {
    m.impl("pwand", TORCH_FN(pw_binary_cpu<TPW_BIT_AND>));
    m.impl("pwor", TORCH_FN(pw_binary_cpu<TPW_BIT_OR>));
    m.impl("pwxor", TORCH_FN(pw_binary_cpu<TPW_BIT_XOR>));
    m.impl("pweq", TORCH_FN(pw_binary_cpu<TPW_BIT_EQ>));
    m.impl("pwne", TORCH_FN(pw_binary_cpu<TPW_BIT_NE>));
    m.impl("pwlt", TORCH_FN(pw_binary_cpu<TPW_CMP_LT>));
    m.impl("pwgt", TORCH_FN(pw_binary_cpu<TPW_CMP_GT>));
    m.impl("pwle", TORCH_FN(pw_binary_cpu<TPW_CMP_LE>));
    m.impl("pwge", TORCH_FN(pw_binary_cpu<TPW_CMP_GE>));
    m.impl("pwand_sum", TORCH_FN((pw_reduce_cpu<TPW_BIT_AND, false>)));
    m.impl("pwor_sum", TORCH_FN((pw_reduce_cpu<TPW_BIT_OR, false>)));
    m.impl("pwxor_sum", TORCH_FN((pw_reduce_cpu<TPW_BIT_XOR, false>)));
    m.impl("pweq_sum", TORCH_FN((pw_reduce_cpu<TPW_BIT_EQ, false>)));
    m.impl("pwne_sum", TORCH_FN((pw_reduce_cpu<TPW_BIT_NE, false>)));
    m.impl("pweq_mean", TORCH_FN((pw_reduce_cpu<TPW_BIT_EQ, true>)));
    m.impl("pwne_mean", TORCH_FN((pw_reduce_cpu<TPW_BIT_NE, true>)));
    m.impl("_jaccard", TORCH_FN(jaccard_cpu));
    m.impl("_row_smallest_mask", TORCH_FN(row_smallest_mask_cpu));
    m.impl("_directed_hausdorff", TORCH_FN(directed_hausdorff_cpu));
    m.impl("__directed_hausdorff_backward", TORCH_FN(directed_hausdorff_backward_cpu));
}

}  // namespace tpw_ext
