// Schema registration of torch.ops.torchpairwise and the public (CompositeImplicitAutograd)
// metric functions.
//
// Public schemas are byte-for-byte those of the reference (csrc/ops/pairwise_metrics.h:76-424,
// registered at csrc/ops/pairwise_metrics.cpp:440-486), so torchpairwise.*_distances callers
// and torch.jit.script code bind unchanged.  Their bodies restate the reference functors:
// the same input checks (check_pairwise_inputs, pairwise_metrics.h:10-67) and formulas, but
// GPU tensors of the hot-path dtypes go to this build's internal ops (HIP kernels behind the
// C ABI) where the reference went to ATen (at::cdist / matmul + prf_div) or to its naive
// kernels.  CPU tensors take the reference's own route (ATen for the cdist/matmul metrics,
// this extension's CPU kernels for the custom ops).
#include "tpw_common.h"

#include <ATen/core/dispatch/Dispatcher.h>
#include <c10/util/Logging.h>

namespace tpw_ext {
namespace {

// ------------------------------------------------------------------------------------
// input checks (restated from csrc/ops/pairwise_metrics.h:10-67)
// ------------------------------------------------------------------------------------
template <bool is_boolean_metric = false, bool is_2d_metric = false>
std::pair<at::Tensor, at::Tensor> check_pairwise_inputs(const char *c, const at::Tensor &x1,
                                                        const c10::optional<at::Tensor> &x2) {
    const bool unbatched = x1.dim() == (is_2d_metric ? 3 : 2);
    if constexpr (is_2d_metric) {
        TORCH_CHECK(unbatched || x1.dim() == 4, "x1 must be 3D tensor (unbatched) or 4D tensor (batched)")
    } else {
        TORCH_CHECK(unbatched || x1.dim() == 3, "x1 must be 2D tensor (unbatched) or 3D tensor (batched)")
    }
    if (x2.has_value()) {
        const at::Tensor &y = x2.value();
        const int64_t f = (is_2d_metric ? 2 : 1) + (unbatched ? 0 : 1);
        if constexpr (is_2d_metric) {
            TORCH_CHECK(unbatched || y.dim() == 4, "x2 must be 3D tensor (unbatched) or 4D tensor (batched)")
        } else {
            TORCH_CHECK(unbatched || y.dim() == 3, "x2 must be 2D tensor (unbatched) or 3D tensor (batched)")
        }
        TORCH_CHECK(x1.size(f) == y.size(f), "x1 and x2 must have same number of features. Got: x1.size(",
                    f, ")=", x1.size(f), ", x2.size(", f, ")=", y.size(f))
        if constexpr (is_boolean_metric) {
            if (x1.scalar_type() != at::kBool || y.scalar_type() != at::kBool) {
                TORCH_WARN("Data was converted to ", at::kBool, " for metric ", c)
            }
            return {x1.to(at::kBool), y.to(at::kBool)};
        } else {
            return {x1, y};
        }
    }
    if constexpr (is_boolean_metric) {
        if (x1.scalar_type() != at::kBool) {
            TORCH_WARN("Data was converted to ", at::kBool, " for metric ", c)
        }
        auto b = x1.to(at::kBool);
        return {b, b};
    } else {
        return {x1, x1};
    }
}

bool hip_float_path(const at::Tensor &a, const at::Tensor &b) {
    return a.is_cuda() && b.is_cuda() && a.scalar_type() == b.scalar_type() &&
           (a.scalar_type() == at::kFloat || a.scalar_type() == at::kBFloat16) &&
           a.dim() == b.dim() && (a.dim() == 2 || a.dim() == 3);
}

// at::cdist broadcasts the batch dimension; the kernels take equal batches.
std::pair<at::Tensor, at::Tensor> broadcast_batch(const at::Tensor &a, const at::Tensor &b) {
    if (a.dim() != 3 || a.size(0) == b.size(0)) return {a, b};
    const int64_t B = std::max(a.size(0), b.size(0));
    TORCH_CHECK(a.size(0) == 1 || b.size(0) == 1, "The size of tensor a (", a.size(0),
                ") must match the size of tensor b (", b.size(0), ") at non-singleton dimension 0");
    return {a.expand({B, a.size(1), a.size(2)}), b.expand({B, b.size(1), b.size(2)})};
}

// at::cdist(x1, x2, p) with the same dispatch rule (p == 2 uses the |a|^2 + |b|^2 - 2ab
// matrix-product form when either operand has more than 25 rows, the direct sum otherwise;
// torch/functional.py documents the rule), served by the HIP kernels for fp32 / bf16 GPU
// tensors.  Anything else is at::cdist itself, as in the reference.
at::Tensor route_cdist(const at::Tensor &x1, const at::Tensor &x2, double p) {
    if (!hip_float_path(x1, x2)) return at::cdist(x1, x2, p);
    TORCH_CHECK(p >= 0, "cdist only supports non-negative p values");
    auto ab = broadcast_batch(x1, x2);
    const at::Tensor &a = ab.first, &b = ab.second;
    if (p == 2.0 && (a.size(-2) > 25 || b.size(-2) > 25)) return pw_inner(a, b, kEuclidean);
    if (a.scalar_type() == at::kBFloat16) {
        // without a gradient to form, the kernel writes the bf16 output itself (one pass over
        // the N x M output instead of a float32 matrix written, read back and converted)
        if (!(at::GradMode::is_enabled() && (a.requires_grad() || b.requires_grad())))
            return lp_distances_bf16_cuda(a.to(at::kFloat), b.to(at::kFloat), p);
        return pw_lp(a.to(at::kFloat), b.to(at::kFloat), p).to(at::kBFloat16);
    }
    return pw_lp(a, b, p);
}


// Public metric schemas, byte-for-byte those of csrc/ops/pairwise_metrics.h:76-424 (also quoted
// by cdist's incompatible-argument error, as the reference quotes its functors' schema_str).
struct PublicSchema {
    const char *name;
    const char *schema;
};
constexpr PublicSchema kPublicSchemas[] = {
    {"euclidean_distances", "euclidean_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"haversine_distances", "haversine_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"manhattan_distances", "manhattan_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"cosine_distances", "cosine_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"linear_kernel", "linear_kernel(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"polynomial_kernel", "polynomial_kernel(Tensor x1, Tensor? x2=None, int degree=3, float? gamma=None, float coef0=1) -> Tensor"},
    {"sigmoid_kernel", "sigmoid_kernel(Tensor x1, Tensor? x2=None, float? gamma=None, float coef0=1) -> Tensor"},
    {"rbf_kernel", "rbf_kernel(Tensor x1, Tensor? x2=None, float? gamma=None) -> Tensor"},
    {"laplacian_kernel", "laplacian_kernel(Tensor x1, Tensor? x2=None, float? gamma=None) -> Tensor"},
    {"cosine_similarity", "cosine_similarity(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"additive_chi2_kernel", "additive_chi2_kernel(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"chi2_kernel", "chi2_kernel(Tensor x1, Tensor? x2=None, float gamma=1.0) -> Tensor"},
    {"directed_hausdorff_distances", "directed_hausdorff_distances(Tensor x1, Tensor? x2=None, *, bool shuffle=False, Generator? generator=None) -> (Tensor output, Tensor x1_indices, Tensor x2_indices)"},
    {"minkowski_distances", "minkowski_distances(Tensor x1, Tensor? x2=None, float p=2) -> Tensor"},
    {"wminkowski_distances", "wminkowski_distances(Tensor x1, Tensor? x2=None, float p=2, Tensor? w=None) -> Tensor"},
    {"sqeuclidean_distances", "sqeuclidean_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"correlation_distances", "correlation_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"hamming_distances", "hamming_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"jaccard_distances", "jaccard_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"kulsinski_distances", "kulsinski_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"kulczynski1_distances", "kulczynski1_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"seuclidean_distances", "seuclidean_distances(Tensor x1, Tensor? x2=None, Tensor? V=None) -> Tensor"},
    {"cityblock_distances", "cityblock_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"mahalanobis_distances", "mahalanobis_distances(Tensor x1, Tensor? x2=None, Tensor? VI=None) -> Tensor"},
    {"chebyshev_distances", "chebyshev_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"braycurtis_distances", "braycurtis_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"canberra_distances", "canberra_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"jensenshannon_distances", "jensenshannon_distances(Tensor x1, Tensor? x2=None, float? base=None) -> Tensor"},
    {"yule_distances", "yule_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"dice_distances", "dice_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"rogerstanimoto_distances", "rogerstanimoto_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"russellrao_distances", "russellrao_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"sokalmichener_distances", "sokalmichener_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"sokalsneath_distances", "sokalsneath_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"snr_distances", "snr_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"l1_distances", "l1_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"l2_distances", "l2_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
    {"lp_distances", "lp_distances(Tensor x1, Tensor? x2=None, float p=2) -> Tensor"},
    {"linf_distances", "linf_distances(Tensor x1, Tensor? x2=None) -> Tensor"},
};

const char *schema_of(c10::string_view name) {
    for (const auto &e : kPublicSchemas)
        if (name == e.name) return e.schema;
    TORCH_INTERNAL_ASSERT(false, "no public schema ", std::string(name));
}

// ------------------------------------------------------------------------------------
// public functions (csrc/ops/pairwise_metrics.cpp)
// ------------------------------------------------------------------------------------
at::Tensor euclidean_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("euclidean_distances", x1, x2);
    return route_cdist(xs.first, xs.second, 2);
}

at::Tensor manhattan_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("manhattan_distances", x1, x2);
    return route_cdist(xs.first, xs.second, 1);
}

at::Tensor cosine_similarity(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("cosine_similarity", x1, x2);
    if (hip_float_path(xs.first, xs.second)) {
        auto ab = broadcast_batch(xs.first, xs.second);
        return pw_inner(ab.first, ab.second, kCosineSim);
    }
    // pairwise_metrics.cpp:112-122
    auto x1_norm = x1.norm(2, -1, true);
    auto x2_norm = x2.has_value() ? xs.second.norm(2, -1, true) : x1_norm;
    auto denom = x1_norm.mul(x2_norm.transpose(-1, -2));
    return prf_div(xs.first.matmul(xs.second.transpose(-1, -2)), denom, "identity");
}

at::Tensor cosine_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("cosine_distances", x1, x2);
    if (hip_float_path(xs.first, xs.second)) {
        auto ab = broadcast_batch(xs.first, xs.second);
        return pw_inner(ab.first, ab.second, kCosineDist);
    }
    return cosine_similarity(x1, x2).neg_().add_(1).clip_(0, 2);  // pairwise_metrics.cpp:51-56
}

at::Tensor linear_kernel(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("linear_kernel", x1, x2);
    // pairwise_metrics.cpp:58-65: x1 @ x2^T; fp32 / bf16 GPU tensors on the MFMA kernel, with
    // matmul's backward (grad @ x2, grad^T @ x1) on the matrix cores
    if (hip_float_path(xs.first, xs.second)) {
        auto ab = broadcast_batch(xs.first, xs.second);
        return pw_inner(ab.first, ab.second, kDot);
    }
    return xs.first.matmul(xs.second.transpose(-1, -2));
}

// pairwise_metrics.cpp:67-78,80-90: matmul, then mul_(gamma).add_(coef0).pow_(degree) /
// tanh_(); fp32 / bf16 GPU tensors run the function in the MFMA kernel's epilogue (one
// write of the output instead of four passes), everything else the composite.
at::Tensor polynomial_kernel(const at::Tensor &x1, const c10::optional<at::Tensor> &x2,
                             int64_t degree, c10::optional<double> gamma, double coef0) {
    auto xs = check_pairwise_inputs("polynomial_kernel", x1, x2);
    const double g = gamma.value_or(1.0 / x1.size(1));
    if (hip_float_path(xs.first, xs.second)) {
        auto ab = broadcast_batch(xs.first, xs.second);
        return pw_kernel(ab.first, ab.second, TPW_KER_POLYNOMIAL, g, coef0, degree);
    }
    return xs.first.matmul(xs.second.transpose(-1, -2)).mul_(g).add_(coef0).pow_(degree);
}

at::Tensor sigmoid_kernel(const at::Tensor &x1, const c10::optional<at::Tensor> &x2,
                          c10::optional<double> gamma, double coef0) {
    auto xs = check_pairwise_inputs("sigmoid_kernel", x1, x2);
    const double g = gamma.value_or(1.0 / x1.size(1));
    if (hip_float_path(xs.first, xs.second)) {
        auto ab = broadcast_batch(xs.first, xs.second);
        return pw_kernel(ab.first, ab.second, TPW_KER_SIGMOID, g, coef0, 0);
    }
    return xs.first.matmul(xs.second.transpose(-1, -2)).mul_(g).add_(coef0).tanh_();
}

at::Tensor sqeuclidean_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("sqeuclidean_distances", x1, x2);
    // pairwise_metrics.cpp:181-188: the direct sum of squared differences (no
    // |a|^2 + |b|^2 - 2ab cancellation: identical points give exactly 0)
    return ppminkowski(xs.first, xs.second, 2);
}

// pairwise_metrics.cpp:92-110: sqeuclidean (_ppminkowski p = 2) or cdist p = 1, then
// mul_(-gamma).exp_(); GPU tensors take the exponential in the VALU kernel's epilogue.
at::Tensor rbf_kernel(const at::Tensor &x1, const c10::optional<at::Tensor> &x2,
                      c10::optional<double> gamma) {
    const double g = gamma.value_or(1.0 / x1.size(1));
    if (x1.is_cuda() && (x1.scalar_type() == at::kFloat || x1.scalar_type() == at::kBFloat16 ||
                         x1.scalar_type() == at::kHalf)) {
        auto xs = check_pairwise_inputs("sqeuclidean_distances", x1, x2);
        return pw_exp_kernel(xs.first, xs.second, TPW_KER_RBF, g);
    }
    return sqeuclidean_distances(x1, x2).mul(-g).exp();
}

at::Tensor laplacian_kernel(const at::Tensor &x1, const c10::optional<at::Tensor> &x2,
                            c10::optional<double> gamma) {
    auto xs = check_pairwise_inputs("laplacian_kernel", x1, x2);
    const double g = gamma.value_or(1.0 / x1.size(1));
    if (hip_float_path(xs.first, xs.second)) {
        auto ab = broadcast_batch(xs.first, xs.second);
        return pw_exp_kernel(ab.first, ab.second, TPW_KER_LAPLACIAN, g);
    }
    return route_cdist(xs.first, xs.second, 1).mul(-g).exp();
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> directed_hausdorff_distances(
    const at::Tensor &x1, const c10::optional<at::Tensor> &x2, bool shuffle,
    c10::optional<at::Generator> generator) {
    auto xs = check_pairwise_inputs<false, true>("directed_hausdorff_distances", x1, x2);
    return directed_hausdorff(xs.first, xs.second, shuffle, generator);
}

at::Tensor minkowski_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2, double p) {
    auto xs = check_pairwise_inputs("minkowski_distances", x1, x2);
    return route_cdist(xs.first, xs.second, p);
}

at::Tensor wminkowski_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2, double p,
                                const c10::optional<at::Tensor> &w) {
    auto xs = check_pairwise_inputs("wminkowski_distances", x1, x2);
    // pairwise_metrics.cpp:170-179
    return w.has_value() ? wminkowski(xs.first, xs.second, w.value(), p) : route_cdist(xs.first, xs.second, p);
}

at::Tensor seuclidean_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2,
                                const c10::optional<at::Tensor> &V) {
    // pairwise_metrics.cpp:245-263 (it checks its inputs under the name euclidean_distances)
    TORCH_CHECK(!x2.has_value() || V.has_value(), "V is required for seuclidean when x2 is passed.")
    auto xs = check_pairwise_inputs("euclidean_distances", x1, x2);
    at::Tensor V_;
    if (V.has_value()) {
        V_ = V.value();
    } else {
        at::NoGradGuard no_grad_guard;
        V_ = xs.first.dim() == 2 ? xs.first.var(at::IntArrayRef{0}) : xs.first.var(at::IntArrayRef{0, 1});
    }
    // prf_ldiv(V, 1, "identity") = V != 0 ? 1 / V : 1, differentiable as such
    auto w = V_.masked_fill(V_ == 0, 1).reciprocal();
    return wminkowski(xs.first, xs.second, w, 2);
}

// pairwise_metrics.cpp:124-145: non-negative inputs required.  (chi2_kernel checks its
// inputs under the additive_chi2_kernel name and passes the raw x1, as the reference.)
void check_non_negative(const at::Tensor &x1, const c10::optional<at::Tensor> &x2, const at::Tensor &x2_) {
    TORCH_CHECK(x1.ge(0).all().item<bool>() && (!x2.has_value() || x2_.ge(0).all().item<bool>()),
                "All elements of x1 and x2 must be positive")
}

at::Tensor additive_chi2_kernel(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("additive_chi2_kernel", x1, x2);
    check_non_negative(xs.first, x2, xs.second);
    return additive_chi2(xs.first, xs.second);
}

at::Tensor chi2_kernel(const at::Tensor &x1, const c10::optional<at::Tensor> &x2, double gamma) {
    auto xs = check_pairwise_inputs("additive_chi2_kernel", x1, x2);
    check_non_negative(xs.first, x2, xs.second);
    return additive_chi2(x1, xs.second).mul_(gamma).exp_();
}

at::Tensor jensenshannon_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2,
                                   c10::optional<double> base) {
    // pairwise_metrics.cpp:325-335: rows normalised to sum 1, then sqrt of _sqjensenshannon
    auto xs = check_pairwise_inputs("jensenshannon_distances", x1, x2);
    auto a = xs.first / xs.first.sum(-1, true);
    auto b = x2.has_value() ? xs.second / xs.second.sum(-1, true) : a;
    return sqjensenshannon(a, b, base).sqrt_();
}

at::Tensor haversine_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("haversine_distances", x1, x2);  // pairwise_metrics.cpp:33-40
    return haversine(xs.first, xs.second);
}

at::Tensor snr_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("snr_distances", x1, x2);  // pairwise_metrics.cpp:401-408
    return snr(xs.first, xs.second).reciprocal();
}

at::Tensor mahalanobis_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2,
                                 const c10::optional<at::Tensor> &VI) {
    // pairwise_metrics.cpp:273-297 (the batched default VI is built as the reference builds it)
    TORCH_CHECK(!x2.has_value() || VI.has_value(), "VI is required for manhalanobis when x2 is passed.")
    auto xs = check_pairwise_inputs("mahalanobis_distances", x1, x2);
    at::Tensor VI_;
    if (VI.has_value()) {
        VI_ = VI.value();
    } else {
        at::NoGradGuard no_grad_guard;
        if (xs.first.dim() == 2) {
            VI_ = at::cov(xs.first.transpose(-1, -2)).inverse().transpose_(-1, -2);
        } else {
            auto cov = at::empty({xs.first.size(0), xs.first.size(1), xs.first.size(1)}, xs.first.options());
            for (int64_t b = 0; b < xs.first.size(0); ++b) cov.index_put_({b}, at::cov(xs.first[b].transpose(-1, -2)));
            VI_ = cov.inverse().transpose_(-1, -2);
        }
    }
    return sqmahalanobis(xs.first, xs.second, VI_).sqrt_();
}

at::Tensor braycurtis_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("braycurtis_distances", x1, x2);  // pairwise_metrics.cpp:307-315
    return braycurtis(xs.first, xs.second);
}

at::Tensor canberra_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("canberra_distances", x1, x2);  // pairwise_metrics.cpp:316-324
    return canberra(xs.first, xs.second);
}

at::Tensor correlation_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("correlation_distances", x1, x2);
    // pairwise_metrics.cpp:190-204: centre, then 1 - cosine similarity (no clip)
    at::Tensor a = xs.first - xs.first.mean(-1, true);
    at::Tensor b = x2.has_value() ? xs.second - xs.second.mean(-1, true) : a;
    if (hip_float_path(a, b)) {  // 1 - s fused into the MFMA epilogue
        auto ab = broadcast_batch(a, b);
        return pw_inner(ab.first, ab.second, kCorrelation);
    }
    auto a_norm = a.norm(2, -1, true);
    auto b_norm = x2.has_value() ? b.norm(2, -1, true) : a_norm;
    auto denom = a_norm.mul(b_norm.transpose(-1, -2));
    return prf_div(a.matmul(b.transpose(-1, -2)), denom, "identity").neg_().add_(1);
}

at::Tensor hamming_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("hamming_distances", x1, x2);
    return pw_binary_reduce("pwne_mean", xs.first, xs.second);
}

at::Tensor jaccard_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs<true>("jaccard_distances", x1, x2);
    return jaccard_fused(xs.first, xs.second);
}

at::Tensor kulsinski_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    TORCH_WARN_DEPRECATION("kulsinski_distances is deprecated in SciPy 1.9.0 and might "
                           "be removed in the future. Please use kulczynski1_distances.")
    auto xs = check_pairwise_inputs<true>("kulsinski_distances", x1, x2);
    if (auto r = bool_count_metric(xs.first, xs.second, "kulsinski"); r.defined()) return r;
    auto S = pw_binary_reduce("pwxor_sum", xs.first, xs.second);
    const int64_t D = x1.size(-1);
    return (S - pw_binary_reduce("pwand_sum", xs.first, xs.second) + D) / (S + D);
}

at::Tensor kulczynski1_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs<true>("kulczynski1_distances", x1, x2);
    if (auto r = bool_count_metric(xs.first, xs.second, "kulczynski1"); r.defined()) return r;
    return pw_binary_reduce("pwand_sum", xs.first, xs.second) /
           pw_binary_reduce("pwxor_sum", xs.first, xs.second);
}

at::Tensor cityblock_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    return manhattan_distances(x1, x2);
}

at::Tensor chebyshev_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs("chebyshev_distances", x1, x2);
    return route_cdist(xs.first, xs.second, std::numeric_limits<double>::infinity());
}

at::Tensor yule_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs<true>("yule_distances", x1, x2);
    if (auto r = bool_count_metric(xs.first, xs.second, "yule"); r.defined()) return r;
    const at::Tensor &a = xs.first, &b = xs.second;
    auto half_R = pw_binary_reduce("pwand_sum", a, b.logical_not()) *
                  pw_binary_reduce("pwand_sum", a.logical_not(), b);
    return prf_div(2 * half_R,
                   pw_binary_reduce("pwand_sum", a, b) *
                           pw_binary_reduce("pwand_sum", a.logical_not(), b.logical_not()) +
                       half_R,
                   "zero");
}

at::Tensor dice_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs<true>("dice_distances", x1, x2);
    if (auto r = bool_count_metric(xs.first, xs.second, "dice"); r.defined()) return r;
    auto R = pw_binary_reduce("pwxor_sum", xs.first, xs.second);
    return R / (2 * pw_binary_reduce("pwand_sum", xs.first, xs.second) + R);
}

at::Tensor rogerstanimoto_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs<true>("rogerstanimoto_distances", x1, x2);
    if (auto r = bool_count_metric(xs.first, xs.second, "rogerstanimoto"); r.defined()) return r;
    auto R = 2 * pw_binary_reduce("pwxor_sum", xs.first, xs.second);
    auto S = pw_binary_reduce("pweq_sum", xs.first, xs.second);
    return R / (S + R);
}

at::Tensor russellrao_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs<true>("russellrao_distances", x1, x2);
    if (auto r = bool_count_metric(xs.first, xs.second, "russellrao"); r.defined()) return r;
    const int64_t D = x1.size(-1);
    return (D - pw_binary_reduce("pwand_sum", xs.first, xs.second)) / D;
}

at::Tensor sokalmichener_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs<true>("sokalmichener_distances", x1, x2);
    if (auto r = bool_count_metric(xs.first, xs.second, "sokalmichener"); r.defined()) return r;
    auto R = 2 * pw_binary_reduce("pwxor_sum", xs.first, xs.second);
    auto S = pw_binary_reduce("pweq_sum", xs.first, xs.second);
    return R / (S + R);
}

at::Tensor sokalsneath_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    auto xs = check_pairwise_inputs<true>("sokalsneath_distances", x1, x2);
    if (auto r = bool_count_metric(xs.first, xs.second, "sokalsneath"); r.defined()) return r;
    auto R = 2 * pw_binary_reduce("pwxor_sum", xs.first, xs.second);
    return R / (pw_binary_reduce("pwand_sum", xs.first, xs.second) + R);
}

at::Tensor l1_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    return manhattan_distances(x1, x2);
}
at::Tensor l2_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    return euclidean_distances(x1, x2);
}
at::Tensor lp_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2, double p) {
    return minkowski_distances(x1, x2, p);
}
at::Tensor linf_distances(const at::Tensor &x1, const c10::optional<at::Tensor> &x2) {
    return chebyshev_distances(x1, x2);
}

// outside the hot path: registered so the schemas match, but not served by this build

// ------------------------------------------------------------------------------------
// cdist(metric=...) and pdist (csrc/ops/cpdist.cpp)
// ------------------------------------------------------------------------------------
struct CdistArgs {
    const c10::optional<at::Tensor> &w, &V, &VI;
    c10::optional<double> p, base;
    c10::optional<bool> shuffle;
    c10::optional<at::Generator> generator;
};

// Which optional arguments a metric accepts, in the order the error message lists them
// (the has_arg table of cpdist.cpp:85-146).
enum ExtraArg : unsigned { kW = 1, kV = 2, kVI = 4, kP = 8, kBase = 16, kShuffle = 32, kGenerator = 64 };

struct CdistMetric {
    const char *metric;
    unsigned accepts;
    at::Tensor (*call)(const at::Tensor &, const at::Tensor &, const CdistArgs &);
};

// cpdist.cpp:35-79: arguments given but not accepted raise TypeError quoting the schema.
void check_extra_args(const CdistMetric &m, const CdistArgs &a) {
    const std::pair<bool, const char *> given[] = {
        {a.w.has_value(), "w"},         {a.V.has_value(), "V"},       {a.VI.has_value(), "VI"},
        {a.p.has_value(), "p"},         {a.base.has_value(), "base"}, {a.shuffle.has_value(), "shuffle"},
        {a.generator.has_value(), "generator"}};
    std::string bad;
    for (int i = 0; i < 7; ++i)
        if (given[i].first && !(m.accepts & (1u << i))) bad += (bad.empty() ? "" : ", ") + std::string(given[i].second);
    const std::string fn = std::string(m.metric) + "_distances";
    TORCH_CHECK_TYPE(bad.empty(), "torchpairwise::", fn, " was called with incompatible arguments ", bad,
                     ".\nThe following signature is supported:\n", "    ", schema_of(fn), "\n")
}

#define TPW_METRIC(NAME, ACCEPTS, EXPR) \
    {#NAME, ACCEPTS, [](const at::Tensor &x1, const at::Tensor &x2, const CdistArgs &a) -> at::Tensor { \
         (void)a;                                                                                        \
         return EXPR;                                                                                    \
     }}
// dispatch order of cpdist.cpp:184-219
const CdistMetric kCdistMetrics[] = {
    TPW_METRIC(euclidean, 0, euclidean_distances(x1, x2)),
    TPW_METRIC(haversine, 0, haversine_distances(x1, x2)),
    TPW_METRIC(manhattan, 0, manhattan_distances(x1, x2)),
    TPW_METRIC(cosine, 0, cosine_distances(x1, x2)),
    TPW_METRIC(directed_hausdorff, kShuffle | kGenerator,
               std::get<0>(directed_hausdorff_distances(x1, x2, a.shuffle.value_or(false), a.generator))),
    TPW_METRIC(minkowski, kP, minkowski_distances(x1, x2, a.p.value_or(2))),
    TPW_METRIC(wminkowski, kW | kP, wminkowski_distances(x1, x2, a.p.value_or(2), a.w)),
    TPW_METRIC(sqeuclidean, 0, sqeuclidean_distances(x1, x2)),
    TPW_METRIC(correlation, 0, correlation_distances(x1, x2)),
    TPW_METRIC(hamming, 0, hamming_distances(x1, x2)),
    TPW_METRIC(jaccard, 0, jaccard_distances(x1, x2)),
    // kept from the reference: its C++ kulsinski_distances, which cdist calls, forwards to the
    // kulczynski1 functor (pairwise_metrics.h:557-561), so cdist(metric="kulsinski") gives
    // kulczynski1 distances (and no deprecation warning); the kulsinski_distances op does not
    TPW_METRIC(kulsinski, 0, kulczynski1_distances(x1, x2)),
    TPW_METRIC(kulczynski1, 0, kulczynski1_distances(x1, x2)),
    TPW_METRIC(seuclidean, kV, seuclidean_distances(x1, x2, a.V)),
    TPW_METRIC(cityblock, 0, cityblock_distances(x1, x2)),
    TPW_METRIC(mahalanobis, kVI, mahalanobis_distances(x1, x2, a.VI)),
    TPW_METRIC(chebyshev, 0, chebyshev_distances(x1, x2)),
    TPW_METRIC(braycurtis, 0, braycurtis_distances(x1, x2)),
    TPW_METRIC(canberra, 0, canberra_distances(x1, x2)),
    TPW_METRIC(jensenshannon, kBase, jensenshannon_distances(x1, x2, a.base)),
    TPW_METRIC(yule, 0, yule_distances(x1, x2)),
    TPW_METRIC(dice, 0, dice_distances(x1, x2)),
    TPW_METRIC(rogerstanimoto, 0, rogerstanimoto_distances(x1, x2)),
    TPW_METRIC(russellrao, 0, russellrao_distances(x1, x2)),
    TPW_METRIC(sokalmichener, 0, sokalmichener_distances(x1, x2)),
    TPW_METRIC(sokalsneath, 0, sokalsneath_distances(x1, x2)),
    TPW_METRIC(snr, 0, snr_distances(x1, x2)),
    TPW_METRIC(l1, 0, l1_distances(x1, x2)),
    TPW_METRIC(l2, 0, l2_distances(x1, x2)),
    TPW_METRIC(lp, kP, lp_distances(x1, x2, a.p.value_or(2))),
    TPW_METRIC(linf, 0, linf_distances(x1, x2)),
};
#undef TPW_METRIC

at::Tensor cdist(const at::Tensor &x1, const at::Tensor &x2, c10::string_view metric,
                 const c10::optional<at::Tensor> &w, const c10::optional<at::Tensor> &V,
                 const c10::optional<at::Tensor> &VI, c10::optional<double> p,
                 c10::optional<double> base, c10::optional<bool> shuffle,
                 c10::optional<at::Generator> generator) {
    C10_LOG_API_USAGE_ONCE("torchpairwise.csrc.ops.cpdist.cdist");
    const CdistArgs args{w, V, VI, p, base, shuffle, std::move(generator)};
    for (const auto &m : kCdistMetrics) {
        if (metric == m.metric) {
            check_extra_args(m, args);
            return m.call(x1, x2, args);
        }
    }
    // the reference's message, spelling included (cpdist.cpp:180-231)
    static const char *const supported[] = {
        "braycurtis", "canberra", "chebyshev", "cityblock", "correlation", "cosine",
        "dice", "directed_hausdorff", "euclidean", "hamming", "haversine", "jaccard",
        "jensenshannon", "kulczynski1", "kulsinski", "l1", "l2", "lp", "linf", "mahalanobis",
        "manhattan", "minkowski", "rogerstanimoto", "russellrao", "seuclidean", "snr",
        "sokalmichener", "sokalsneath", "sqeuclidean", "wminkowski", "yule"};
    std::string list;
    for (const char *s : supported) list += (list.empty() ? "" : ", ") + std::string(s);
    TORCH_CHECK(false, "Got unkown distance metric: ", std::string(metric), ". Supported metrics are [",
                list, "]")
}

at::Tensor pdist(const at::Tensor &, c10::string_view, const c10::optional<at::Tensor> &,
                 const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,
                 c10::optional<double>, c10::optional<double>, c10::optional<bool>,
                 c10::optional<at::Generator>) {
    C10_LOG_API_USAGE_ONCE("torchpairwise.csrc.ops.cpdist.pdist");
    TORCH_CHECK_NOT_IMPLEMENTED(false, "pdist is yet to be implemented.")  // cpdist.cpp:244-245
}

// ------------------------------------------------------------------------------------
// neighbour masks (csrc/ops/neighbors.cpp)
// ------------------------------------------------------------------------------------
// neighbors.cpp:29-34 literally: argsort every row, keep the first k + 1 columns, scatter
// true.  (When k + 1 exceeds the number of columns the two index tensors of index_put_ do
// not broadcast and ATen raises; that behaviour is kept by running this same code.)
at::Tensor k_neighbors_from_argsort(const at::Tensor &dists, int64_t k, int64_t n1, int64_t n2) {
    auto neighbors_inds = dists.argsort(1, false).slice(1, 0, k + 1);
    auto first_dim = at::arange(0, n1, neighbors_inds.options()).view({-1, 1}).repeat({1, k + 1});
    auto output = at::zeros({n1, n2}, dists.options().dtype(at::kBool));
    output.index_put_({first_dim.flatten(), neighbors_inds.flatten()}, true);
    return output;
}

// Largest k + 1 the fused euclidean k-neighbour route takes.  At 16384 x 16384 x 128 fp32 the
// fused route takes 0.67 / 0.74 ms for k + 1 = 2 / 4 against 0.84 ms for the distances and the
// selection kernel; at 8 and 16 the wider candidate lists (two blocks per CU) make it slower
// (1.01 / 1.46 ms).
constexpr int64_t kKnnFusedMaxCount = 4;

at::Tensor k_neighbors_mask(const at::Tensor &x1, const c10::optional<at::Tensor> &x2, int64_t k,
                            c10::string_view metric, const c10::optional<at::Tensor> &w,
                            const c10::optional<at::Tensor> &V, const c10::optional<at::Tensor> &VI,
                            c10::optional<double> p, c10::optional<double> base,
                            c10::optional<bool> shuffle, c10::optional<at::Generator> generator) {
    C10_LOG_API_USAGE_ONCE("torchpairwise.csrc.ops.neighbors.k_neighbors_mask");
    auto xs = check_pairwise_inputs("k_neighbors_mask", x1, x2);
    TORCH_CHECK(k >= 0, "k must be non-negative. Got k=", k)
    at::NoGradGuard no_grad_guard;
    // the euclidean metric on the GPU's matrix-product path (route_cdist's rule) for small k: the
    // tile kernel keeps each row's k + 1 smallest per tile and the distances are never written
    if (metric == "euclidean" && !w.has_value() && !V.has_value() && !VI.has_value() && !p.has_value() &&
        !base.has_value() && !shuffle.has_value() && !generator.has_value() && hip_float_path(xs.first, xs.second) &&
        xs.first.dim() == 2 && (xs.first.size(0) > 25 || xs.second.size(0) > 25) && k + 1 <= kKnnFusedMaxCount &&
        tpw_knn_mask_euclidean_supported(xs.first.scalar_type() == at::kFloat ? TPW_F32 : TPW_BF16, xs.first.size(0),
                                         xs.second.size(0), xs.first.size(1), k + 1) &&
        xs.first.is_contiguous() && xs.second.is_contiguous()) {
        static auto op = c10::Dispatcher::singleton()
                             .findSchemaOrThrow("torchpairwise::_knn_mask_euclidean", "")
                             .typed<at::Tensor(const at::Tensor &, const at::Tensor &, int64_t)>();
        return op.call(xs.first, xs.second, k + 1);
    }
    auto dists = cdist(xs.first, xs.second, metric, w, V, VI, p, base, shuffle, std::move(generator));
    const int64_t n1 = x1.size(0), n2 = xs.second.size(0);
    // GPU: one pass over the distances selecting each row's k + 1 smallest (HIP kernel)
    if (dists.is_cuda() && dists.dim() == 2 && dists.size(0) == n1 && dists.size(1) == n2 &&
        k < n2 &&
        (dists.scalar_type() == at::kFloat || dists.scalar_type() == at::kBFloat16 ||
         dists.scalar_type() == at::kHalf))
        return row_smallest_mask(dists, k + 1);
    return k_neighbors_from_argsort(dists, k, n1, n2);
}

at::Tensor radius_neighbors_mask(const at::Tensor &x1, const c10::optional<at::Tensor> &x2,
                                 double epsilon, c10::string_view metric,
                                 const c10::optional<at::Tensor> &w, const c10::optional<at::Tensor> &V,
                                 const c10::optional<at::Tensor> &VI, c10::optional<double> p,
                                 c10::optional<double> base, c10::optional<bool> shuffle,
                                 c10::optional<at::Generator> generator) {
    // (the reference logs this one under the k_neighbors_mask key too, neighbors.cpp:49)
    C10_LOG_API_USAGE_ONCE("torchpairwise.csrc.ops.neighbors.k_neighbors_mask");
    auto xs = check_pairwise_inputs("radius_neighbors_mask", x1, x2);
    TORCH_CHECK(epsilon >= 0., "epsilon must be non-negative. Got epsilon=", epsilon)
    at::NoGradGuard no_grad_guard;
    // the euclidean metric on the GPU's matrix-product path (route_cdist's rule): the mask straight
    // from the MFMA epilogue, the same distances compared without writing them
    if (metric == "euclidean" && !w.has_value() && !V.has_value() && !VI.has_value() && !p.has_value() &&
        !base.has_value() && !shuffle.has_value() && !generator.has_value() && hip_float_path(xs.first, xs.second)) {
        auto ab = broadcast_batch(xs.first, xs.second);
        if (ab.first.size(-2) > 25 || ab.second.size(-2) > 25) {
            static auto op = c10::Dispatcher::singleton()
                                 .findSchemaOrThrow("torchpairwise::_radius_mask_euclidean", "")
                                 .typed<at::Tensor(const at::Tensor &, const at::Tensor &, double)>();
            return op.call(ab.first, ab.second, epsilon);
        }
    }
    auto dists = cdist(xs.first, xs.second, metric, w, V, VI, p, base, shuffle, std::move(generator));
    return dists.le(epsilon);
}

int64_t cuda_version() { return tpw_runtime_version(); }
std::string cuda_arch_flags() { return "gfx950"; }

}  // namespace

// ------------------------------------------------------------------------------------
// dispatcher handles of the internal ops
// ------------------------------------------------------------------------------------
at::Tensor pw_kernel(const at::Tensor &x1, const at::Tensor &x2, int64_t kind, double gamma,
                     double coef0, int64_t degree) {
    static auto op = c10::Dispatcher::singleton().findSchemaOrThrow("torchpairwise::_pw_kernel", "")
                         .typed<at::Tensor(const at::Tensor &, const at::Tensor &, int64_t, double,
                                           double, int64_t)>();
    return op.call(x1, x2, kind, gamma, coef0, degree);
}

std::tuple<at::Tensor, at::Tensor> pw_kernel_backward(const at::Tensor &grad, const at::Tensor &x1,
                                                      const at::Tensor &x2, const at::Tensor &res,
                                                      int64_t kind, double gamma, double coef0,
                                                      int64_t degree) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("torchpairwise::_pw_kernel_backward", "")
                         .typed<std::tuple<at::Tensor, at::Tensor>(
                             const at::Tensor &, const at::Tensor &, const at::Tensor &,
                             const at::Tensor &, int64_t, double, double, int64_t)>();
    return op.call(grad, x1, x2, res, kind, gamma, coef0, degree);
}

at::Tensor pw_inner(const at::Tensor &x1, const at::Tensor &x2, int64_t epilogue) {
    static auto op = c10::Dispatcher::singleton().findSchemaOrThrow("torchpairwise::_pw_inner", "")
                         .typed<at::Tensor(const at::Tensor &, const at::Tensor &, int64_t)>();
    return op.call(x1, x2, epilogue);
}

std::tuple<at::Tensor, at::Tensor> pw_inner_backward(const at::Tensor &grad, const at::Tensor &x1,
                                                     const at::Tensor &x2, const at::Tensor &res,
                                                     int64_t epilogue) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("torchpairwise::_pw_inner_backward", "")
                         .typed<std::tuple<at::Tensor, at::Tensor>(
                             const at::Tensor &, const at::Tensor &, const at::Tensor &,
                             const at::Tensor &, int64_t)>();
    return op.call(grad, x1, x2, res, epilogue);
}

at::Tensor pw_lp(const at::Tensor &x1, const at::Tensor &x2, double p) {
    static auto op = c10::Dispatcher::singleton().findSchemaOrThrow("torchpairwise::_pw_lp", "")
                         .typed<at::Tensor(const at::Tensor &, const at::Tensor &, double)>();
    return op.call(x1, x2, p);
}

std::tuple<at::Tensor, at::Tensor> pw_lp_backward(const at::Tensor &grad, const at::Tensor &x1,
                                                  const at::Tensor &x2, const at::Tensor &dist,
                                                  double p) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("torchpairwise::_pw_lp_backward", "")
                         .typed<std::tuple<at::Tensor, at::Tensor>(
                             const at::Tensor &, const at::Tensor &, const at::Tensor &,
                             const at::Tensor &, double)>();
    return op.call(grad, x1, x2, dist, p);
}

at::Tensor pw_binary_reduce(const char *name, const at::Tensor &x1, const at::Tensor &x2) {
    auto op = c10::Dispatcher::singleton()
                  .findSchemaOrThrow((std::string("torchpairwise::") + name).c_str(), "")
                  .typed<at::Tensor(const at::Tensor &, const at::Tensor &)>();
    return op.call(x1, x2);
}

at::Tensor jaccard_fused(const at::Tensor &x1, const at::Tensor &x2) {
    static auto op = c10::Dispatcher::singleton().findSchemaOrThrow("torchpairwise::_jaccard", "")
                         .typed<at::Tensor(const at::Tensor &, const at::Tensor &)>();
    return op.call(x1, x2);
}

at::Tensor prf_div(const at::Tensor &x, const at::Tensor &y, c10::string_view mode) {
    static auto op = c10::Dispatcher::singleton().findSchemaOrThrow("torchpairwise::prf_div", "")
                         .typed<at::Tensor(const at::Tensor &, const at::Tensor &, c10::string_view)>();
    return op.call(x, y, mode);
}

std::tuple<at::Tensor, at::Tensor> prf_div_backward(const at::Tensor &g, const at::Tensor &x,
                                                    const at::Tensor &y, c10::string_view mode) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("torchpairwise::_prf_div_backward", "")
                         .typed<std::tuple<at::Tensor, at::Tensor>(
                             const at::Tensor &, const at::Tensor &, const at::Tensor &,
                             c10::string_view)>();
    return op.call(g, x, y, mode);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> directed_hausdorff(
    const at::Tensor &x1, const at::Tensor &x2, bool shuffle, c10::optional<at::Generator> gen) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("torchpairwise::_directed_hausdorff", "")
                         .typed<std::tuple<at::Tensor, at::Tensor, at::Tensor>(
                             const at::Tensor &, const at::Tensor &, bool,
                             c10::optional<at::Generator>)>();
    return op.call(x1, x2, shuffle, gen);
}

std::tuple<at::Tensor, at::Tensor> directed_hausdorff_backward(
    const at::Tensor &grad, const at::Tensor &x1, const at::Tensor &x2, bool shuffle,
    c10::optional<at::Generator> gen) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("torchpairwise::__directed_hausdorff_backward", "")
                         .typed<std::tuple<at::Tensor, at::Tensor>(
                             const at::Tensor &, const at::Tensor &, const at::Tensor &, bool,
                             c10::optional<at::Generator>)>();
    return op.call(grad, x1, x2, shuffle, gen);
}

at::Tensor row_smallest_mask(const at::Tensor &dist, int64_t count) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("torchpairwise::_row_smallest_mask", "")
                         .typed<at::Tensor(const at::Tensor &, int64_t)>();
    return op.call(dist, count);
}

TORCH_LIBRARY_FRAGMENT(torchpairwise, m) {
    // ---- internal ops of this build (HIP kernels; Autograd in autograd.cpp) ----
    m.def("_pw_inner(Tensor x1, Tensor x2, int epilogue) -> Tensor");
    m.def("_radius_mask_euclidean(Tensor x1, Tensor x2, float epsilon) -> Tensor");
    m.def("_knn_mask_euclidean(Tensor x1, Tensor x2, int count) -> Tensor");
    m.def("_pw_kernel(Tensor x1, Tensor x2, int kind, float gamma, float coef0, int degree) -> Tensor");
    m.def("_pw_kernel_backward(Tensor grad, Tensor x1, Tensor x2, Tensor result, int kind, "
          "float gamma, float coef0, int degree) -> (Tensor, Tensor)");
    m.def("_pw_inner_backward(Tensor grad, Tensor x1, Tensor x2, Tensor result, int epilogue) -> "
          "(Tensor grad_x1, Tensor grad_x2)");
    m.def("_pw_lp(Tensor x1, Tensor x2, float p) -> Tensor");
    m.def("_pw_lp_backward(Tensor grad, Tensor x1, Tensor x2, Tensor dist, float p) -> "
          "(Tensor grad_x1, Tensor grad_x2)");
    m.def("_jaccard(Tensor x1, Tensor x2) -> Tensor");
    m.def("_row_smallest_mask(Tensor dist, int count) -> Tensor");

    // ---- internal ops of the reference (same schemas) ----
    // csrc/ops/pairwise_binary.cpp:135-160
    for (const char *op : {"pwand", "pwor", "pwxor", "pweq", "pwne", "pwlt", "pwgt", "pwle", "pwge"})
        m.def((std::string(op) + "(Tensor x1, Tensor x2) -> Tensor").c_str());
    for (const char *op : {"pwand_sum", "pwor_sum", "pwxor_sum", "pweq_sum", "pwne_sum", "pweq_mean",
                           "pwne_mean"})
        m.def((std::string(op) + "(Tensor x1, Tensor x2) -> Tensor").c_str());
    // csrc/ops/prf_div.cpp:359-400: the prf_div family is registered in prf_div.cpp
    // csrc/ops/hausdorff.cpp:33-40
    m.def("_directed_hausdorff(Tensor x1, Tensor x2, *, bool shuffle=False, Generator? generator=None) "
          "-> (Tensor output, Tensor x1_indices, Tensor x2_indices)");
    m.def("__directed_hausdorff_backward(Tensor grad, Tensor x1, Tensor x2, *, bool shuffle=False, "
          "Generator? generator=None) -> (Tensor grad_x1, Tensor grad_x2)");
    // csrc/torchpairwise.cpp:53-56
    m.def("_cuda_version() -> int", &cuda_version);
    m.def("_cuda_arch_flags() -> str", &cuda_arch_flags);

    // ---- public metrics (csrc/ops/pairwise_metrics.h schemas) ----
#define TPW_PUBLIC(fn) m.def(schema_of(#fn), TORCH_FN(fn))
    TPW_PUBLIC(euclidean_distances);
    TPW_PUBLIC(haversine_distances);
    TPW_PUBLIC(manhattan_distances);
    TPW_PUBLIC(cosine_distances);
    TPW_PUBLIC(linear_kernel);
    TPW_PUBLIC(polynomial_kernel);
    TPW_PUBLIC(sigmoid_kernel);
    TPW_PUBLIC(rbf_kernel);
    TPW_PUBLIC(laplacian_kernel);
    TPW_PUBLIC(cosine_similarity);
    TPW_PUBLIC(additive_chi2_kernel);
    TPW_PUBLIC(chi2_kernel);
    TPW_PUBLIC(directed_hausdorff_distances);
    TPW_PUBLIC(minkowski_distances);
    TPW_PUBLIC(wminkowski_distances);
    TPW_PUBLIC(sqeuclidean_distances);
    TPW_PUBLIC(correlation_distances);
    TPW_PUBLIC(hamming_distances);
    TPW_PUBLIC(jaccard_distances);
    TPW_PUBLIC(kulsinski_distances);
    TPW_PUBLIC(kulczynski1_distances);
    TPW_PUBLIC(seuclidean_distances);
    TPW_PUBLIC(cityblock_distances);
    TPW_PUBLIC(mahalanobis_distances);
    TPW_PUBLIC(chebyshev_distances);
    TPW_PUBLIC(braycurtis_distances);
    TPW_PUBLIC(canberra_distances);
    TPW_PUBLIC(jensenshannon_distances);
    TPW_PUBLIC(yule_distances);
    TPW_PUBLIC(dice_distances);
    TPW_PUBLIC(rogerstanimoto_distances);
    TPW_PUBLIC(russellrao_distances);
    TPW_PUBLIC(sokalmichener_distances);
    TPW_PUBLIC(sokalsneath_distances);
    TPW_PUBLIC(snr_distances);
    TPW_PUBLIC(l1_distances);
    TPW_PUBLIC(l2_distances);
    TPW_PUBLIC(lp_distances);
    TPW_PUBLIC(linf_distances);
#undef TPW_PUBLIC

    // ---- cdist / pdist (csrc/ops/cpdist.cpp:248-255) and neighbour masks (neighbors.cpp:62-67) ----
#define TPW_CPDIST_EXTRA "Tensor? w=None, Tensor? V=None, Tensor? VI=None, float? p=None, float? base=None, bool? shuffle=None, Generator? generator=None"
    m.def("cdist(Tensor x1, Tensor x2, str metric=\"minkowski\", *, " TPW_CPDIST_EXTRA ") -> Tensor", TORCH_FN(cdist));
    m.def("pdist(Tensor input, str metric=\"minkowski\", *, " TPW_CPDIST_EXTRA ") -> Tensor", TORCH_FN(pdist));
    m.def("k_neighbors_mask(Tensor x1, Tensor? x2=None, int k=1, str metric=\"euclidean\", *, " TPW_CPDIST_EXTRA ") -> Tensor", TORCH_FN(k_neighbors_mask));
    m.def("radius_neighbors_mask(Tensor x1, Tensor? x2=None, float epsilon=0., str metric=\"euclidean\", *, " TPW_CPDIST_EXTRA ") -> Tensor", TORCH_FN(radius_neighbors_mask));
#undef TPW_CPDIST_EXTRA
}

}  // namespace tpw_ext
