// The reference's remaining custom metric ops: _haversine, _snr and _sqmahalanobis with their
// __*_backward ops (csrc/ops/{haversine,snr,sqmahalanobis}.cpp), CPU, GPU and Autograd.
//
// _haversine runs HIP kernels on the GPU (haversine.hip: fp32, 16-bit types through fp32;
// valu_f64.hip: float64).
// _snr is a composition on the GPU:
//   _snr(x1, x2)[i, j] = V1[i] / DV[i, j], V1 = sum_k (x1 - mean x1)^2 and
//     DV = sum_k (d - mean d)^2 with d = x2[j] - x1[i]; since mean d = mean x2[j] - mean x1[i],
//     DV is the squared distance between the row-centred points, i.e. _ppminkowski(x1c, x2c, 2)
//     on the VALU kernel; its gradient comes from autograd through that composition.
// _sqmahalanobis runs mahalanobis.hip on the GPU: d^T VI d from the difference d and per-row
// projections x VI^T, O(d) per pair; its backward uses the matrix-core sqeuclidean products.
// CPU tensors run loops restating the reference's kernels.
#include "tpw_common.h"

#include <ATen/Parallel.h>
#include <ATen/core/dispatch/Dispatcher.h>
#include <torch/autograd.h>

#include <cmath>

namespace tpw_ext {
namespace {

using torch::autograd::AutogradContext;
using torch::autograd::Variable;
using torch::autograd::variable_list;
using T2 = std::tuple<at::Tensor, at::Tensor>;
using T3 = std::tuple<at::Tensor, at::Tensor, at::Tensor>;

template <typename Sig>
c10::TypedOperatorHandle<Sig> op_handle(const char *name) {
    return c10::Dispatcher::singleton().findSchemaOrThrow(name, "").typed<Sig>();
}

inline at::Tensor batched(const at::Tensor &t, bool ub) { return ub ? t.unsqueeze(0).contiguous() : t.contiguous(); }
inline at::Tensor unbatch(const at::Tensor &t, bool ub) { return ub ? t.squeeze(0) : t; }

template <typename F>
void for_rows(int64_t rows, F f) {
    at::parallel_for(0, rows, 1, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; ++r) f(r);
    });
}

// ================================================================== haversine
bool check_haversine(const at::Tensor &x1, const at::Tensor &x2) {  // cpu/haversine_kernel.cpp:32-47
    at::CheckedFrom c = "_haversine_forward";
    auto args = {at::TensorArg(x1, "x1", 1), at::TensorArg(x2, "x2", 2)};
    at::checkAllSameType(c, args);
    const bool ub = x1.dim() == 2;
    TORCH_CHECK(ub || x1.dim() == 3, "x1 must be 2-D (unbatched) or 3-D (batched) tensor.")
    TORCH_CHECK(ub || x2.dim() == 3, "x2 must be 2-D (unbatched) or 3-D (batched) tensor.")
    TORCH_CHECK(ub || x1.size(0) == x2.size(0), "batch_size of x1 and x2 do not match.")
    TORCH_CHECK((ub && x1.size(1) == 2 && x2.size(1) == 2) || (!ub && x1.size(2) == 2 && x2.size(2) == 2),
                "feature dimension of x1 and x2 must be 2.")
    return ub;
}

at::Tensor haversine_cpu(const at::Tensor &x1, const at::Tensor &x2) {
    const bool ub = check_haversine(x1, x2);
    auto a = batched(x1, ub), b = batched(x2, ub);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1);
    auto out = at::empty({B, n, m}, a.options());
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, a.scalar_type(), "_haversine_forward_cpu", [&] {
        using acc_t = std::conditional_t<std::is_same_v<scalar_t, double>, double, float>;
        const scalar_t *P = a.data_ptr<scalar_t>(), *Q = b.data_ptr<scalar_t>();
        scalar_t *O = out.data_ptr<scalar_t>();
        for_rows(B * n, [&](int64_t r) {  // cpu/haversine_kernel.cpp:22-24
            const int64_t bb = r / n;
            const acc_t la = P[2 * r], lo = P[2 * r + 1];
            for (int64_t j = 0; j < m; ++j) {
                const acc_t lb = Q[2 * (bb * m + j)], lob = Q[2 * (bb * m + j) + 1];
                const acc_t sa = std::sin((la - lb) / 2), so = std::sin((lo - lob) / 2);
                O[r * m + j] = (scalar_t)(2 * std::asin(std::sqrt(sa * sa + std::cos(la) * std::cos(lb) * so * so)));
            }
        });
    });
    return unbatch(out, ub);
}

T2 haversine_backward_cpu(const at::Tensor &grad, const at::Tensor &x1, const at::Tensor &x2) {
    const bool ub = x1.dim() == 2;
    auto a = batched(x1, ub), b = batched(x2, ub), g = batched(grad, ub);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1);
    auto gx1 = at::zeros_like(a), gx2 = at::zeros_like(b);
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, a.scalar_type(), "_haversine_backward_cpu", [&] {
        using acc_t = std::conditional_t<std::is_same_v<scalar_t, double>, double, float>;
        const scalar_t *P = a.data_ptr<scalar_t>(), *Q = b.data_ptr<scalar_t>(), *G = g.data_ptr<scalar_t>();
        scalar_t *GX1 = gx1.data_ptr<scalar_t>(), *GX2 = gx2.data_ptr<scalar_t>();
        // per pair: grad / (sqrt(val) sqrt(1 - val)) (cpu/haversine_kernel.cpp:88-93)
        auto weight = [&](int64_t bb, int64_t i, int64_t j) -> acc_t {
            const acc_t la = P[2 * (bb * n + i)], lo = P[2 * (bb * n + i) + 1];
            const acc_t lb = Q[2 * (bb * m + j)], lob = Q[2 * (bb * m + j) + 1];
            const acc_t sa = std::sin((la - lb) / 2), so = std::sin((lo - lob) / 2);
            const acc_t val = sa * sa + std::cos(la) * std::cos(lb) * so * so;
            return (acc_t)G[(bb * n + i) * m + j] / (std::sqrt(val) * std::sqrt(1 - val));
        };
        for_rows(B * n, [&](int64_t r) {  // :111-116
            const int64_t bb = r / n, i = r % n;
            const acc_t la = P[2 * r], lo = P[2 * r + 1];
            acc_t dlat = 0, dlon = 0;
            for (int64_t j = 0; j < m; ++j) {
                const acc_t lb = Q[2 * (bb * m + j)], lob = Q[2 * (bb * m + j) + 1], w = weight(bb, i, j);
                const acc_t so = std::sin((lo - lob) / 2);
                dlat += w * (-std::sin(la) * so * so * std::cos(lb) + std::sin(la - lb) / 2);
                dlon += w * (so * std::cos(la) * std::cos(lb) * std::cos((lo - lob) / 2));
            }
            GX1[2 * r] = (scalar_t)dlat;
            GX1[2 * r + 1] = (scalar_t)dlon;
        });
        for_rows(B * m, [&](int64_t r) {  // :138-143
            const int64_t bb = r / m, j = r % m;
            const acc_t lb = Q[2 * r], lob = Q[2 * r + 1];
            acc_t dlat = 0, dlon = 0;
            for (int64_t i = 0; i < n; ++i) {
                const acc_t la = P[2 * (bb * n + i)], lo = P[2 * (bb * n + i) + 1], w = weight(bb, i, j);
                const acc_t so = std::sin((lo - lob) / 2);
                dlat += w * (-std::sin(lb) * so * so * std::cos(la) - std::sin(la - lb) / 2);
                dlon += w * (-so * std::cos(la) * std::cos(lb) * std::cos((lo - lob) / 2));
            }
            GX2[2 * r] = (scalar_t)dlat;
            GX2[2 * r + 1] = (scalar_t)dlon;
        });
    });
    return {unbatch(gx1, ub), unbatch(gx2, ub)};
}

// fp32 operands (16-bit types computed in fp32); float64 takes the fp64 kernels.
at::Tensor gpu_f32(const at::Tensor &t, const char *) { return t.to(at::kFloat).contiguous(); }

at::Tensor haversine_cuda(const at::Tensor &x1, const at::Tensor &x2) {
    const bool ub = check_haversine(x1, x2);
    check_float_dispatch(x1.scalar_type(), true, "_haversine_forward_cuda");
    DeviceGuard guard(x1.device());
    if (x1.scalar_type() == at::kDouble) {
        auto a = batched(x1, ub), b = batched(x2, ub);
        auto out = at::empty({a.size(0), a.size(1), b.size(1)}, a.options());
        check_rc(tpw_haversine_f64(a.data_ptr<double>(), b.data_ptr<double>(), a.size(0), a.size(1), b.size(1),
                                   out.data_ptr<double>(), current_stream()),
                 "_haversine");
        return unbatch(out, ub);
    }
    auto a = batched(gpu_f32(x1, "_haversine"), ub), b = batched(gpu_f32(x2, "_haversine"), ub);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1);
    auto out = at::empty({B, n, m}, a.options());
    auto ws = workspace(tpw_haversine_workspace_size(B, n, m), a);
    check_rc(tpw_haversine(a.data_ptr<float>(), b.data_ptr<float>(), B, n, m, out.data_ptr<float>(),
                           ws.data_ptr(), current_stream()),
             "_haversine");
    return unbatch(out, ub).to(x1.scalar_type());
}

T2 haversine_backward_cuda(const at::Tensor &grad, const at::Tensor &x1, const at::Tensor &x2) {
    const bool ub = x1.dim() == 2;
    check_float_dispatch(grad.scalar_type(), true, "_haversine_backward_cuda");
    DeviceGuard guard(x1.device());
    if (x1.scalar_type() == at::kDouble) {
        auto a = batched(x1, ub), b = batched(x2, ub), g = batched(grad.to(at::kDouble), ub);
        auto gx1 = at::empty_like(a), gx2 = at::empty_like(b);
        check_rc(tpw_haversine_f64_backward(g.data_ptr<double>(), a.data_ptr<double>(), b.data_ptr<double>(),
                                            a.size(0), a.size(1), b.size(1), gx1.data_ptr<double>(),
                                            gx2.data_ptr<double>(), current_stream()),
                 "_haversine_backward");
        return {unbatch(gx1, ub), unbatch(gx2, ub)};
    }
    auto a = batched(gpu_f32(x1, "_haversine_backward"), ub), b = batched(gpu_f32(x2, "_haversine_backward"), ub);
    auto g = batched(gpu_f32(grad, "_haversine_backward"), ub);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1);
    auto gx1 = at::empty_like(a), gx2 = at::empty_like(b);
    auto ws = workspace(tpw_haversine_workspace_size(B, n, m), a);
    check_rc(tpw_haversine_backward(g.data_ptr<float>(), a.data_ptr<float>(), b.data_ptr<float>(), B, n, m,
                                    gx1.data_ptr<float>(), gx2.data_ptr<float>(), ws.data_ptr(),
                                    current_stream()),
             "_haversine_backward");
    return {unbatch(gx1, ub).to(x1.scalar_type()), unbatch(gx2, ub).to(x2.scalar_type())};
}

// ================================================================== snr
bool check_snr(const at::Tensor &x1, const at::Tensor &x2) {  // cpu/snr_kernel.cpp:70-85
    at::CheckedFrom c = "_snr_forward";
    auto args = {at::TensorArg(x1, "x1", 1), at::TensorArg(x2, "x2", 2)};
    at::checkAllSameType(c, args);
    const bool ub = x1.dim() == 2;
    TORCH_CHECK(ub || x1.dim() == 3, "x1 must be 2-D (unbatched) or 3-D (batched) tensor.")
    TORCH_CHECK(ub || x2.dim() == 3, "x2 must be 2-D (unbatched) or 3-D (batched) tensor.")
    TORCH_CHECK(ub || (x1.size(0) == x2.size(0)), "batch_size of x1 and x2 do not match.")
    TORCH_CHECK((ub && x1.size(1) == x2.size(1)) || (!ub && x1.size(2) == x2.size(2)),
                "feature dimension of x1 and x2 do not match.")
    return ub;
}

// The reference's two passes per pair: mean of d = x2[j] - x1[i], then sum (d - mean)^2.
template <typename acc_t, typename scalar_t>
void snr_pair_stats(const scalar_t *u, const scalar_t *v, int64_t d, acc_t &mean, acc_t &var) {
    mean = 0;
    for (int64_t k = 0; k < d; ++k) mean += (acc_t)v[k] - (acc_t)u[k];
    mean /= (acc_t)d;
    var = 0;
    for (int64_t k = 0; k < d; ++k) {
        const acc_t t = (acc_t)v[k] - (acc_t)u[k] - mean;
        var += t * t;
    }
}

at::Tensor snr_cpu(const at::Tensor &x1, const at::Tensor &x2) {
    const bool ub = check_snr(x1, x2);
    auto a = batched(x1, ub), b = batched(x2, ub);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options());
    auto v1 = at::var(a, at::IntArrayRef{2}, /*unbiased=*/false).mul_(d).contiguous();  // cpu/snr_kernel.cpp:96
    check_float_dispatch(a.scalar_type(), false, "_snr_forward_cpu");
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, a.scalar_type(), "_snr_forward_cpu", [&] {
        using acc_t = std::conditional_t<std::is_same_v<scalar_t, double>, double, float>;
        const scalar_t *P = a.data_ptr<scalar_t>(), *Q = b.data_ptr<scalar_t>(), *V = v1.data_ptr<scalar_t>();
        scalar_t *O = out.data_ptr<scalar_t>();
        for_rows(B * n, [&](int64_t r) {  // cpu/snr_kernel.cpp:13-33
            const int64_t bb = r / n;
            for (int64_t j = 0; j < m; ++j) {
                acc_t mean, var;
                snr_pair_stats<acc_t>(P + r * d, Q + (bb * m + j) * d, d, mean, var);
                O[r * m + j] = (scalar_t)((acc_t)V[r] / var);
            }
        });
    });
    return unbatch(out, ub);
}

T2 snr_backward_cpu(const at::Tensor &grad, const at::Tensor &x1, const at::Tensor &x2) {
    const bool ub = x1.dim() == 2;
    auto a = batched(x1, ub), b = batched(x2, ub), g = batched(grad, ub);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto gx1 = at::zeros_like(a), gx2 = at::zeros_like(b);
    auto mu1 = a.mean(2).contiguous();
    auto v1 = at::var(a, at::IntArrayRef{2}, /*unbiased=*/false).mul_(d).contiguous();
    check_float_dispatch(g.scalar_type(), false, "_snr_backward_cpu");
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, a.scalar_type(), "_snr_backward_cpu", [&] {
        using acc_t = std::conditional_t<std::is_same_v<scalar_t, double>, double, float>;
        const scalar_t *P = a.data_ptr<scalar_t>(), *Q = b.data_ptr<scalar_t>(), *G = g.data_ptr<scalar_t>();
        const scalar_t *MU = mu1.data_ptr<scalar_t>(), *V = v1.data_ptr<scalar_t>();
        scalar_t *GX1 = gx1.data_ptr<scalar_t>(), *GX2 = gx2.data_ptr<scalar_t>();
        // cpu/snr_kernel.cpp:118-143 (x1) and 145-168 (x2)
        for_rows(B * n, [&](int64_t r) {
            const int64_t bb = r / n;
            for (int64_t j = 0; j < m; ++j) {
                const scalar_t *u = P + r * d, *v = Q + (bb * m + j) * d;
                acc_t mean, var;
                snr_pair_stats<acc_t>(u, v, d, mean, var);
                const acc_t gv = G[r * m + j];
                for (int64_t k = 0; k < d; ++k)
                    GX1[r * d + k] = (scalar_t)((acc_t)GX1[r * d + k] +
                        gv * 2 * ((-(acc_t)MU[r] + (acc_t)u[k]) + (-mean + (acc_t)v[k] - (acc_t)u[k]) * (acc_t)V[r] / var) / var);
            }
        });
        for_rows(B * m, [&](int64_t r) {
            const int64_t bb = r / m, j = r % m;
            for (int64_t i = 0; i < n; ++i) {
                const scalar_t *u = P + (bb * n + i) * d, *v = Q + r * d;
                acc_t mean, var;
                snr_pair_stats<acc_t>(u, v, d, mean, var);
                const acc_t gv = G[(bb * n + i) * m + j];
                for (int64_t k = 0; k < d; ++k)
                    GX2[r * d + k] = (scalar_t)((acc_t)GX2[r * d + k] +
                        gv * 2 * (-mean + (acc_t)v[k] - (acc_t)u[k]) * -(acc_t)V[bb * n + i] / (var * var));
            }
        });
    });
    return {unbatch(gx1, ub), unbatch(gx2, ub)};
}

// GPU composition (differentiable: autograd runs through it when called with grad mode on)
at::Tensor snr_composite(const at::Tensor &x1, const at::Tensor &x2) {
    check_snr(x1, x2);
    auto a = x1 - x1.mean(-1, true);
    auto b = x2 - x2.mean(-1, true);
    auto v1 = (a * a).sum(-1, true);
    return v1 / ppminkowski(a, b, 2);
}

// The reference's forward takes at::var of x1 before its dtype dispatch (cuda/snr_kernel.cu:
// 100-105), so integer inputs fail in at::var and bfloat16 in the dispatch; the same here.
void snr_check_cuda(const at::Tensor &x1, const at::Tensor &x2) {
    check_snr(x1, x2);
    if (!at::isFloatingType(x1.scalar_type())) (void)at::var(x1, -1, false);
    check_float_dispatch(x1.scalar_type(), false, "_snr_forward_cuda");
}

// Below autograd (the backward recomputes through the composition): for float32 the centred
// rows and the numerator are O((n + m) d), and the pairs' squared distances and the divide are
// one pass of the VALU kernel (tpw_snr_centered), which writes the output once.
at::Tensor snr_cuda(const at::Tensor &x1, const at::Tensor &x2) {
    snr_check_cuda(x1, x2);
    if (x1.scalar_type() != at::kFloat || x2.scalar_type() != at::kFloat || x1.dim() != x2.dim() ||
        (x1.dim() != 2 && x1.dim() != 3))
        return snr_composite(x1, x2);
    DeviceGuard guard(x1.device());
    auto a3 = x1.dim() == 3 ? x1 : x1.unsqueeze(0);
    auto b3 = x2.dim() == 3 ? x2 : x2.unsqueeze(0);
    if (a3.size(0) != b3.size(0)) return snr_composite(x1, x2);
    auto a = (a3 - a3.mean(-1, true)).contiguous();
    auto b = (b3 - b3.mean(-1, true)).contiguous();
    auto v1 = (a * a).sum(-1).contiguous();
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options());
    check_rc(tpw_snr_centered(a.data_ptr<float>(), b.data_ptr<float>(), v1.data_ptr<float>(), B, n, m, d,
                              out.data_ptr<float>(), current_stream()),
             "_snr");
    return x1.dim() == 3 ? out : out[0];
}

// Gradients of a GPU composition by autograd, whatever the caller's grad mode.
template <typename F>
variable_list composite_grads(F f, const at::Tensor &grad, std::vector<at::Tensor> inputs) {
    at::AutoGradMode enable(true);
    std::vector<Variable> vars;
    for (auto &t : inputs) vars.push_back(t.detach().requires_grad_(true));
    auto out = f(vars);
    return torch::autograd::grad({out}, vars, {grad}, /*retain_graph=*/false, /*create_graph=*/false,
                                 /*allow_unused=*/true);
}

T2 snr_backward_cuda(const at::Tensor &grad, const at::Tensor &x1, const at::Tensor &x2) {
    check_float_dispatch(grad.scalar_type(), false, "_snr_backward_cuda");
    auto g = composite_grads([](const std::vector<Variable> &v) { return snr_composite(v[0], v[1]); },
                             grad, {x1, x2});
    return {g[0], g[1]};
}

// ================================================================== sqmahalanobis
bool check_mahalanobis(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &VI) {
    at::CheckedFrom c = "_sqmahalanobis_forward";  // cpu/sqmahalanobis_kernel.cpp:42-60
    auto args = {at::TensorArg(x1, "x1", 1), at::TensorArg(x2, "x2", 2), at::TensorArg(VI, "VI", 3)};
    at::checkAllSameType(c, args);
    const bool ub = x1.dim() == 2;
    TORCH_CHECK(ub || x1.dim() == 3, "x1 must be 2-D (unbatched) or 3-D (batched) tensor.")
    TORCH_CHECK(ub || x2.dim() == 3, "x2 must be 2-D (unbatched) or 3-D (batched) tensor.")
    TORCH_CHECK(ub || VI.dim() == 3, "VI must be 2-D (unbatched) or 3-D (batched) tensor.")
    TORCH_CHECK(ub || (x1.size(0) == x2.size(0) && x1.size(0) == VI.size(0)),
                "batch_size of x1, x2, and VI do not match.")
    TORCH_CHECK((ub && x1.size(1) == x2.size(1) && x1.size(1) == VI.size(0)) ||
                    (!ub && x1.size(2) == x2.size(2) && x1.size(2) == VI.size(1)),
                "feature dimension of x1, x2, and VI do not match.")
    return ub;
}

at::Tensor sqmahalanobis_cpu(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &VI) {
    const bool ub = check_mahalanobis(x1, x2, VI);
    auto a = batched(x1, ub), b = batched(x2, ub), w = batched(VI, ub);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options());
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, a.scalar_type(), "_sqmahalanobis_forward_cpu", [&] {
        using acc_t = std::conditional_t<std::is_same_v<scalar_t, double>, double, float>;
        const scalar_t *P = a.data_ptr<scalar_t>(), *Q = b.data_ptr<scalar_t>(), *W = w.data_ptr<scalar_t>();
        scalar_t *O = out.data_ptr<scalar_t>();
        for_rows(B * n, [&](int64_t r) {  // cpu/sqmahalanobis_kernel.cpp:13-33
            const int64_t bb = r / n;
            for (int64_t j = 0; j < m; ++j) {
                const scalar_t *u = P + r * d, *v = Q + (bb * m + j) * d;
                acc_t val = 0;
                for (int64_t k = 0; k < d; ++k)
                    for (int64_t l = 0; l < d; ++l)
                        val += ((acc_t)u[k] - (acc_t)v[k]) * (acc_t)W[(bb * d + k) * d + l] * ((acc_t)u[l] - (acc_t)v[l]);
                O[r * m + j] = (scalar_t)val;
            }
        });
    });
    return unbatch(out, ub);
}

T3 sqmahalanobis_backward_cpu(const at::Tensor &grad, const at::Tensor &x1, const at::Tensor &x2,
                              const at::Tensor &VI) {
    const bool ub = x1.dim() == 2;
    auto a = batched(x1, ub), b = batched(x2, ub), w = batched(VI, ub), g = batched(grad, ub);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto gx1 = at::zeros_like(a), gx2 = at::zeros_like(b), gw = at::zeros_like(w);
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, a.scalar_type(), "_sqmahalanobis_backward_cpu", [&] {
        using acc_t = std::conditional_t<std::is_same_v<scalar_t, double>, double, float>;
        const scalar_t *P = a.data_ptr<scalar_t>(), *Q = b.data_ptr<scalar_t>(), *W = w.data_ptr<scalar_t>();
        const scalar_t *G = g.data_ptr<scalar_t>();
        scalar_t *GX1 = gx1.data_ptr<scalar_t>(), *GX2 = gx2.data_ptr<scalar_t>(), *GW = gw.data_ptr<scalar_t>();
        // d/dx1[k] of sum_kl d_k VI_kl d_l = sum_l (VI_kl + VI_lk) d_l (cpu/sqmahalanobis_kernel.cpp:93-139)
        for_rows(B * n, [&](int64_t r) {
            const int64_t bb = r / n;
            for (int64_t k = 0; k < d; ++k) {
                acc_t s = 0;
                for (int64_t j = 0; j < m; ++j) {
                    const scalar_t *v = Q + (bb * m + j) * d;
                    acc_t t = 0;
                    for (int64_t l = 0; l < d; ++l) {
                        const acc_t dl = (acc_t)P[r * d + l] - (acc_t)v[l];
                        t += ((acc_t)W[(bb * d + k) * d + l] + (acc_t)W[(bb * d + l) * d + k]) * dl;
                    }
                    s += (acc_t)G[r * m + j] * t;
                }
                GX1[r * d + k] = (scalar_t)s;
            }
        });
        for_rows(B * m, [&](int64_t r) {
            const int64_t bb = r / m, j = r % m;
            for (int64_t k = 0; k < d; ++k) {
                acc_t s = 0;
                for (int64_t i = 0; i < n; ++i) {
                    const scalar_t *u = P + (bb * n + i) * d;
                    acc_t t = 0;
                    for (int64_t l = 0; l < d; ++l) {
                        const acc_t dl = (acc_t)u[l] - (acc_t)Q[r * d + l];
                        t += ((acc_t)W[(bb * d + k) * d + l] + (acc_t)W[(bb * d + l) * d + k]) * dl;
                    }
                    s -= (acc_t)G[(bb * n + i) * m + j] * t;
                }
                GX2[r * d + k] = (scalar_t)s;
            }
        });
        for_rows(B * d * d, [&](int64_t r) {  // :142-164
            const int64_t bb = r / (d * d), k = (r / d) % d, l = r % d;
            acc_t s = 0;
            for (int64_t i = 0; i < n; ++i)
                for (int64_t j = 0; j < m; ++j)
                    s += (acc_t)G[(bb * n + i) * m + j] * ((acc_t)P[(bb * n + i) * d + k] - (acc_t)Q[(bb * m + j) * d + k]) *
                         ((acc_t)P[(bb * n + i) * d + l] - (acc_t)Q[(bb * m + j) * d + l]);
            GW[r] = (scalar_t)s;
        });
    });
    return {unbatch(gx1, ub), unbatch(gx2, ub), unbatch(gw, ub)};
}

// GPU: d^T VI d per pair from the difference d and the per-row projections x VI^T
// (tpw_sqmahalanobis, mahalanobis.hip).  16-bit types compute in float32, float64 in double.
at::ScalarType mahalanobis_compute_type(at::ScalarType t, const char *name = "_sqmahalanobis_forward_cuda") {
    check_float_dispatch(t, true, name);
    return t == at::kDouble ? at::kDouble : at::kFloat;
}

at::Tensor sqmahalanobis_cuda(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &VI) {
    const bool ub = check_mahalanobis(x1, x2, VI);
    DeviceGuard guard(x1.device());
    const auto dt = x1.scalar_type(), ct = mahalanobis_compute_type(dt);
    auto a = batched(x1, ub).to(ct);
    auto b = x2.is_same(x1) ? a : batched(x2, ub).to(ct);
    auto w = batched(VI, ub).to(ct);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    const int code = ct == at::kDouble ? TPW_F64 : TPW_F32;
    auto out = at::empty({B, n, m}, a.options());
    auto ws = workspace(tpw_sqmahalanobis_workspace_size(code, B, n, m, d), a);
    check_rc(tpw_sqmahalanobis(a.data_ptr(), b.data_ptr(), w.data_ptr(), code, B, n, m, d, out.data_ptr(),
                               ws.data_ptr(), current_stream()),
             "_sqmahalanobis");
    return unbatch(out.to(dt), ub);
}

// Gradients with the reference's formulas (cpu/sqmahalanobis_kernel.cpp:91-164), regrouped:
// with H1[i] = sum_j g[i,j] (x1[i] - x2[j]) and H2[j] = sum_i g[i,j] (x2[j] - x1[i]),
// grad_x1 = H1 (VI + VI^T), grad_x2 = H2 (VI + VI^T), grad_VI = x1^T H1 + x2^T H2.  H1 and H2
// are half of the sqeuclidean gradients, whose g x2 / g^T x1 products run on the matrix cores
// (tpw_sqeuclidean_backward); H (VI + VI^T) runs there too (tpw_pairwise_inner, DOT: the
// right operand is symmetric).  float64 forms the same sums with ATen products.
T3 sqmahalanobis_backward_cuda(const at::Tensor &grad, const at::Tensor &x1, const at::Tensor &x2,
                               const at::Tensor &VI) {
    const bool ub = check_mahalanobis(x1, x2, VI);
    DeviceGuard guard(x1.device());
    const auto dt = x1.scalar_type(), ct = mahalanobis_compute_type(grad.scalar_type(), "_sqmahalanobis_backward_cuda");
    auto a = batched(x1, ub).to(ct), b = batched(x2, ub).to(ct), w = batched(VI, ub).to(ct);
    auto g = batched(grad, ub).to(ct);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto S = (w + w.mT()).contiguous();
    at::Tensor H1, H2, gx1, gx2;
    if (ct == at::kFloat && n > 0 && m > 0 && d > 0) {
        void *s = current_stream();
        H1 = at::empty_like(a);
        H2 = at::empty_like(b);
        auto ws = workspace(tpw_inner_backward_workspace_size(B, n, m, d), a);
        check_rc(tpw_sqeuclidean_backward(g.data_ptr(), a.data_ptr(), b.data_ptr(), TPW_F32, B, n, m, d,
                                          H1.data_ptr(), H2.data_ptr(), ws.data_ptr(), s),
                 "__sqmahalanobis_backward");
        H1.mul_(0.5);
        H2.mul_(0.5);
        gx1 = at::empty_like(a);
        gx2 = at::empty_like(b);
        check_rc(tpw_pairwise_inner(H1.data_ptr(), S.data_ptr(), TPW_F32, B, n, d, d, nullptr, nullptr,
                                    TPW_EPI_DOT, gx1.data_ptr(), s),
                 "__sqmahalanobis_backward");
        check_rc(tpw_pairwise_inner(H2.data_ptr(), S.data_ptr(), TPW_F32, B, m, d, d, nullptr, nullptr,
                                    TPW_EPI_DOT, gx2.data_ptr(), s),
                 "__sqmahalanobis_backward");
    } else {
        H1 = a * g.sum(-1, true) - at::matmul(g, b);
        H2 = b * g.sum(-2).unsqueeze(-1) - at::matmul(g.mT(), a);
        gx1 = at::matmul(H1, S);
        gx2 = at::matmul(H2, S);
    }
    auto gw = at::matmul(a.mT(), H1) + at::matmul(b.mT(), H2);
    return {unbatch(gx1.to(dt), ub), unbatch(gx2.to(dt), ub), unbatch(gw.to(dt), ub)};
}

// ================================================================== autograd
T2 haversine_backward_op(const at::Tensor &g, const at::Tensor &x1, const at::Tensor &x2) {
    static auto op = op_handle<T2(const at::Tensor &, const at::Tensor &, const at::Tensor &)>(
        "torchpairwise::__haversine_backward");
    return op.call(g, x1, x2);
}
T2 snr_backward_op(const at::Tensor &g, const at::Tensor &x1, const at::Tensor &x2) {
    static auto op = op_handle<T2(const at::Tensor &, const at::Tensor &, const at::Tensor &)>(
        "torchpairwise::__snr_backward");
    return op.call(g, x1, x2);
}
T3 sqmahalanobis_backward_op(const at::Tensor &g, const at::Tensor &x1, const at::Tensor &x2,
                             const at::Tensor &VI) {
    static auto op = op_handle<T3(const at::Tensor &, const at::Tensor &, const at::Tensor &, const at::Tensor &)>(
        "torchpairwise::__sqmahalanobis_backward");
    return op.call(g, x1, x2, VI);
}
at::Tensor haversine_op(const at::Tensor &x1, const at::Tensor &x2) {
    static auto op = op_handle<at::Tensor(const at::Tensor &, const at::Tensor &)>("torchpairwise::_haversine");
    return op.call(x1, x2);
}
at::Tensor snr_op(const at::Tensor &x1, const at::Tensor &x2) {
    static auto op = op_handle<at::Tensor(const at::Tensor &, const at::Tensor &)>("torchpairwise::_snr");
    return op.call(x1, x2);
}
at::Tensor sqmahalanobis_op(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &VI) {
    static auto op = op_handle<at::Tensor(const at::Tensor &, const at::Tensor &, const at::Tensor &)>(
        "torchpairwise::_sqmahalanobis");
    return op.call(x1, x2, VI);
}

class HaversineFunction : public torch::autograd::Function<HaversineFunction> {
   public:
    static Variable forward(AutogradContext *ctx, const Variable &x1, const Variable &x2) {
        at::AutoDispatchBelowADInplaceOrView g;
        ctx->save_for_backward({x1, x2});
        return haversine_op(x1, x2);
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad) {
        auto s = ctx->get_saved_variables();
        auto r = haversine_backward_op(grad[0], s[0], s[1]);
        return {std::get<0>(r), std::get<1>(r)};
    }
};

class SnrFunction : public torch::autograd::Function<SnrFunction> {
   public:
    static Variable forward(AutogradContext *ctx, const Variable &x1, const Variable &x2) {
        at::AutoDispatchBelowADInplaceOrView g;
        ctx->save_for_backward({x1, x2});
        return snr_op(x1, x2);
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad) {
        auto s = ctx->get_saved_variables();
        auto r = snr_backward_op(grad[0], s[0], s[1]);
        return {std::get<0>(r), std::get<1>(r)};
    }
};

class SqMahalanobisFunction : public torch::autograd::Function<SqMahalanobisFunction> {
   public:
    static Variable forward(AutogradContext *ctx, const Variable &x1, const Variable &x2, const Variable &VI) {
        at::AutoDispatchBelowADInplaceOrView g;
        ctx->save_for_backward({x1, x2, VI});
        return sqmahalanobis_op(x1, x2, VI);
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad) {
        auto s = ctx->get_saved_variables();
        auto r = sqmahalanobis_backward_op(grad[0], s[0], s[1], s[2]);
        return {std::get<0>(r), std::get<1>(r), std::get<2>(r)};
    }
};

// GPU snr differentiates through its composition (the VALU kernel's own backward); the other
// ops, on either device, through the reference-formula backward op.
at::Tensor haversine_autograd(const at::Tensor &x1, const at::Tensor &x2) {
    return HaversineFunction::apply(x1, x2);
}
at::Tensor snr_autograd(const at::Tensor &x1, const at::Tensor &x2) {
    if (x1.is_cuda()) {
        snr_check_cuda(x1, x2);
        return snr_composite(x1, x2);
    }
    return SnrFunction::apply(x1, x2);
}
at::Tensor sqmahalanobis_autograd(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &VI) {
    return SqMahalanobisFunction::apply(x1, x2, VI);
}

}  // namespace

// public handles (the reference's functors call these internal ops)
at::Tensor haversine(const at::Tensor &x1, const at::Tensor &x2) { return haversine_op(x1, x2); }
at::Tensor snr(const at::Tensor &x1, const at::Tensor &x2) { return snr_op(x1, x2); }
at::Tensor sqmahalanobis(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &VI) {
    return sqmahalanobis_op(x1, x2, VI);
}

// schemas: csrc/ops/{haversine,snr,sqmahalanobis}.cpp:30-39
TORCH_LIBRARY_FRAGMENT(torchpairwise, m) {
    m.def("_haversine(Tensor x1, Tensor x2) -> Tensor");
    m.def("__haversine_backward(Tensor grad, Tensor x1, Tensor x2) -> (Tensor grad_x1, Tensor grad_x2)");
    m.def("_snr(Tensor x1, Tensor x2) -> Tensor");
    m.def("__snr_backward(Tensor grad, Tensor x1, Tensor x2) -> (Tensor grad_x1, Tensor grad_x2)");
    m.def("_sqmahalanobis(Tensor x1, Tensor x2, Tensor VI) -> Tensor");
    m.def("__sqmahalanobis_backward(Tensor grad, Tensor x1, Tensor x2, Tensor VI) -> (Tensor grad_x1, Tensor grad_x2, Tensor grad_VI)");
}

TORCH_LIBRARY_IMPL(torchpairwise, CPU, m) {
    m.impl("_haversine", TORCH_FN(haversine_cpu));
    m.impl("__haversine_backward", TORCH_FN(haversine_backward_cpu));
    m.impl("_snr", TORCH_FN(snr_cpu));
    m.impl("__snr_backward", TORCH_FN(snr_backward_cpu));
    m.impl("_sqmahalanobis", TORCH_FN(sqmahalanobis_cpu));
    m.impl("__sqmahalanobis_backward", TORCH_FN(sqmahalanobis_backward_cpu));
}

TORCH_LIBRARY_IMPL(torchpairwise, CUDA, m) {
    m.impl("_haversine", TORCH_FN(haversine_cuda));
    m.impl("__haversine_backward", TORCH_FN(haversine_backward_cuda));
    m.impl("_snr", TORCH_FN(snr_cuda));
    m.impl("__snr_backward", TORCH_FN(snr_backward_cuda));
    m.impl("_sqmahalanobis", TORCH_FN(sqmahalanobis_cuda));
    m.impl("__sqmahalanobis_backward", TORCH_FN(sqmahalanobis_backward_cuda));
}

TORCH_LIBRARY_IMPL(torchpairwise, Autograd, m) {
    m.impl("_haversine", TORCH_FN(haversine_autograd));
    m.impl("_snr", TORCH_FN(snr_autograd));
    m.impl("_sqmahalanobis", TORCH_FN(sqmahalanobis_autograd));
}

}  // namespace tpw_ext
