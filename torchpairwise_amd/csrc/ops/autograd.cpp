// Autograd kernels of the differentiable internal ops.  Each forward redispatches below
// autograd and saves what its backward op needs:
//   _pw_inner            -> _pw_inner_backward (the _euclidean_dist_backward formula for
//                           EUCLIDEAN, the cosine graph of pairwise_metrics.cpp:51-56,112-122)
//   _pw_kernel           -> _pw_kernel_backward (autograd of the polynomial / sigmoid composites)
//   _pw_lp               -> _pw_lp_backward (at::_cdist_backward formulas)
//   (the prf_div family's autograd functions are in prf_div.cpp)
//   _directed_hausdorff  -> __directed_hausdorff_backward, with the generator cloned so the
//                           backward replays the forward's permutations
//                           (csrc/ops/autograd/hausdorff_kernel.cpp:9-77)
#include <torch/autograd.h>

#include "tpw_common.h"

namespace tpw_ext {
namespace {

using torch::autograd::AutogradContext;
using torch::autograd::Variable;
using torch::autograd::variable_list;

class PwInnerFunction : public torch::autograd::Function<PwInnerFunction> {
   public:
    static Variable forward(AutogradContext *ctx, const Variable &x1, const Variable &x2,
                            int64_t epilogue) {
        at::AutoDispatchBelowADInplaceOrView g;
        auto out = pw_inner(x1, x2, epilogue);
        // euclidean's backward divides by the output; the cosine family's forms its weights
        // from it on the GPU (no recomputed x1 . x2^T)
        const bool cos_family = epilogue == TPW_EPI_COSINE_SIM || epilogue == TPW_EPI_COSINE_DIST ||
                                epilogue == TPW_EPI_CORRELATION;
        if (epilogue == kEuclidean || (cos_family && out.is_cuda()))
            ctx->save_for_backward({x1, x2, out});
        else
            ctx->save_for_backward({x1, x2});
        ctx->saved_data["epilogue"] = epilogue;
        return out;
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad_output) {
        auto saved = ctx->get_saved_variables();
        const int64_t epi = ctx->saved_data["epilogue"].toInt();
        at::Tensor res = saved.size() > 2 ? saved[2] : at::Tensor();
        auto grads = pw_inner_backward(grad_output[0], saved[0], saved[1], res, epi);
        return {std::get<0>(grads), std::get<1>(grads), Variable()};
    }
};

class PwKernelFunction : public torch::autograd::Function<PwKernelFunction> {
   public:
    static Variable forward(AutogradContext *ctx, const Variable &x1, const Variable &x2, int64_t kind,
                            double gamma, double coef0, int64_t degree) {
        at::AutoDispatchBelowADInplaceOrView g;
        auto out = pw_kernel(x1, x2, kind, gamma, coef0, degree);
        if (kind == TPW_KER_SIGMOID)
            ctx->save_for_backward({x1, x2, out});  // tanh's backward uses its output
        else
            ctx->save_for_backward({x1, x2});  // the polynomial's recomputes x1 . x2^T
        ctx->saved_data["kind"] = kind;
        ctx->saved_data["gamma"] = gamma;
        ctx->saved_data["coef0"] = coef0;
        ctx->saved_data["degree"] = degree;
        return out;
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad_output) {
        auto saved = ctx->get_saved_variables();
        at::Tensor res = saved.size() > 2 ? saved[2] : at::Tensor();
        auto grads = pw_kernel_backward(grad_output[0], saved[0], saved[1], res,
                                        ctx->saved_data["kind"].toInt(), ctx->saved_data["gamma"].toDouble(),
                                        ctx->saved_data["coef0"].toDouble(), ctx->saved_data["degree"].toInt());
        return {std::get<0>(grads), std::get<1>(grads), Variable(), Variable(), Variable(), Variable()};
    }
};

class PwLpFunction : public torch::autograd::Function<PwLpFunction> {
   public:
    static Variable forward(AutogradContext *ctx, const Variable &x1, const Variable &x2, double p) {
        at::AutoDispatchBelowADInplaceOrView g;
        auto out = pw_lp(x1, x2, p);
        ctx->save_for_backward({x1, x2, out});
        ctx->saved_data["p"] = p;
        return out;
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad_output) {
        auto saved = ctx->get_saved_variables();
        auto grads = pw_lp_backward(grad_output[0], saved[0], saved[1], saved[2],
                                    ctx->saved_data["p"].toDouble());
        return {std::get<0>(grads), std::get<1>(grads), Variable()};
    }
};

class DirectedHausdorffFunction : public torch::autograd::Function<DirectedHausdorffFunction> {
   public:
    static variable_list forward(AutogradContext *ctx, const Variable &x1, const Variable &x2,
                                 bool shuffle, c10::optional<at::Generator> generator) {
        at::AutoDispatchBelowADInplaceOrView g;
        ctx->saved_data["shuffle"] = shuffle;
        ctx->saved_data["generator"] =
            generator.has_value() ? c10::make_optional(generator->clone()) : generator;
        auto r = directed_hausdorff(x1, x2, shuffle, generator);
        ctx->mark_non_differentiable({std::get<1>(r), std::get<2>(r)});
        // only the output's gradient is read: no zero tensors for the index outputs
        ctx->set_materialize_grads(false);
        // The reference's backward re-runs the forward.  Without shuffling, or with a generator
        // (whose cloned state the backward replays), that re-run returns exactly this forward's
        // output and indices, so on the GPU the backward takes them from here instead of
        // scanning again; a shuffle from the default generator draws a new permutation in the
        // reference's backward and keeps the re-run.
        const bool reuse = x1.is_cuda() && (!shuffle || generator.has_value());
        ctx->saved_data["reuse"] = reuse;
        if (reuse)
            ctx->save_for_backward({x1, x2, std::get<0>(r), std::get<1>(r), std::get<2>(r)});
        else
            ctx->save_for_backward({x1, x2});
        return {std::get<0>(r), std::get<1>(r), std::get<2>(r)};
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad_output) {
        if (!grad_output[0].defined()) return {Variable(), Variable(), Variable(), Variable()};
        auto saved = ctx->get_saved_variables();
        if (ctx->saved_data["reuse"].toBool()) {
            auto grads = directed_hausdorff_backward_indexed_cuda(grad_output[0], saved[0], saved[1],
                                                                  saved[2], saved[3], saved[4]);
            return {std::get<0>(grads), std::get<1>(grads), Variable(), Variable()};
        }
        auto gen = ctx->saved_data["generator"].toOptional<at::Generator>();
        auto grads = directed_hausdorff_backward(grad_output[0], saved[0], saved[1],
                                                 ctx->saved_data["shuffle"].toBool(), gen);
        return {std::get<0>(grads), std::get<1>(grads), Variable(), Variable()};
    }
};

at::Tensor pw_kernel_autograd(const at::Tensor &x1, const at::Tensor &x2, int64_t kind, double gamma,
                              double coef0, int64_t degree) {
    return PwKernelFunction::apply(x1, x2, kind, gamma, coef0, degree);
}

at::Tensor pw_inner_autograd(const at::Tensor &x1, const at::Tensor &x2, int64_t epilogue) {
    return PwInnerFunction::apply(x1, x2, epilogue);
}

at::Tensor pw_lp_autograd(const at::Tensor &x1, const at::Tensor &x2, double p) {
    return PwLpFunction::apply(x1, x2, p);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> directed_hausdorff_autograd(
    const at::Tensor &x1, const at::Tensor &x2, bool shuffle, c10::optional<at::Generator> gen) {
    auto r = DirectedHausdorffFunction::apply(x1, x2, shuffle, gen);
    return {r[0], r[1], r[2]};
}

}  // namespace

TORCH_LIBRARY_IMPL(torchpairwise, Autograd, m) {
    m.impl("_pw_inner", TORCH_FN(pw_inner_autograd));
    m.impl("_pw_kernel", TORCH_FN(pw_kernel_autograd));
    m.impl("_pw_lp", TORCH_FN(pw_lp_autograd));
    m.impl("_directed_hausdorff", TORCH_FN(directed_hausdorff_autograd));
}

}  // namespace tpw_ext
