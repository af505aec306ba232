// The prf_div family ("pseudo-reciprocal-free" divide): the 20 schemas of
// csrc/ops/prf_div.cpp:359-400 — prf_div / prf_ldiv over (Tensor, Tensor), (Tensor, Scalar),
// (Scalar, Tensor), their in-place forms and the ten backward ops — with the reference's
// semantics (csrc/ops/cpu/prf_div_kernel.cpp, csrc/ops/autograd/prf_div_kernel.cpp):
//
//   prf_divide(x, y) = y != 0 ? x / y : (mode "zero": 0 | "identity": x)   (cpu/prf_divide.h)
//   prf_ldiv(a, b) = prf_divide(b, a)  (left division)
//
// * no broadcasting: tensor operands must have the same shape (the reference's message);
// * the result type is at::result_type of the operands, integral (and bool) -> float32;
// * the in-place forms check at::can_cast(result, self) and write into self;
// * backward reads grad, self and other as grad's element type (their flatten() views, as the
//   reference does, so operands of another dtype raise there too);
// * the in-place autograd functions save `self` after the write, so their backward sees the
//   quotient as `self` — the reference's behaviour (autograd/prf_div_kernel.cpp:275-...),
//   kept so gradients match it.
//
// One function per op serves both devices: the elementwise step runs a CPU loop for CPU
// tensors and the HIP kernels of the C ABI (tpw_prf_div*, elementwise.hip) for GPU tensors.
#include "tpw_common.h"

#include <ATen/Dispatch.h>
#include <ATen/core/dispatch/Dispatcher.h>
#include <ATen/Parallel.h>
#include <ATen/TensorUtils.h>
#include <torch/autograd.h>

namespace tpw_ext {
namespace {

using torch::autograd::AutogradContext;
using torch::autograd::Variable;
using torch::autograd::variable_list;

at::ScalarType prf_result_type(at::ScalarType t) {
    return at::isIntegralType(t, /*includeBool=*/true) ? at::kFloat : t;
}

void check_same_shape(const char *name, const at::Tensor &self, const at::Tensor &other) {
    TORCH_CHECK(self.sizes() == other.sizes(), "Broadcasting semantic is not implemented for ", name,
                ". Expect self's shape to be identical to other's shape. Got self.shape=", self.sizes(),
                ", while other.shape=", other.sizes())
}

void check_same_gpu(const char *name, const at::Tensor &self, const at::Tensor &other) {
    if (self.is_cuda() || other.is_cuda())
        at::checkAllSameGPU(name, {at::TensorArg(self, "self", 1), at::TensorArg(other, "other", 2)});
}

template <typename T>
inline T prf_divide(T x, T y, bool identity) {
    return y != T(0) ? T(x / y) : (identity ? x : T(0));
}

template <typename F>
void cpu_loop(int64_t n, F f) {
    at::parallel_for(0, n, 16384, [&](int64_t beg, int64_t end) {
        for (int64_t i = beg; i < end; ++i) f(i);
    });
}

// out[i] = prf_divide(num[i], den[i]); all three contiguous, of dtype `t`; out may alias.
void run_tt(const at::Tensor &num, const at::Tensor &den, at::Tensor &out, bool identity) {
    const int64_t n = out.numel();
    if (out.is_cuda()) {
        DeviceGuard guard(out.device());
        check_rc(tpw_prf_div(num.data_ptr(), den.data_ptr(), float_code(out.scalar_type()), n, identity,
                             out.data_ptr(), current_stream()),
                 "prf_div");
        return;
    }
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, out.scalar_type(), "prf_div", [&] {
        const scalar_t *X = num.data_ptr<scalar_t>(), *Y = den.data_ptr<scalar_t>();
        scalar_t *O = out.data_ptr<scalar_t>();
        cpu_loop(n, [&](int64_t i) { O[i] = prf_divide<scalar_t>(X[i], Y[i], identity); });
    });
}

// scalar_first ? out[i] = prf_divide(c, x[i]) : out[i] = prf_divide(x[i], c)
template <typename scalar_t>
void run_ts(const at::Tensor &x, scalar_t c, at::Tensor &out, bool identity, bool scalar_first) {
    const int64_t n = out.numel();
    if (out.is_cuda()) {
        DeviceGuard guard(out.device());
        check_rc(tpw_prf_div_scalar(x.data_ptr(), static_cast<double>(c), float_code(out.scalar_type()), n,
                                    identity, scalar_first, out.data_ptr(), current_stream()),
                 "prf_div");
        return;
    }
    const scalar_t *X = x.data_ptr<scalar_t>();
    scalar_t *O = out.data_ptr<scalar_t>();
    if (scalar_first) {
        cpu_loop(n, [&](int64_t i) { O[i] = prf_divide<scalar_t>(c, X[i], identity); });
    } else if (c == scalar_t(0)) {
        cpu_loop(n, [&](int64_t i) { O[i] = identity ? X[i] : scalar_t(0); });
    } else {
        cpu_loop(n, [&](int64_t i) { O[i] = X[i] / c; });
    }
}

// ------------------------------------------------------------------------------- forward
// prf_div / prf_ldiv (cpu/prf_div_kernel.cpp:57-103)
template <bool left>
at::Tensor prf_div_tt(const at::Tensor &self, const at::Tensor &other, c10::string_view mode) {
    check_same_gpu("prf_div_forward_kernel", self, other);
    check_same_shape("prf_div", self, other);
    const auto rt = prf_result_type(at::result_type(self, other));
    auto self_c = self.contiguous().to(rt), other_c = other.contiguous().to(rt);
    auto out = at::empty_like(self_c);
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, rt, "prf_div", [&] {
        const bool identity = prf_identity(mode);
        left ? run_tt(other_c, self_c, out, identity) : run_tt(self_c, other_c, out, identity);
    });
    return out;
}

// prf_div.Scalar / prf_ldiv.Scalar (cpu/prf_div_kernel.cpp:105-142)
template <bool left>
at::Tensor prf_div_ts(const at::Tensor &self, const at::Scalar &other, c10::string_view mode) {
    const auto rt = prf_result_type(at::result_type(self, other));
    auto self_c = self.contiguous().to(rt);
    auto out = at::empty_like(self_c);
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, rt, "prf_div_Scalar", [&] {
        const bool identity = prf_identity(mode);
        run_ts<scalar_t>(self_c, other.to<scalar_t>(), out, identity, left);
    });
    return out;
}

// prf_div.rScalar / prf_ldiv.rScalar = the Scalar form with the roles swapped
// (cpu/prf_div_kernel.cpp:144-150)
template <bool left>
at::Tensor prf_div_st(const at::Scalar &self, const at::Tensor &other, c10::string_view mode) {
    return prf_div_ts<!left>(other, self, mode);
}

void check_castable(at::ScalarType rt, const at::Tensor &self) {
    TORCH_CHECK(at::can_cast(rt, self.scalar_type()), "result type ", rt,
                " can't be cast to the desired output type ", self.scalar_type())
}

// prf_div_ / prf_ldiv_ (cpu/prf_div_kernel.cpp:152-207)
template <bool left>
at::Tensor prf_div_inplace_tt(at::Tensor &self, const at::Tensor &other, c10::string_view mode) {
    check_same_gpu("prf_div__forward_kernel", self, other);
    check_same_shape("prf_div_", self, other);
    const auto rt = prf_result_type(at::result_type(self, other));
    check_castable(rt, self);
    auto self_c = self.contiguous().to(rt), other_c = other.contiguous().to(rt);
    const bool needs_cast = !self.is_contiguous() || rt != self.scalar_type();
    auto out = needs_cast ? at::empty_like(self_c) : self_c;  // else self_c is self
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, rt, "prf_div_", [&] {
        const bool identity = prf_identity(mode);
        left ? run_tt(other_c, self_c, out, identity) : run_tt(self_c, other_c, out, identity);
    });
    if (needs_cast) self.copy_(out);
    return self;
}

// prf_div_.Scalar / prf_ldiv_.Scalar (cpu/prf_div_kernel.cpp:209-255)
template <bool left>
at::Tensor prf_div_inplace_ts(at::Tensor &self, const at::Scalar &other, c10::string_view mode) {
    const auto rt = prf_result_type(at::result_type(self, other));
    check_castable(rt, self);
    auto self_c = self.contiguous().to(rt);
    const bool needs_cast = !self.is_contiguous();
    auto out = needs_cast ? at::empty_like(self_c) : self_c;
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, rt, "prf_div__Scalar", [&] {
        const bool identity = prf_identity(mode);
        run_ts<scalar_t>(self_c, other.to<scalar_t>(), out, identity, left);
    });
    if (needs_cast) self.copy_(out);
    return self;
}

// ------------------------------------------------------------------------------ backward
void check_numel(const at::Tensor &grad, const at::Tensor &t) {
    TORCH_CHECK(grad.numel() == t.numel(), "prf_div backward: grad has ", grad.numel(),
                " elements, the operand ", t.numel())
}

// _prf_div_backward / _prf_ldiv_backward and their in-place twins
// (cpu/prf_div_kernel.cpp:257-278,314-360).  Not left (z = self / other): o = other;
// left (z = other / self): o = self, with the two gradients' roles swapped.
template <bool left>
std::tuple<at::Tensor, at::Tensor> prf_div_backward_tt(const at::Tensor &grad, const at::Tensor &self,
                                                       const at::Tensor &other, c10::string_view mode) {
    check_same_gpu("prf_div_backward_kernel", self, other);
    check_numel(grad, self);
    check_numel(grad, other);
    const auto rt = grad.scalar_type();
    auto self_c = self.contiguous().to(rt), other_c = other.contiguous().to(rt);
    auto grad_self = at::zeros_like(self_c), grad_other = at::zeros_like(other_c);
    auto g = grad.flatten(), s = self.flatten(), o = other.flatten();
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, rt, "prf_div_backward", [&] {
        const bool identity = prf_identity(mode);
        const scalar_t *G = g.data_ptr<scalar_t>(), *S = s.data_ptr<scalar_t>(), *O = o.data_ptr<scalar_t>();
        // x = the dividend, y = the divisor of z = x / y
        const scalar_t *X = left ? O : S, *Y = left ? S : O;
        at::Tensor &gx = left ? grad_other : grad_self, &gy = left ? grad_self : grad_other;
        const int64_t n = g.numel();
        if (grad.is_cuda()) {
            DeviceGuard guard(grad.device());
            check_rc(tpw_prf_div_backward(G, X, Y, float_code(rt), n, identity, gx.data_ptr(), gy.data_ptr(),
                                          current_stream()),
                     "prf_div backward");
            return;
        }
        scalar_t *GX = gx.data_ptr<scalar_t>(), *GY = gy.data_ptr<scalar_t>();
        cpu_loop(n, [&](int64_t i) {
            const scalar_t y = Y[i];
            if (y != scalar_t(0)) {
                const scalar_t gs = G[i] / y;
                GX[i] = gs;
                GY[i] = scalar_t(gs * -X[i]) / y;
            } else if (identity) {
                GX[i] = G[i];
            }
        });
    });
    return {grad_self.to(self.scalar_type()), grad_other.to(other.scalar_type())};
}

// grad_x of z = x / c (scalar_first = false) or z = c / x (true), into grad_x
// (cpu/prf_div_kernel.cpp:279-311)
template <typename scalar_t>
void run_scalar_backward(const at::Tensor &g, const at::Tensor &x, scalar_t c, bool identity,
                         bool scalar_first, at::Tensor &grad_x) {
    const int64_t n = g.numel();
    if (g.is_cuda()) {
        DeviceGuard guard(g.device());
        check_rc(tpw_prf_div_scalar_backward(g.data_ptr(), scalar_first ? x.data_ptr() : nullptr,
                                             static_cast<double>(c), float_code(g.scalar_type()), n, identity,
                                             scalar_first, grad_x.data_ptr(), current_stream()),
                 "prf_div backward");
        return;
    }
    const scalar_t *G = g.data_ptr<scalar_t>();
    scalar_t *GX = grad_x.data_ptr<scalar_t>();
    if (scalar_first) {
        const scalar_t *X = x.data_ptr<scalar_t>();
        cpu_loop(n, [&](int64_t i) {
            const scalar_t o = X[i];
            if (o != scalar_t(0)) GX[i] = scalar_t(G[i] * -c) / scalar_t(o * o);
        });
    } else if (c != scalar_t(0)) {
        cpu_loop(n, [&](int64_t i) { GX[i] = G[i] / c; });
    } else if (identity) {
        cpu_loop(n, [&](int64_t i) { GX[i] = G[i]; });
    }
}

// _prf_div_backward.Scalar / _prf_ldiv_backward.Scalar and the in-place twins
// (cpu/prf_div_kernel.cpp:362-401)
template <bool left>
at::Tensor prf_div_backward_ts(const at::Tensor &grad, const at::Tensor &self, const at::Scalar &other,
                               c10::string_view mode) {
    check_numel(grad, self);
    const auto rt = grad.scalar_type();
    auto self_c = self.contiguous().to(rt);
    auto grad_self = at::zeros_like(self_c);
    auto g = grad.flatten(), s = self.flatten();
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, rt, "prf_div_Scalar_backward", [&] {
        const bool identity = prf_identity(mode);
        if (left) (void)s.data_ptr<scalar_t>();
        run_scalar_backward<scalar_t>(g, s, other.to<scalar_t>(), identity, left, grad_self);
    });
    return grad_self.to(self.scalar_type());
}

// _prf_div_backward.rScalar / _prf_ldiv_backward.rScalar (cpu/prf_div_kernel.cpp:403-442)
template <bool left>
at::Tensor prf_div_backward_st(const at::Tensor &grad, const at::Scalar &self, const at::Tensor &other,
                               c10::string_view mode) {
    check_numel(grad, other);
    const auto rt = grad.scalar_type();
    auto other_c = other.contiguous().to(rt);
    auto grad_other = at::zeros_like(other_c);
    auto g = grad.flatten(), o = other.flatten();
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, rt, "prf_div_rScalar_backward", [&] {
        const bool identity = prf_identity(mode);
        if (!left) (void)o.data_ptr<scalar_t>();
        // prf_div.rScalar: z = s / other (the scalar is the dividend); prf_ldiv.rScalar: other / s
        run_scalar_backward<scalar_t>(g, o, self.to<scalar_t>(), identity, !left, grad_other);
    });
    return grad_other.to(other.scalar_type());
}

// ------------------------------------------------------------------ dispatcher handles
template <typename Sig>
c10::TypedOperatorHandle<Sig> op_handle(const char *name, const char *overload) {
    return c10::Dispatcher::singleton().findSchemaOrThrow(name, overload).typed<Sig>();
}

using TTSig = at::Tensor(const at::Tensor &, const at::Tensor &, c10::string_view);
using TSSig = at::Tensor(const at::Tensor &, const at::Scalar &, c10::string_view);
using STSig = at::Tensor(const at::Scalar &, const at::Tensor &, c10::string_view);
using ITTSig = at::Tensor(at::Tensor &, const at::Tensor &, c10::string_view);
using ITSSig = at::Tensor(at::Tensor &, const at::Scalar &, c10::string_view);
using BTTSig = std::tuple<at::Tensor, at::Tensor>(const at::Tensor &, const at::Tensor &, const at::Tensor &,
                                                  c10::string_view);
using BTSSig = at::Tensor(const at::Tensor &, const at::Tensor &, const at::Scalar &, c10::string_view);
using BSTSig = at::Tensor(const at::Tensor &, const at::Scalar &, const at::Tensor &, c10::string_view);

// ------------------------------------------------------------------------------ autograd
// The ten autograd functions of csrc/ops/autograd/prf_div_kernel.cpp:9-454: each saves what
// the reference saves and calls the reference's backward op through the dispatcher.
template <bool left>
struct PrfDivTT : public torch::autograd::Function<PrfDivTT<left>> {
    static Variable forward(AutogradContext *ctx, const Variable &self, const Variable &other,
                            c10::string_view mode) {
        at::AutoDispatchBelowADInplaceOrView g;
        static auto op = op_handle<TTSig>(left ? "torchpairwise::prf_ldiv" : "torchpairwise::prf_div", "");
        auto out = op.call(self, other, mode);
        ctx->save_for_backward({self, other});
        ctx->saved_data["mode"] = std::string(mode);
        return out;
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad_output) {
        static auto op = op_handle<BTTSig>(left ? "torchpairwise::_prf_ldiv_backward"
                                                : "torchpairwise::_prf_div_backward", "");
        auto saved = ctx->get_saved_variables();
        auto grads = op.call(grad_output[0], saved[0], saved[1], ctx->saved_data["mode"].toStringRef());
        return {std::get<0>(grads), std::get<1>(grads), Variable()};
    }
};

template <bool left>
struct PrfDivTS : public torch::autograd::Function<PrfDivTS<left>> {
    static Variable forward(AutogradContext *ctx, const Variable &self, const at::Scalar &other,
                            c10::string_view mode) {
        at::AutoDispatchBelowADInplaceOrView g;
        static auto op = op_handle<TSSig>(left ? "torchpairwise::prf_ldiv" : "torchpairwise::prf_div", "Scalar");
        auto out = op.call(self, other, mode);
        ctx->save_for_backward({self});
        ctx->saved_data["other"] = other;
        ctx->saved_data["mode"] = std::string(mode);
        return out;
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad_output) {
        static auto op = op_handle<BTSSig>(left ? "torchpairwise::_prf_ldiv_backward"
                                                : "torchpairwise::_prf_div_backward", "Scalar");
        auto saved = ctx->get_saved_variables();
        auto gs = op.call(grad_output[0], saved[0], ctx->saved_data["other"].toScalar(),
                          ctx->saved_data["mode"].toStringRef());
        return {gs, Variable(), Variable()};
    }
};

template <bool left>
struct PrfDivST : public torch::autograd::Function<PrfDivST<left>> {
    static Variable forward(AutogradContext *ctx, const at::Scalar &self, const Variable &other,
                            c10::string_view mode) {
        at::AutoDispatchBelowADInplaceOrView g;
        static auto op = op_handle<STSig>(left ? "torchpairwise::prf_ldiv" : "torchpairwise::prf_div", "rScalar");
        auto out = op.call(self, other, mode);
        ctx->save_for_backward({other});
        ctx->saved_data["self"] = self;
        ctx->saved_data["mode"] = std::string(mode);
        return out;
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad_output) {
        static auto op = op_handle<BSTSig>(left ? "torchpairwise::_prf_ldiv_backward"
                                                : "torchpairwise::_prf_div_backward", "rScalar");
        auto saved = ctx->get_saved_variables();
        auto go = op.call(grad_output[0], ctx->saved_data["self"].toScalar(), saved[0],
                          ctx->saved_data["mode"].toStringRef());
        return {Variable(), go, Variable()};
    }
};

// In place: `self` is saved after the write (it is the op's output then), as the reference
// does, so the backward reads the quotient as `self`.
template <bool left>
struct PrfDivInplaceTT : public torch::autograd::Function<PrfDivInplaceTT<left>> {
    static Variable forward(AutogradContext *ctx, Variable &self, const Variable &other, c10::string_view mode) {
        at::AutoDispatchBelowADInplaceOrView g;
        ctx->mark_dirty({self});
        static auto op = op_handle<ITTSig>(left ? "torchpairwise::prf_ldiv_" : "torchpairwise::prf_div_", "");
        auto out = op.call(self, other, mode);
        ctx->save_for_backward({self, other});
        ctx->saved_data["mode"] = std::string(mode);
        return out;
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad_output) {
        static auto op = op_handle<BTTSig>(left ? "torchpairwise::_prf_ldiv__backward"
                                                : "torchpairwise::_prf_div__backward", "");
        auto saved = ctx->get_saved_variables();
        auto grads = op.call(grad_output[0], saved[0], saved[1], ctx->saved_data["mode"].toStringRef());
        return {std::get<0>(grads), std::get<1>(grads), Variable()};
    }
};

template <bool left>
struct PrfDivInplaceTS : public torch::autograd::Function<PrfDivInplaceTS<left>> {
    static Variable forward(AutogradContext *ctx, Variable &self, const at::Scalar &other, c10::string_view mode) {
        at::AutoDispatchBelowADInplaceOrView g;
        ctx->mark_dirty({self});
        static auto op = op_handle<ITSSig>(left ? "torchpairwise::prf_ldiv_" : "torchpairwise::prf_div_", "Scalar");
        auto out = op.call(self, other, mode);
        ctx->save_for_backward({self});
        ctx->saved_data["other"] = other;
        ctx->saved_data["mode"] = std::string(mode);
        return out;
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad_output) {
        static auto op = op_handle<BTSSig>(left ? "torchpairwise::_prf_ldiv__backward"
                                                : "torchpairwise::_prf_div__backward", "Scalar");
        auto saved = ctx->get_saved_variables();
        auto gs = op.call(grad_output[0], saved[0], ctx->saved_data["other"].toScalar(),
                          ctx->saved_data["mode"].toStringRef());
        return {gs, Variable(), Variable()};
    }
};

template <bool left>
at::Tensor tt_autograd(const at::Tensor &self, const at::Tensor &other, c10::string_view mode) {
    return PrfDivTT<left>::apply(self, other, mode);
}
template <bool left>
at::Tensor ts_autograd(const at::Tensor &self, const at::Scalar &other, c10::string_view mode) {
    return PrfDivTS<left>::apply(self, other, mode);
}
template <bool left>
at::Tensor st_autograd(const at::Scalar &self, const at::Tensor &other, c10::string_view mode) {
    return PrfDivST<left>::apply(self, other, mode);
}
template <bool left>
at::Tensor inplace_tt_autograd(at::Tensor &self, const at::Tensor &other, c10::string_view mode) {
    return PrfDivInplaceTT<left>::apply(self, other, mode);
}
template <bool left>
at::Tensor inplace_ts_autograd(at::Tensor &self, const at::Scalar &other, c10::string_view mode) {
    return PrfDivInplaceTS<left>::apply(self, other, mode);
}

void register_impls(torch::Library &m) {
    m.impl("prf_div", TORCH_FN(prf_div_tt<false>));
    m.impl("prf_ldiv", TORCH_FN(prf_div_tt<true>));
    m.impl("prf_div.Scalar", TORCH_FN(prf_div_ts<false>));
    m.impl("prf_ldiv.Scalar", TORCH_FN(prf_div_ts<true>));
    m.impl("prf_div.rScalar", TORCH_FN(prf_div_st<false>));
    m.impl("prf_ldiv.rScalar", TORCH_FN(prf_div_st<true>));
    m.impl("prf_div_", TORCH_FN(prf_div_inplace_tt<false>));
    m.impl("prf_ldiv_", TORCH_FN(prf_div_inplace_tt<true>));
    m.impl("prf_div_.Scalar", TORCH_FN(prf_div_inplace_ts<false>));
    m.impl("prf_ldiv_.Scalar", TORCH_FN(prf_div_inplace_ts<true>));
    m.impl("_prf_div_backward", TORCH_FN(prf_div_backward_tt<false>));
    m.impl("_prf_ldiv_backward", TORCH_FN(prf_div_backward_tt<true>));
    m.impl("_prf_div_backward.Scalar", TORCH_FN(prf_div_backward_ts<false>));
    m.impl("_prf_ldiv_backward.Scalar", TORCH_FN(prf_div_backward_ts<true>));
    m.impl("_prf_div_backward.rScalar", TORCH_FN(prf_div_backward_st<false>));
    m.impl("_prf_ldiv_backward.rScalar", TORCH_FN(prf_div_backward_st<true>));
    m.impl("_prf_div__backward", TORCH_FN(prf_div_backward_tt<false>));
    m.impl("_prf_ldiv__backward", TORCH_FN(prf_div_backward_tt<true>));
    m.impl("_prf_div__backward.Scalar", TORCH_FN(prf_div_backward_ts<false>));
    m.impl("_prf_ldiv__backward.Scalar", TORCH_FN(prf_div_backward_ts<true>));
}

}  // namespace

at::Tensor prf_div_cpu(const at::Tensor &x, const at::Tensor &y, c10::string_view mode) {
    return prf_div_tt<false>(x, y, mode);
}

// csrc/ops/prf_div.cpp:359-400, byte for byte
TORCH_LIBRARY_FRAGMENT(torchpairwise, m) {
    m.def("prf_div(Tensor input, Tensor other, str mode=\"zero\") -> Tensor");
    m.def("prf_ldiv(Tensor input, Tensor other, str mode=\"zero\") -> Tensor");
    m.def("prf_div.Scalar(Tensor input, Scalar other, str mode=\"zero\") -> Tensor");
    m.def("prf_ldiv.Scalar(Tensor input, Scalar other, str mode=\"zero\") -> Tensor");
    m.def("prf_div.rScalar(Scalar input, Tensor other, str mode=\"zero\") -> Tensor");
    m.def("prf_ldiv.rScalar(Scalar input, Tensor other, str mode=\"zero\") -> Tensor");
    m.def("prf_div_(Tensor(a!) input, Tensor other, str mode=\"zero\") -> Tensor(a!)");
    m.def("prf_ldiv_(Tensor(a!) input, Tensor other, str mode=\"zero\") -> Tensor(a!)");
    m.def("prf_div_.Scalar(Tensor(a!) input, Scalar other, str mode=\"zero\") -> Tensor(a!)");
    m.def("prf_ldiv_.Scalar(Tensor(a!) input, Scalar other, str mode=\"zero\") -> Tensor(a!)");
    m.def("_prf_div_backward(Tensor grad, Tensor self, Tensor other, str mode=\"zero\") -> (Tensor grad_self, Tensor grad_other)");
    m.def("_prf_ldiv_backward(Tensor grad, Tensor self, Tensor other, str mode=\"zero\") -> (Tensor grad_self, Tensor grad_other)");
    m.def("_prf_div_backward.Scalar(Tensor grad, Tensor self, Scalar other, str mode=\"zero\") -> Tensor grad_self");
    m.def("_prf_ldiv_backward.Scalar(Tensor grad, Tensor self, Scalar other, str mode=\"zero\") -> Tensor grad_self");
    m.def("_prf_div_backward.rScalar(Tensor grad, Scalar self, Tensor other, str mode=\"zero\") -> Tensor grad_other");
    m.def("_prf_ldiv_backward.rScalar(Tensor grad, Scalar self, Tensor other, str mode=\"zero\") -> Tensor grad_other");
    m.def("_prf_div__backward(Tensor grad, Tensor self, Tensor other, str mode=\"zero\") -> (Tensor grad_self, Tensor grad_other)");
    m.def("_prf_ldiv__backward(Tensor grad, Tensor self, Tensor other, str mode=\"zero\") -> (Tensor grad_self, Tensor grad_other)");
    m.def("_prf_div__backward.Scalar(Tensor grad, Tensor self, Scalar other, str mode=\"zero\") -> Tensor grad_self");
    m.def("_prf_ldiv__backward.Scalar(Tensor grad, Tensor self, Scalar other, str mode=\"zero\") -> Tensor grad_self");
}

TORCH_LIBRARY_IMPL(torchpairwise, CPU, m) { register_impls(m); }
TORCH_LIBRARY_IMPL(torchpairwise, CUDA, m) { register_impls(m); }

TORCH_LIBRARY_IMPL(torchpairwise, Autograd, m) {
    m.impl("prf_div", TORCH_FN(tt_autograd<false>));
    m.impl("prf_ldiv", TORCH_FN(tt_autograd<true>));
    m.impl("prf_div.Scalar", TORCH_FN(ts_autograd<false>));
    m.impl("prf_ldiv.Scalar", TORCH_FN(ts_autograd<true>));
    m.impl("prf_div.rScalar", TORCH_FN(st_autograd<false>));
    m.impl("prf_ldiv.rScalar", TORCH_FN(st_autograd<true>));
    m.impl("prf_div_", TORCH_FN(inplace_tt_autograd<false>));
    m.impl("prf_ldiv_", TORCH_FN(inplace_tt_autograd<true>));
    m.impl("prf_div_.Scalar", TORCH_FN(inplace_ts_autograd<false>));
    m.impl("prf_ldiv_.Scalar", TORCH_FN(inplace_ts_autograd<true>));
}

}  // namespace tpw_ext
