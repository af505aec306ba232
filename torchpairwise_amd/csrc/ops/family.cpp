// The reference's own VALU metric ops: _ppminkowski, _wminkowski, _canberra, _braycurtis,
// _additive_chi2_kernel, _sqjensenshannon and their __*_backward ops
// (csrc/ops/{ppminkowski,wminkowski,canberra,braycurtis,additive_chi2_kernel,sqjensenshannon}.cpp),
// with CPU, GPU and Autograd kernels.
//
// GPU: fp32 kernels behind the C ABI (valu_lp.hip); bfloat16 / float16 inputs are computed
// in fp32 and rounded back; float64 runs the fp64 kernels (valu_f64.hip) in double.  CPU: loops restating the reference's CPU kernels (one output per iteration,
// sequential over k), accumulating in the input type (float / double; float for the 16-bit
// types).  Autograd: saves (x1, x2[, w]) and calls __*_backward, as the reference's
// autograd kernels do (autograd/*_kernel.cpp).
#include "tpw_common.h"

#include <ATen/Parallel.h>
#include <ATen/core/dispatch/Dispatcher.h>
#include <torch/autograd.h>

#include <cmath>

namespace tpw_ext {
namespace {

// ------------------------------------------------------------------------ shape checks
// (cpu/ppminkowski_kernel.cpp:62-78 and the same block in the other three kernels)
bool check_family_shapes(const char *from, const at::Tensor &x1, const at::Tensor &x2,
                         const at::Tensor *w = nullptr) {
    at::CheckedFrom c = from;
    if (w) {
        auto args = {at::TensorArg(x1, "x1", 1), at::TensorArg(x2, "x2", 2), at::TensorArg(*w, "w", 3)};
        at::checkAllSameType(c, args);
    } else {
        auto args = {at::TensorArg(x1, "x1", 1), at::TensorArg(x2, "x2", 2)};
        at::checkAllSameType(c, args);
    }
    const bool unbatched = x1.dim() == 2;
    TORCH_CHECK(unbatched || x1.dim() == 3, "x1 must be 2-D (unbatched) or 3-D (batched) tensor.")
    TORCH_CHECK(unbatched || x2.dim() == 3, "x2 must be 2-D (unbatched) or 3-D (batched) tensor.")
    if (w) {
        TORCH_CHECK(unbatched || w->dim() == 2, "w must be 1-D (unbatched) or 2-D (batched) tensor.")
        TORCH_CHECK(unbatched || (x1.size(0) == x2.size(0) && x1.size(0) == w->size(0)),
                    "batch_size of x1, x2, and w do not match.")
        TORCH_CHECK((unbatched && x1.size(1) == x2.size(1) && x1.size(1) == w->size(0)) ||
                        (!unbatched && x1.size(2) == x2.size(2) && x1.size(1) == w->size(1)),
                    "feature dimension of x1, x2, and w do not match.")
    } else {
        TORCH_CHECK(unbatched || (x1.size(0) == x2.size(0)), "batch_size of x1 and x2 do not match.")
        TORCH_CHECK((unbatched && x1.size(1) == x2.size(1)) || (!unbatched && x1.size(2) == x2.size(2)),
                    "feature dimension of x1 and x2 do not match.")
    }
    return unbatched;
}

inline at::Tensor batched(const at::Tensor &t, bool unbatched) {
    return unbatched ? t.unsqueeze(0).contiguous() : t.contiguous();
}
inline at::Tensor unbatch(const at::Tensor &t, bool unbatched) { return unbatched ? t.squeeze(0) : t; }

// ------------------------------------------------------------------------ CPU loops
template <typename T>
inline T sgn(T v) { return (T(0) < v) - (v < T(0)); }

// f(b, i, j) for every output, parallel over (b, i) rows.
template <typename F>
void for_pairs(int64_t B, int64_t n, int64_t m, F f) {
    at::parallel_for(0, B * n, 1, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; ++r)
            for (int64_t j = 0; j < m; ++j) f(r / n, r % n, j);
    });
}

enum Fam { kPP, kW, kCanb, kBray, kChi2, kJS };

// The reference's kernel names and dtypes: the Minkowski members take bfloat16, the others
// floating types and half only (cpu/ and cuda/<op>_kernel.*).
constexpr const char *fam_name(Fam F) {
    return F == kPP ? "_ppminkowski" : F == kW ? "_wminkowski" : F == kCanb ? "_canberra"
         : F == kBray ? "_braycurtis" : F == kChi2 ? "_additive_chi2_kernel" : "_sqjensenshannon";
}
inline void fam_check_dtype(Fam F, at::ScalarType t, const char *suffix) {
    check_float_dispatch(t, F == kPP || F == kW, std::string(fam_name(F)) + suffix);
}

// rel_entr of cpu/rel_entr.h
template <typename T>
inline T rel_entr(T x, T y) {
    if (std::isnan(x)) return x;
    if (x > T(0) && y > T(0)) return x * std::log(x / y);
    if (x == T(0) && y >= T(0)) return T(0);
    return std::numeric_limits<T>::infinity();
}

// out[b,i,j] for one member, accumulating in acc_t (cpu/*_kernel.cpp forward loops).
template <Fam F, typename acc_t, typename scalar_t>
void family_forward_loop(const at::Tensor &a, const at::Tensor &bb, const at::Tensor *w, double p,
                         at::Tensor &out) {
    const int64_t B = a.size(0), n = a.size(1), m = bb.size(1), d = a.size(2);
    const scalar_t *X1 = a.data_ptr<scalar_t>(), *X2 = bb.data_ptr<scalar_t>();
    const scalar_t *W = w ? w->data_ptr<scalar_t>() : nullptr;
    scalar_t *O = out.data_ptr<scalar_t>();
    const acc_t pp = (acc_t)p;
    const bool inf = std::isinf(p), neg = p < 0;
    for_pairs(B, n, m, [&](int64_t b, int64_t i, int64_t j) {
        const scalar_t *u = X1 + (b * n + i) * d, *v = X2 + (b * m + j) * d;
        acc_t val = 0;
        if constexpr (F == kPP || F == kW) {
            if (inf) {
                for (int64_t k = 0; k < d; ++k) {
                    acc_t t = std::fabs((acc_t)u[k] - (acc_t)v[k]);
                    if constexpr (F == kW) t *= (acc_t)W[b * d + k];
                    if (k == 0 || (neg ? t < val : t > val)) val = t;
                }
            } else {
                for (int64_t k = 0; k < d; ++k) {
                    acc_t t = std::pow(std::fabs((acc_t)u[k] - (acc_t)v[k]), pp);
                    if constexpr (F == kW) t *= (acc_t)W[b * d + k];
                    val += t;
                }
                if constexpr (F == kW) val = std::pow(val, (acc_t)1 / pp);
            }
        } else if constexpr (F == kCanb) {
            for (int64_t k = 0; k < d; ++k) {
                const acc_t den = std::fabs((acc_t)u[k]) + std::fabs((acc_t)v[k]);
                if (den != 0) val += std::fabs((acc_t)u[k] - (acc_t)v[k]) / den;
            }
        } else if constexpr (F == kChi2) {  // cpu/additive_chi2_kernel.cpp:13-30
            for (int64_t k = 0; k < d; ++k) {
                const acc_t nom = (acc_t)u[k] + (acc_t)v[k];
                if (nom != 0) {
                    const acc_t den = (acc_t)u[k] - (acc_t)v[k];
                    val -= den * den / nom;
                }
            }
        } else if constexpr (F == kJS) {  // cpu/sqjensenshannon_kernel.cpp:13-30,74 (p = divisor)
            for (int64_t k = 0; k < d; ++k) {
                const acc_t mid = ((acc_t)u[k] + (acc_t)v[k]) / (acc_t)2;
                val += rel_entr((acc_t)u[k], mid) + rel_entr((acc_t)v[k], mid);
            }
            val /= (acc_t)p;
        } else {
            acc_t diff = 0, sum = 0;
            for (int64_t k = 0; k < d; ++k) {
                diff += std::fabs((acc_t)u[k] - (acc_t)v[k]);
                sum += std::fabs((acc_t)u[k] + (acc_t)v[k]);
            }
            val = diff / sum;
        }
        O[(b * n + i) * m + j] = (scalar_t)val;
    });
}

template <Fam F>
at::Tensor family_forward_cpu(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor *w,
                              double p, const char *from) {
    const bool ub = check_family_shapes(from, x1, x2, w);
    auto a = batched(x1, ub), bb = batched(x2, ub);
    at::Tensor wc = w ? batched(*w, ub) : at::Tensor();
    auto out = at::empty({a.size(0), a.size(1), bb.size(1)}, a.options());
    if ((F == kPP || F == kW) && p == 0) {
        out.fill_(a.size(2));  // ppminkowski_kernel.cpp:90-91, wminkowski_kernel.cpp:101-102
        return unbatch(out, ub);
    }
    fam_check_dtype(F, a.scalar_type(), "_forward_cpu");
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, a.scalar_type(), "family_forward", [&] {
        using acc_t = std::conditional_t<std::is_same_v<scalar_t, double>, double, float>;
        family_forward_loop<F, acc_t, scalar_t>(a, bb, w ? &wc : nullptr, p, out);
    });
    return unbatch(out, ub);
}

// Gradients by the reference's backward loops (cpu/*_kernel.cpp), deterministic: grad_x1 is
// accumulated per (b, i) row over j, grad_x2 per (b, j) row over i, grad_w per (b, k).
template <Fam F, typename acc_t, typename scalar_t>
void family_backward_loop(const at::Tensor &gc, const at::Tensor &a, const at::Tensor &bb,
                          const at::Tensor *w, double p, at::Tensor &gx1, at::Tensor &gx2,
                          at::Tensor *gw) {
    const int64_t B = a.size(0), n = a.size(1), m = bb.size(1), d = a.size(2);
    const scalar_t *G = gc.data_ptr<scalar_t>(), *X1 = a.data_ptr<scalar_t>(), *X2 = bb.data_ptr<scalar_t>();
    const scalar_t *W = w ? w->data_ptr<scalar_t>() : nullptr;
    const acc_t pp = (acc_t)p;
    const bool inf = std::isinf(p), neg = p < 0;
    // per-pair factor: 1 (pp, canberra), S^(1/p - 1) (w), (1 / ss, sd / ss^2) (bray)
    std::vector<acc_t> f1((size_t)(B * n * m)), f2(F == kBray ? (size_t)(B * n * m) : 0);
    std::vector<int64_t> kstar((F == kPP || F == kW) && inf ? (size_t)(B * n * m) : 0);
    for_pairs(B, n, m, [&](int64_t b, int64_t i, int64_t j) {
        const scalar_t *u = X1 + (b * n + i) * d, *v = X2 + (b * m + j) * d;
        const size_t at = (size_t)((b * n + i) * m + j);
        if constexpr (F == kPP || F == kW) {
            if (inf) {  // first k reaching the max (min) of w |diff|
                acc_t best = 0;
                int64_t kb = 0;
                for (int64_t k = 0; k < d; ++k) {
                    acc_t t = std::fabs((acc_t)u[k] - (acc_t)v[k]);
                    if constexpr (F == kW) t *= (acc_t)W[b * d + k];
                    if (k == 0 || (neg ? t < best : t > best)) best = t, kb = k;
                }
                kstar[at] = kb;
                f1[at] = 1;
            } else if constexpr (F == kW) {
                acc_t s = 0;
                for (int64_t k = 0; k < d; ++k)
                    s += std::pow(std::fabs((acc_t)u[k] - (acc_t)v[k]), pp) * (acc_t)W[b * d + k];
                f1[at] = std::pow(s, (acc_t)1 / pp - 1);
            } else {
                f1[at] = 1;
            }
        } else if constexpr (F == kBray) {
            acc_t sd = 0, ss = 0;
            for (int64_t k = 0; k < d; ++k) {
                sd += std::fabs((acc_t)u[k] - (acc_t)v[k]);
                ss += std::fabs((acc_t)u[k] + (acc_t)v[k]);
            }
            f1[at] = (acc_t)1 / ss;
            f2[at] = sd / ss / ss;
        } else {
            f1[at] = 1;
        }
    });
    // term of d(out)/d(own value `x`) for the pair (x, y), own sign s = +1 for x1, -1 for x2
    auto term = [&](acc_t x, acc_t y, acc_t wk, size_t at, int64_t k) -> acc_t {
        const acc_t diff = x - y;
        if constexpr (F == kPP || F == kW) {
            if (inf) return k == kstar[at] ? wk * sgn(diff) : 0;
            return std::pow(std::fabs(diff), pp - 1) * sgn(diff) * wk * f1[at] * (F == kPP ? pp : 1);
        } else if constexpr (F == kCanb) {
            const acc_t nom = std::fabs(x) + std::fabs(y);
            return sgn(diff) / nom - sgn(x) * std::fabs(diff) / nom / nom;
        } else if constexpr (F == kChi2) {  // cpu/additive_chi2_kernel.cpp:90-125
            const acc_t nom = x + y;
            return nom != 0 ? diff * diff / (nom * nom) - 2 * diff / nom : acc_t(0);
        } else if constexpr (F == kJS) {  // cpu/sqjensenshannon_kernel.cpp:92-140, before / p
            const acc_t sum = x + y, mid = sum / (acc_t)2;
            acc_t t = 0;
            if (mid > 0) {
                if (x > 0) t += (y + sum * std::log(x / mid)) / sum;
                if (y > 0) t += -y / sum;
            }
            return t;
        } else {
            return sgn(diff) * f1[at] - sgn(x + y) * f2[at];
        }
    };
    scalar_t *GX1 = gx1.data_ptr<scalar_t>(), *GX2 = gx2.data_ptr<scalar_t>();
    at::parallel_for(0, B * n, 1, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; ++r) {
            const int64_t b = r / n, i = r % n;
            for (int64_t k = 0; k < d; ++k) {
                const acc_t wk = W ? (acc_t)W[b * d + k] : (acc_t)1;
                acc_t s = 0;
                for (int64_t j = 0; j < m; ++j) {
                    const size_t at = (size_t)((b * n + i) * m + j);
                    s += (acc_t)G[at] * term((acc_t)X1[r * d + k], (acc_t)X2[(b * m + j) * d + k], wk, at, k);
                }
                GX1[r * d + k] = (scalar_t)(F == kJS ? s / pp : s);
            }
        }
    });
    at::parallel_for(0, B * m, 1, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; ++r) {
            const int64_t b = r / m, j = r % m;
            for (int64_t k = 0; k < d; ++k) {
                const acc_t wk = W ? (acc_t)W[b * d + k] : (acc_t)1;
                acc_t s = 0;
                for (int64_t i = 0; i < n; ++i) {
                    const size_t at = (size_t)((b * n + i) * m + j);
                    s += (acc_t)G[at] * term((acc_t)X2[r * d + k], (acc_t)X1[(b * n + i) * d + k], wk, at, k);
                }
                GX2[r * d + k] = (scalar_t)(F == kJS ? s / pp : s);
            }
        }
    });
    if constexpr (F == kW) {
        scalar_t *GW = gw->data_ptr<scalar_t>();
        at::parallel_for(0, B * d, 1, [&](int64_t lo, int64_t hi) {
            for (int64_t r = lo; r < hi; ++r) {
                const int64_t b = r / d, k = r % d;
                acc_t s = 0;
                for (int64_t i = 0; i < n; ++i)
                    for (int64_t j = 0; j < m; ++j) {
                        const size_t at = (size_t)((b * n + i) * m + j);
                        const acc_t diff = (acc_t)X2[(b * m + j) * d + k] - (acc_t)X1[(b * n + i) * d + k];
                        if (inf) {
                            if (k == kstar[at]) s += (acc_t)G[at] * std::fabs(diff);
                        } else {
                            s += (acc_t)G[at] * std::pow(std::fabs(diff), pp) / pp * f1[at];
                        }
                    }
                GW[r] = (scalar_t)s;
            }
        });
    }
}

template <Fam F>
std::vector<at::Tensor> family_backward_cpu(const at::Tensor &grad, const at::Tensor &x1,
                                            const at::Tensor &x2, const at::Tensor *w, double p) {
    const bool ub = x1.dim() == 2;
    auto a = batched(x1, ub), bb = batched(x2, ub), g = batched(grad, ub);
    at::Tensor wc = w ? batched(*w, ub) : at::Tensor();
    auto gx1 = at::zeros_like(a), gx2 = at::zeros_like(bb);
    at::Tensor gw = w ? at::zeros_like(wc) : at::Tensor();
    if (!((F == kPP || F == kW) && p == 0)) fam_check_dtype(F, g.scalar_type(), "_backward_cpu");
    if (!((F == kPP || F == kW) && p == 0) && a.numel() && bb.numel()) {
        AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, a.scalar_type(), "family_backward", [&] {
            using acc_t = std::conditional_t<std::is_same_v<scalar_t, double>, double, float>;
            family_backward_loop<F, acc_t, scalar_t>(g, a, bb, w ? &wc : nullptr, p, gx1, gx2, w ? &gw : nullptr);
        });
    }
    std::vector<at::Tensor> r{unbatch(gx1, ub), unbatch(gx2, ub)};
    if (w) r.push_back(unbatch(gw, ub));
    return r;
}

// ------------------------------------------------------------------------ GPU
// fp32 views of the operands (16-bit types computed in fp32); float64 takes the fp64 kernels.
at::Tensor gpu_f32(const at::Tensor &t, const char *from) {
    TORCH_CHECK(at::isFloatingType(t.scalar_type()), from, ": expected a floating-point tensor");
    return t.to(at::kFloat).contiguous();
}

constexpr int fam_code(Fam F) {
    return F == kPP ? TPW_FAM_PPMINKOWSKI : F == kW ? TPW_FAM_WMINKOWSKI : F == kCanb ? TPW_FAM_CANBERRA
         : F == kChi2 ? TPW_FAM_CHI2 : F == kJS ? TPW_FAM_JS : TPW_FAM_BRAYCURTIS;
}

// float64: the fp64 kernels (tpw_family_f64*), in double throughout, as the reference's CUDA
// kernels compute double.
template <Fam F>
at::Tensor family_forward_f64(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor *w, double p,
                              bool ub, const char *from) {
    auto a = batched(x1, ub), bb = batched(x2, ub);
    at::Tensor wc = w ? batched(*w, ub) : at::Tensor();
    const int64_t B = a.size(0), n = a.size(1), m = bb.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options());
    check_rc(tpw_family_f64(fam_code(F), a.data_ptr<double>(), bb.data_ptr<double>(),
                            w ? wc.data_ptr<double>() : nullptr, B, n, m, d, p, out.data_ptr<double>(),
                            current_stream()),
             from);
    return unbatch(out, ub);
}

template <Fam F>
std::vector<at::Tensor> family_backward_f64(const at::Tensor &grad, const at::Tensor &x1, const at::Tensor &x2,
                                            const at::Tensor *w, double p, bool ub, const char *from) {
    auto a = batched(x1, ub), bb = batched(x2, ub), g = batched(grad.to(at::kDouble), ub);
    at::Tensor wc = w ? batched(*w, ub) : at::Tensor();
    const int64_t B = a.size(0), n = a.size(1), m = bb.size(1), d = a.size(2);
    auto gx1 = at::empty_like(a), gx2 = at::empty_like(bb);
    at::Tensor gw = w ? at::empty_like(wc) : at::Tensor();
    auto ws = workspace(tpw_family_f64_backward_workspace_size(fam_code(F), B, n, m, d, p), a);
    check_rc(tpw_family_f64_backward(fam_code(F), g.data_ptr<double>(), a.data_ptr<double>(), bb.data_ptr<double>(),
                                     w ? wc.data_ptr<double>() : nullptr, B, n, m, d, p, gx1.data_ptr<double>(),
                                     gx2.data_ptr<double>(), w ? gw.data_ptr<double>() : nullptr, ws.data_ptr(),
                                     current_stream()),
             from);
    std::vector<at::Tensor> r{unbatch(gx1, ub), unbatch(gx2, ub)};
    if (w) r.push_back(unbatch(gw, ub));
    return r;
}

template <Fam F>
at::Tensor family_forward_cuda(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor *w,
                               double p, const char *from) {
    const bool ub = check_family_shapes(from, x1, x2, w);
    DeviceGuard guard(x1.device());
    if (!((F == kPP || F == kW) && p == 0)) fam_check_dtype(F, x1.scalar_type(), "_forward_cuda");
    if (x1.scalar_type() == at::kDouble) return family_forward_f64<F>(x1, x2, w, p, ub, from);
    auto a = batched(gpu_f32(x1, from), ub), bb = batched(gpu_f32(x2, from), ub);
    at::Tensor wc = w ? batched(gpu_f32(*w, from), ub) : at::Tensor();
    const int64_t B = a.size(0), n = a.size(1), m = bb.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options());
    const float *A = a.data_ptr<float>(), *Bp = bb.data_ptr<float>();
    float *O = out.data_ptr<float>();
    void *s = current_stream();
    int rc;
    if constexpr (F == kPP) rc = tpw_ppminkowski(A, Bp, B, n, m, d, p, O, s);
    else if constexpr (F == kW) rc = tpw_wminkowski(A, Bp, wc.data_ptr<float>(), B, n, m, d, p, O, s);
    else if constexpr (F == kCanb) rc = tpw_canberra(A, Bp, B, n, m, d, O, s);
    else if constexpr (F == kChi2) rc = tpw_additive_chi2(A, Bp, B, n, m, d, O, s);
    else if constexpr (F == kJS) rc = tpw_sqjensenshannon(A, Bp, B, n, m, d, p, O, s);
    else rc = tpw_braycurtis(A, Bp, B, n, m, d, O, s);
    check_rc(rc, from);
    return unbatch(out, ub).to(x1.scalar_type());
}

template <Fam F>
std::vector<at::Tensor> family_backward_cuda(const at::Tensor &grad, const at::Tensor &x1,
                                             const at::Tensor &x2, const at::Tensor *w, double p,
                                             const at::Tensor *out_in, const char *from) {
    const bool ub = x1.dim() == 2;
    DeviceGuard guard(x1.device());
    if (!((F == kPP || F == kW) && p == 0)) fam_check_dtype(F, grad.scalar_type(), "_backward_cuda");
    if (x1.scalar_type() == at::kDouble) return family_backward_f64<F>(grad, x1, x2, w, p, ub, from);
    auto a = batched(gpu_f32(x1, from), ub), bb = batched(gpu_f32(x2, from), ub);
    auto g = batched(gpu_f32(grad, from), ub);
    at::Tensor wc = w ? batched(gpu_f32(*w, from), ub) : at::Tensor();
    const int64_t B = a.size(0), n = a.size(1), m = bb.size(1), d = a.size(2);
    auto gx1 = at::empty_like(a), gx2 = at::empty_like(bb);
    at::Tensor gw = w ? at::empty_like(wc) : at::Tensor();
    // the forward result (recomputed, as the reference's backward does, unless given)
    at::Tensor out;
    if (F == kW || F == kBray) {
        if (out_in) {
            out = batched(out_in->to(at::kFloat), ub);
        } else {
            out = at::empty({B, n, m}, a.options());
            const int rc = F == kW ? tpw_wminkowski(a.data_ptr<float>(), bb.data_ptr<float>(), wc.data_ptr<float>(),
                                                    B, n, m, d, p, out.data_ptr<float>(), current_stream())
                                   : tpw_braycurtis(a.data_ptr<float>(), bb.data_ptr<float>(), B, n, m, d,
                                                    out.data_ptr<float>(), current_stream());
            check_rc(rc, from);
        }
    }
    const int metric = fam_code(F);
    auto ws = workspace(tpw_family_backward_workspace_size(metric, B, n, m, d), a);
    const float *G = g.data_ptr<float>(), *A = a.data_ptr<float>(), *Bp = bb.data_ptr<float>();
    void *s = current_stream();
    int rc;
    if constexpr (F == kPP)
        rc = tpw_ppminkowski_backward(G, A, Bp, B, n, m, d, p, gx1.data_ptr<float>(), gx2.data_ptr<float>(),
                                      ws.data_ptr(), s);
    else if constexpr (F == kW)
        rc = tpw_wminkowski_backward(G, A, Bp, wc.data_ptr<float>(), out.data_ptr<float>(), B, n, m, d, p,
                                     gx1.data_ptr<float>(), gx2.data_ptr<float>(), gw.data_ptr<float>(),
                                     ws.data_ptr(), s);
    else if constexpr (F == kCanb)
        rc = tpw_canberra_backward(G, A, Bp, B, n, m, d, gx1.data_ptr<float>(), gx2.data_ptr<float>(),
                                   ws.data_ptr(), s);
    else if constexpr (F == kChi2)
        rc = tpw_additive_chi2_backward(G, A, Bp, B, n, m, d, gx1.data_ptr<float>(), gx2.data_ptr<float>(),
                                        ws.data_ptr(), s);
    else if constexpr (F == kJS)
        rc = tpw_sqjensenshannon_backward(G, A, Bp, B, n, m, d, p, gx1.data_ptr<float>(),
                                          gx2.data_ptr<float>(), ws.data_ptr(), s);
    else
        rc = tpw_braycurtis_backward(G, A, Bp, out.data_ptr<float>(), B, n, m, d, gx1.data_ptr<float>(),
                                     gx2.data_ptr<float>(), ws.data_ptr(), s);
    check_rc(rc, from);
    std::vector<at::Tensor> r{unbatch(gx1, ub).to(x1.scalar_type()), unbatch(gx2, ub).to(x2.scalar_type())};
    if (w) r.push_back(unbatch(gw, ub).to(w->scalar_type()));
    return r;
}

// ------------------------------------------------------------------------ op kernels
at::Tensor ppminkowski_cpu(const at::Tensor &x1, const at::Tensor &x2, double p) {
    return family_forward_cpu<kPP>(x1, x2, nullptr, p, "_ppminkowski_forward");
}
at::Tensor ppminkowski_cuda(const at::Tensor &x1, const at::Tensor &x2, double p) {
    return family_forward_cuda<kPP>(x1, x2, nullptr, p, "_ppminkowski_forward");
}
std::tuple<at::Tensor, at::Tensor> ppminkowski_backward_cpu(const at::Tensor &g, const at::Tensor &x1,
                                                            const at::Tensor &x2, double p) {
    auto r = family_backward_cpu<kPP>(g, x1, x2, nullptr, p);
    return {r[0], r[1]};
}
std::tuple<at::Tensor, at::Tensor> ppminkowski_backward_cuda(const at::Tensor &g, const at::Tensor &x1,
                                                             const at::Tensor &x2, double p) {
    auto r = family_backward_cuda<kPP>(g, x1, x2, nullptr, p, nullptr, "_ppminkowski_backward");
    return {r[0], r[1]};
}

at::Tensor wminkowski_cpu(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &w, double p) {
    return family_forward_cpu<kW>(x1, x2, &w, p, "_wminkowski_forward");
}
at::Tensor wminkowski_cuda(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &w, double p) {
    return family_forward_cuda<kW>(x1, x2, &w, p, "_wminkowski_forward");
}
std::tuple<at::Tensor, at::Tensor, at::Tensor> wminkowski_backward_cpu(
    const at::Tensor &g, const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &w, double p) {
    auto r = family_backward_cpu<kW>(g, x1, x2, &w, p);
    return {r[0], r[1], r[2]};
}
std::tuple<at::Tensor, at::Tensor, at::Tensor> wminkowski_backward_cuda(
    const at::Tensor &g, const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &w, double p) {
    auto r = family_backward_cuda<kW>(g, x1, x2, &w, p, nullptr, "_wminkowski_backward");
    return {r[0], r[1], r[2]};
}

at::Tensor canberra_cpu(const at::Tensor &x1, const at::Tensor &x2) {
    return family_forward_cpu<kCanb>(x1, x2, nullptr, 1.0, "_canberra_forward");
}
at::Tensor canberra_cuda(const at::Tensor &x1, const at::Tensor &x2) {
    return family_forward_cuda<kCanb>(x1, x2, nullptr, 1.0, "_canberra_forward");
}
std::tuple<at::Tensor, at::Tensor> canberra_backward_cpu(const at::Tensor &g, const at::Tensor &x1,
                                                         const at::Tensor &x2) {
    auto r = family_backward_cpu<kCanb>(g, x1, x2, nullptr, 1.0);
    return {r[0], r[1]};
}
std::tuple<at::Tensor, at::Tensor> canberra_backward_cuda(const at::Tensor &g, const at::Tensor &x1,
                                                          const at::Tensor &x2) {
    auto r = family_backward_cuda<kCanb>(g, x1, x2, nullptr, 1.0, nullptr, "_canberra_backward");
    return {r[0], r[1]};
}

at::Tensor braycurtis_cpu(const at::Tensor &x1, const at::Tensor &x2) {
    return family_forward_cpu<kBray>(x1, x2, nullptr, 1.0, "_braycurtis_forward");
}
at::Tensor braycurtis_cuda(const at::Tensor &x1, const at::Tensor &x2) {
    return family_forward_cuda<kBray>(x1, x2, nullptr, 1.0, "_braycurtis_forward");
}
std::tuple<at::Tensor, at::Tensor> braycurtis_backward_cpu(const at::Tensor &g, const at::Tensor &x1,
                                                           const at::Tensor &x2) {
    auto r = family_backward_cpu<kBray>(g, x1, x2, nullptr, 1.0);
    return {r[0], r[1]};
}
std::tuple<at::Tensor, at::Tensor> braycurtis_backward_cuda(const at::Tensor &g, const at::Tensor &x1,
                                                            const at::Tensor &x2) {
    auto r = family_backward_cuda<kBray>(g, x1, x2, nullptr, 1.0, nullptr, "_braycurtis_backward");
    return {r[0], r[1]};
}

// the divisor of _sqjensenshannon: 2, or 2 ln(base) (cpu/sqjensenshannon_kernel.cpp:74)
double js_divisor(c10::optional<double> base) { return base.has_value() ? 2 * std::log(base.value()) : 2.0; }

at::Tensor chi2_cpu(const at::Tensor &x1, const at::Tensor &x2) {
    return family_forward_cpu<kChi2>(x1, x2, nullptr, 1.0, "_additive_chi2_kernel_forward");
}
at::Tensor chi2_cuda(const at::Tensor &x1, const at::Tensor &x2) {
    return family_forward_cuda<kChi2>(x1, x2, nullptr, 1.0, "_additive_chi2_kernel_forward");
}
std::tuple<at::Tensor, at::Tensor> chi2_backward_cpu(const at::Tensor &g, const at::Tensor &x1,
                                                     const at::Tensor &x2) {
    auto r = family_backward_cpu<kChi2>(g, x1, x2, nullptr, 1.0);
    return {r[0], r[1]};
}
std::tuple<at::Tensor, at::Tensor> chi2_backward_cuda(const at::Tensor &g, const at::Tensor &x1,
                                                      const at::Tensor &x2) {
    auto r = family_backward_cuda<kChi2>(g, x1, x2, nullptr, 1.0, nullptr, "_additive_chi2_kernel_backward");
    return {r[0], r[1]};
}

at::Tensor js_cpu(const at::Tensor &x1, const at::Tensor &x2, c10::optional<double> base) {
    return family_forward_cpu<kJS>(x1, x2, nullptr, js_divisor(base), "_sqjensenshannon_forward");
}
at::Tensor js_cuda(const at::Tensor &x1, const at::Tensor &x2, c10::optional<double> base) {
    return family_forward_cuda<kJS>(x1, x2, nullptr, js_divisor(base), "_sqjensenshannon_forward");
}
std::tuple<at::Tensor, at::Tensor> js_backward_cpu(const at::Tensor &g, const at::Tensor &x1,
                                                   const at::Tensor &x2, c10::optional<double> base) {
    auto r = family_backward_cpu<kJS>(g, x1, x2, nullptr, js_divisor(base));
    return {r[0], r[1]};
}
std::tuple<at::Tensor, at::Tensor> js_backward_cuda(const at::Tensor &g, const at::Tensor &x1,
                                                    const at::Tensor &x2, c10::optional<double> base) {
    auto r = family_backward_cuda<kJS>(g, x1, x2, nullptr, js_divisor(base), nullptr, "_sqjensenshannon_backward");
    return {r[0], r[1]};
}

// rbf_kernel / laplacian_kernel (pairwise_metrics.cpp:92-110): exp(-gamma * distance) with the
// exponential in the VALU kernel's epilogue (sqeuclidean = _ppminkowski p = 2; cdist p = 1).
at::Tensor exp_kernel_cuda(const at::Tensor &x1, const at::Tensor &x2, int64_t kind, double gamma) {
    const char *from = "_pw_exp_kernel";
    TORCH_CHECK(kind == TPW_KER_RBF || kind == TPW_KER_LAPLACIAN, from, ": unknown kernel ", kind);
    const bool ub = check_family_shapes(from, x1, x2, nullptr);
    DeviceGuard guard(x1.device());
    TORCH_CHECK_NOT_IMPLEMENTED(x1.scalar_type() != at::kDouble, from,
                                ": float64 takes the distance op and ATen's exp (rbf_kernel and "
                                "laplacian_kernel route it there)");
    auto a = batched(gpu_f32(x1, from), ub), bb = batched(gpu_f32(x2, from), ub);
    const int64_t B = a.size(0), n = a.size(1), m = bb.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options());
    check_rc(tpw_pairwise_exp_kernel(a.data_ptr<float>(), bb.data_ptr<float>(), B, n, m, d, (int)kind,
                                     (float)gamma, out.data_ptr<float>(), current_stream()),
             from);
    return unbatch(out, ub).to(x1.scalar_type());
}

// Gradients of exp_kernel_cuda's out for fp32 operands: the pair gradient (grad * out) * -gamma
// formed inside the backward kernel (rbf) or in one elementwise pass (laplacian) by
// tpw_pairwise_exp_kernel_backward, instead of two ATen passes.
std::tuple<at::Tensor, at::Tensor> exp_kernel_backward_cuda(const at::Tensor &grad, const at::Tensor &x1,
                                                            const at::Tensor &x2, const at::Tensor &out,
                                                            int64_t kind, double gamma) {
    const char *from = "_pw_exp_kernel_backward";
    const bool ub = check_family_shapes(from, x1, x2, nullptr);
    DeviceGuard guard(x1.device());
    auto a = batched(gpu_f32(x1, from), ub), bb = batched(gpu_f32(x2, from), ub);
    const int64_t B = a.size(0), n = a.size(1), m = bb.size(1), d = a.size(2);
    auto g = grad.to(at::kFloat).reshape({B, n, m}).contiguous();
    auto o = out.to(at::kFloat).reshape({B, n, m}).contiguous();
    auto gx1 = at::empty_like(a), gx2 = at::empty_like(bb);
    auto ws = workspace(tpw_pairwise_exp_kernel_backward_workspace_size((int)kind, B, n, m, d), a);
    check_rc(tpw_pairwise_exp_kernel_backward(g.data_ptr<float>(), o.data_ptr<float>(), a.data_ptr<float>(),
                                              bb.data_ptr<float>(), B, n, m, d, (int)kind, (float)gamma,
                                              gx1.data_ptr<float>(), gx2.data_ptr<float>(), ws.data_ptr(),
                                              current_stream()),
             from);
    return {unbatch(gx1, ub), unbatch(gx2, ub)};
}

// ------------------------------------------------------------------------ dispatcher handles
template <typename Sig>
c10::TypedOperatorHandle<Sig> op_handle(const char *name) {
    return c10::Dispatcher::singleton().findSchemaOrThrow(name, "").typed<Sig>();
}
using T2 = std::tuple<at::Tensor, at::Tensor>;
using T3 = std::tuple<at::Tensor, at::Tensor, at::Tensor>;

T2 ppminkowski_backward_op(const at::Tensor &g, const at::Tensor &x1, const at::Tensor &x2, double p) {
    static auto op = op_handle<T2(const at::Tensor &, const at::Tensor &, const at::Tensor &, double)>(
        "torchpairwise::__ppminkowski_backward");
    return op.call(g, x1, x2, p);
}
T3 wminkowski_backward_op(const at::Tensor &g, const at::Tensor &x1, const at::Tensor &x2,
                          const at::Tensor &w, double p) {
    static auto op = op_handle<T3(const at::Tensor &, const at::Tensor &, const at::Tensor &,
                                  const at::Tensor &, double)>("torchpairwise::__wminkowski_backward");
    return op.call(g, x1, x2, w, p);
}
T2 canberra_backward_op(const at::Tensor &g, const at::Tensor &x1, const at::Tensor &x2) {
    static auto op = op_handle<T2(const at::Tensor &, const at::Tensor &, const at::Tensor &)>(
        "torchpairwise::__canberra_backward");
    return op.call(g, x1, x2);
}
T2 braycurtis_backward_op(const at::Tensor &g, const at::Tensor &x1, const at::Tensor &x2) {
    static auto op = op_handle<T2(const at::Tensor &, const at::Tensor &, const at::Tensor &)>(
        "torchpairwise::__braycurtis_backward");
    return op.call(g, x1, x2);
}

T2 chi2_backward_op(const at::Tensor &g, const at::Tensor &x1, const at::Tensor &x2) {
    static auto op = op_handle<T2(const at::Tensor &, const at::Tensor &, const at::Tensor &)>(
        "torchpairwise::__additive_chi2_kernel_backward");
    return op.call(g, x1, x2);
}
T2 js_backward_op(const at::Tensor &g, const at::Tensor &x1, const at::Tensor &x2, c10::optional<double> base) {
    static auto op = op_handle<T2(const at::Tensor &, const at::Tensor &, const at::Tensor &,
                                  c10::optional<double>)>("torchpairwise::__sqjensenshannon_backward");
    return op.call(g, x1, x2, base);
}

// ------------------------------------------------------------------------ autograd
using torch::autograd::AutogradContext;
using torch::autograd::Variable;
using torch::autograd::variable_list;

class PPMinkowskiFunction : public torch::autograd::Function<PPMinkowskiFunction> {
   public:
    static Variable forward(AutogradContext *ctx, const Variable &x1, const Variable &x2, double p) {
        at::AutoDispatchBelowADInplaceOrView g;
        ctx->save_for_backward({x1, x2});
        ctx->saved_data["p"] = p;
        return ppminkowski(x1, x2, p);
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad) {
        auto s = ctx->get_saved_variables();
        auto r = ppminkowski_backward_op(grad[0], s[0], s[1], ctx->saved_data["p"].toDouble());
        return {std::get<0>(r), std::get<1>(r), Variable()};
    }
};

class WMinkowskiFunction : public torch::autograd::Function<WMinkowskiFunction> {
   public:
    static Variable forward(AutogradContext *ctx, const Variable &x1, const Variable &x2,
                            const Variable &w, double p) {
        at::AutoDispatchBelowADInplaceOrView g;
        ctx->save_for_backward({x1, x2, w});
        ctx->saved_data["p"] = p;
        return wminkowski(x1, x2, w, p);
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad) {
        auto s = ctx->get_saved_variables();
        auto r = wminkowski_backward_op(grad[0], s[0], s[1], s[2], ctx->saved_data["p"].toDouble());
        return {std::get<0>(r), std::get<1>(r), std::get<2>(r), Variable()};
    }
};

template <at::Tensor (*FWD)(const at::Tensor &, const at::Tensor &),
          T2 (*BWD)(const at::Tensor &, const at::Tensor &, const at::Tensor &)>
class PairFunction : public torch::autograd::Function<PairFunction<FWD, BWD>> {
   public:
    static Variable forward(AutogradContext *ctx, const Variable &x1, const Variable &x2) {
        at::AutoDispatchBelowADInplaceOrView g;
        ctx->save_for_backward({x1, x2});
        return FWD(x1, x2);
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad) {
        auto s = ctx->get_saved_variables();
        auto r = BWD(grad[0], s[0], s[1]);
        return {std::get<0>(r), std::get<1>(r)};
    }
};

class JSFunction : public torch::autograd::Function<JSFunction> {
   public:
    static Variable forward(AutogradContext *ctx, const Variable &x1, const Variable &x2,
                            c10::optional<double> base) {
        at::AutoDispatchBelowADInplaceOrView g;
        ctx->save_for_backward({x1, x2});
        ctx->saved_data["has_base"] = base.has_value();
        ctx->saved_data["base"] = base.value_or(0.0);
        return sqjensenshannon(x1, x2, base);
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad) {
        auto s = ctx->get_saved_variables();
        c10::optional<double> base;
        if (ctx->saved_data["has_base"].toBool()) base = ctx->saved_data["base"].toDouble();
        auto r = js_backward_op(grad[0], s[0], s[1], base);
        return {std::get<0>(r), std::get<1>(r), Variable()};
    }
};

// The reference's composite differentiated: exp_'s backward grad * out, mul_'s * (-gamma),
// then the distance's own backward (_ppminkowski p = 2, or cdist p = 1, which does not read
// its distance argument).
class ExpKernelFunction : public torch::autograd::Function<ExpKernelFunction> {
   public:
    static Variable forward(AutogradContext *ctx, const Variable &x1, const Variable &x2, int64_t kind,
                            double gamma) {
        at::AutoDispatchBelowADInplaceOrView g;
        auto out = pw_exp_kernel(x1, x2, kind, gamma);
        ctx->save_for_backward({x1, x2, out});
        ctx->saved_data["kind"] = kind;
        ctx->saved_data["gamma"] = gamma;
        return out;
    }
    static variable_list backward(AutogradContext *ctx, const variable_list &grad) {
        auto s = ctx->get_saved_variables();
        const double gamma = ctx->saved_data["gamma"].toDouble();
        if (s[0].is_cuda() && s[0].scalar_type() == at::kFloat && s[1].scalar_type() == at::kFloat &&
            grad[0].scalar_type() == at::kFloat) {
            // fp32 on the GPU: (grad * out) * -gamma inside the C entry point, the same two
            // roundings as the composite below
            auto r = exp_kernel_backward_cuda(grad[0], s[0], s[1], s[2], ctx->saved_data["kind"].toInt(), gamma);
            return {std::get<0>(r), std::get<1>(r), Variable(), Variable()};
        }
        auto gf = grad[0].mul(s[2]).mul(-gamma);
        if (ctx->saved_data["kind"].toInt() == TPW_KER_RBF) {
            T2 r = ppminkowski_backward_op(gf, s[0], s[1], 2.0);  // 16-bit types via fp32 inside
            return {std::get<0>(r), std::get<1>(r), Variable(), Variable()};
        }
        // the L1 backward kernel is fp32 (as cdist's route converts 16-bit operands)
        const auto f = at::kFloat;
        T2 r = pw_lp_backward(gf.to(f), s[0].to(f), s[1].to(f), s[2].to(f), 1.0);
        return {std::get<0>(r).to(s[0].scalar_type()), std::get<1>(r).to(s[1].scalar_type()), Variable(),
                Variable()};
    }
};

at::Tensor exp_kernel_autograd(const at::Tensor &x1, const at::Tensor &x2, int64_t kind, double gamma) {
    return ExpKernelFunction::apply(x1, x2, kind, gamma);
}

at::Tensor ppminkowski_autograd(const at::Tensor &x1, const at::Tensor &x2, double p) {
    return PPMinkowskiFunction::apply(x1, x2, p);
}
at::Tensor wminkowski_autograd(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &w, double p) {
    return WMinkowskiFunction::apply(x1, x2, w, p);
}
at::Tensor canberra_autograd(const at::Tensor &x1, const at::Tensor &x2) {
    return PairFunction<canberra, canberra_backward_op>::apply(x1, x2);
}
at::Tensor braycurtis_autograd(const at::Tensor &x1, const at::Tensor &x2) {
    return PairFunction<braycurtis, braycurtis_backward_op>::apply(x1, x2);
}
at::Tensor chi2_autograd(const at::Tensor &x1, const at::Tensor &x2) {
    return PairFunction<additive_chi2, chi2_backward_op>::apply(x1, x2);
}
at::Tensor js_autograd(const at::Tensor &x1, const at::Tensor &x2, c10::optional<double> base) {
    return JSFunction::apply(x1, x2, base);
}

}  // namespace

// ------------------------------------------------------------------------ public handles
at::Tensor ppminkowski(const at::Tensor &x1, const at::Tensor &x2, double p) {
    static auto op = op_handle<at::Tensor(const at::Tensor &, const at::Tensor &, double)>(
        "torchpairwise::_ppminkowski");
    return op.call(x1, x2, p);
}
at::Tensor wminkowski(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &w, double p) {
    static auto op = op_handle<at::Tensor(const at::Tensor &, const at::Tensor &, const at::Tensor &, double)>(
        "torchpairwise::_wminkowski");
    return op.call(x1, x2, w, p);
}
at::Tensor canberra(const at::Tensor &x1, const at::Tensor &x2) {
    static auto op = op_handle<at::Tensor(const at::Tensor &, const at::Tensor &)>("torchpairwise::_canberra");
    return op.call(x1, x2);
}
at::Tensor braycurtis(const at::Tensor &x1, const at::Tensor &x2) {
    static auto op = op_handle<at::Tensor(const at::Tensor &, const at::Tensor &)>("torchpairwise::_braycurtis");
    return op.call(x1, x2);
}
at::Tensor additive_chi2(const at::Tensor &x1, const at::Tensor &x2) {
    static auto op = op_handle<at::Tensor(const at::Tensor &, const at::Tensor &)>(
        "torchpairwise::_additive_chi2_kernel");
    return op.call(x1, x2);
}
at::Tensor pw_exp_kernel(const at::Tensor &x1, const at::Tensor &x2, int64_t kind, double gamma) {
    static auto op = op_handle<at::Tensor(const at::Tensor &, const at::Tensor &, int64_t, double)>(
        "torchpairwise::_pw_exp_kernel");
    return op.call(x1, x2, kind, gamma);
}
at::Tensor sqjensenshannon(const at::Tensor &x1, const at::Tensor &x2, c10::optional<double> base) {
    static auto op = op_handle<at::Tensor(const at::Tensor &, const at::Tensor &, c10::optional<double>)>(
        "torchpairwise::_sqjensenshannon");
    return op.call(x1, x2, base);
}

// schemas: csrc/ops/{ppminkowski,wminkowski,canberra,braycurtis,additive_chi2_kernel,
// sqjensenshannon}.cpp:30-39
TORCH_LIBRARY_FRAGMENT(torchpairwise, m) {
    m.def("_ppminkowski(Tensor x1, Tensor x2, float p=2) -> Tensor");
    m.def("__ppminkowski_backward(Tensor grad, Tensor x1, Tensor x2, float p) -> (Tensor grad_x1, Tensor grad_x2)");
    m.def("_wminkowski(Tensor x1, Tensor x2, Tensor w, float p=2) -> Tensor");
    m.def("__wminkowski_backward(Tensor grad, Tensor x1, Tensor x2, Tensor w, float p) -> (Tensor grad_x1, Tensor grad_x2, Tensor grad_w)");
    m.def("_canberra(Tensor x1, Tensor x2) -> Tensor");
    m.def("__canberra_backward(Tensor grad, Tensor x1, Tensor x2) -> (Tensor grad_x1, Tensor grad_x2)");
    m.def("_braycurtis(Tensor x1, Tensor x2) -> Tensor");
    m.def("__braycurtis_backward(Tensor grad, Tensor x1, Tensor x2) -> (Tensor grad_x1, Tensor grad_x2)");
    m.def("_additive_chi2_kernel(Tensor x1, Tensor x2) -> Tensor");
    m.def("__additive_chi2_kernel_backward(Tensor grad, Tensor x1, Tensor x2) -> (Tensor grad_x1, Tensor grad_x2)");
    m.def("_sqjensenshannon(Tensor x1, Tensor x2, float? base=None) -> Tensor");
    m.def("__sqjensenshannon_backward(Tensor grad, Tensor x1, Tensor x2, float? base) -> (Tensor grad_x1, Tensor grad_x2)");
    // this build's fused rbf / laplacian (no counterpart schema in the reference)
    m.def("_pw_exp_kernel(Tensor x1, Tensor x2, int kind, float gamma) -> Tensor");
}

TORCH_LIBRARY_IMPL(torchpairwise, CPU, m) {
    m.impl("_ppminkowski", TORCH_FN(ppminkowski_cpu));
    m.impl("__ppminkowski_backward", TORCH_FN(ppminkowski_backward_cpu));
    m.impl("_wminkowski", TORCH_FN(wminkowski_cpu));
    m.impl("__wminkowski_backward", TORCH_FN(wminkowski_backward_cpu));
    m.impl("_canberra", TORCH_FN(canberra_cpu));
    m.impl("__canberra_backward", TORCH_FN(canberra_backward_cpu));
    m.impl("_braycurtis", TORCH_FN(braycurtis_cpu));
    m.impl("__braycurtis_backward", TORCH_FN(braycurtis_backward_cpu));
    m.impl("_additive_chi2_kernel", TORCH_FN(chi2_cpu));
    m.impl("__additive_chi2_kernel_backward", TORCH_FN(chi2_backward_cpu));
    m.impl("_sqjensenshannon", TORCH_FN(js_cpu));
    m.impl("__sqjensenshannon_backward", TORCH_FN(js_backward_cpu));
}

TORCH_LIBRARY_IMPL(torchpairwise, CUDA, m) {
    m.impl("_ppminkowski", TORCH_FN(ppminkowski_cuda));
    m.impl("__ppminkowski_backward", TORCH_FN(ppminkowski_backward_cuda));
    m.impl("_wminkowski", TORCH_FN(wminkowski_cuda));
    m.impl("__wminkowski_backward", TORCH_FN(wminkowski_backward_cuda));
    m.impl("_canberra", TORCH_FN(canberra_cuda));
    m.impl("__canberra_backward", TORCH_FN(canberra_backward_cuda));
    m.impl("_braycurtis", TORCH_FN(braycurtis_cuda));
    m.impl("__braycurtis_backward", TORCH_FN(braycurtis_backward_cuda));
    m.impl("_additive_chi2_kernel", TORCH_FN(chi2_cuda));
    m.impl("__additive_chi2_kernel_backward", TORCH_FN(chi2_backward_cuda));
    m.impl("_sqjensenshannon", TORCH_FN(js_cuda));
    m.impl("__sqjensenshannon_backward", TORCH_FN(js_backward_cuda));
    m.impl("_pw_exp_kernel", TORCH_FN(exp_kernel_cuda));
}

TORCH_LIBRARY_IMPL(torchpairwise, Autograd, m) {
    m.impl("_ppminkowski", TORCH_FN(ppminkowski_autograd));
    m.impl("_wminkowski", TORCH_FN(wminkowski_autograd));
    m.impl("_canberra", TORCH_FN(canberra_autograd));
    m.impl("_braycurtis", TORCH_FN(braycurtis_autograd));
    m.impl("_additive_chi2_kernel", TORCH_FN(chi2_autograd));
    m.impl("_sqjensenshannon", TORCH_FN(js_autograd));
    m.impl("_pw_exp_kernel", TORCH_FN(exp_kernel_autograd));
}

}  // namespace tpw_ext
