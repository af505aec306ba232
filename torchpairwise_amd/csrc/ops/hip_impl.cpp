// GPU (DispatchKey::CUDA, which PyTorch-ROCm uses for HIP tensors) implementations of the
// internal ops: shape/dtype checks, output allocation from the caching allocator, then one
// call into the C ABI (include/torchpairwise_amd.h) on the current HIP stream.  There is no
// other route: a missing kernel library fails at load time, unsupported dtypes raise.
#include "tpw_common.h"

namespace tpw_ext {
namespace {

void check_cuda_pair(const char *name, const at::Tensor &x1, const at::Tensor &x2) {
    TORCH_CHECK(x1.is_cuda() && x2.is_cuda(), name, ": expected GPU tensors");
    TORCH_CHECK(x1.get_device() == x2.get_device(), name, ": x1 and x2 are on different devices");
    TORCH_CHECK(x1.dim() == x2.dim() && (x1.dim() == 2 || x1.dim() == 3), name,
                ": x1 and x2 must both be 2-D or both 3-D");
    TORCH_CHECK(x1.size(-1) == x2.size(-1), name, ": feature dimension of x1 and x2 do not match.");
    TORCH_CHECK(x1.dim() == 2 || x1.size(0) == x2.size(0), name, ": batch_size of x1 and x2 do not match.");
}

int float_dtype(const char *name, const at::Tensor &x) {
    TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kBFloat16, name,
                ": supports float32 and bfloat16 on the GPU, got ", x.scalar_type());
    return x.scalar_type() == at::kFloat ? TPW_F32 : TPW_BF16;
}

at::Tensor out_shape(const at::Tensor &out3, const at::Tensor &x1) {
    return x1.dim() == 2 ? out3.squeeze(0) : out3;
}

// ---------------------------------------------------------------- inner-product (MFMA)
// radius_neighbors_mask's euclidean route: the mask straight from the MFMA epilogue (x1, x2 of
// equal batch, fp32 or bf16); epsilon compared as the inputs' dtype holds it, as Tensor.le does.
at::Tensor radius_mask_euclidean_cuda(const at::Tensor &x1, const at::Tensor &x2, double epsilon) {
    check_cuda_pair("_radius_mask_euclidean", x1, x2);
    TORCH_CHECK(x1.scalar_type() == x2.scalar_type(), "_radius_mask_euclidean: x1 and x2 dtypes differ");
    const int dt = float_dtype("_radius_mask_euclidean", x1);
    DeviceGuard guard(x1.device());
    auto a = as3(x1), b = as3(x2);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options().dtype(at::kBool));
    void *s = current_stream();
    auto n1 = at::empty({B, n}, a.options().dtype(at::kFloat));
    check_rc(tpw_row_norms(a.data_ptr(), dt, B * n, d, 1, n1.data_ptr<float>(), s), "row norms");
    at::Tensor n2 = n1;
    if (!x2.is_same(x1)) {
        n2 = at::empty({B, m}, a.options().dtype(at::kFloat));
        check_rc(tpw_row_norms(b.data_ptr(), dt, B * m, d, 1, n2.data_ptr<float>(), s), "row norms");
    }
    const float eps = x1.scalar_type() == at::kBFloat16 ? static_cast<float>(c10::BFloat16(static_cast<float>(epsilon)))
                                                         : static_cast<float>(epsilon);
    check_rc(tpw_radius_mask_euclidean(a.data_ptr(), b.data_ptr(), dt, B, n, m, d, n1.data_ptr<float>(),
                                       n2.data_ptr<float>(), eps, reinterpret_cast<uint8_t *>(out.data_ptr<bool>()), s),
             "_radius_mask_euclidean");
    return out_shape(out, x1);
}

// k_neighbors_mask (euclidean) without the distance matrix: the tile kernel's per-tile candidates
// and a select pass (tpw_knn_mask_euclidean); the same mask as the distances followed by
// _row_smallest_mask.
at::Tensor knn_mask_euclidean_cuda(const at::Tensor &x1, const at::Tensor &x2, int64_t count) {
    check_cuda_pair("_knn_mask_euclidean", x1, x2);
    TORCH_CHECK(x1.dim() == 2 && x2.dim() == 2, "_knn_mask_euclidean: expected 2-D inputs");
    TORCH_CHECK(x1.scalar_type() == x2.scalar_type(), "_knn_mask_euclidean: x1 and x2 dtypes differ");
    const int dt = float_dtype("_knn_mask_euclidean", x1);
    DeviceGuard guard(x1.device());
    auto a = x1.contiguous(), b = x2.contiguous();
    const int64_t n = a.size(0), m = b.size(0), d = a.size(1);
    TORCH_CHECK(tpw_knn_mask_euclidean_supported(dt, n, m, d, count),
                "_knn_mask_euclidean: unsupported sizes (n ", n, ", m ", m, ", d ", d, ", count ", count, ")");
    auto mask = at::empty({n, m}, a.options().dtype(at::kBool));
    void *s = current_stream();
    auto n1 = at::empty({n}, a.options().dtype(at::kFloat));
    check_rc(tpw_row_norms(a.data_ptr(), dt, n, d, 1, n1.data_ptr<float>(), s), "row norms");
    at::Tensor n2 = n1;
    if (!x2.is_same(x1)) {
        n2 = at::empty({m}, a.options().dtype(at::kFloat));
        check_rc(tpw_row_norms(b.data_ptr(), dt, m, d, 1, n2.data_ptr<float>(), s), "row norms");
    }
    auto ws = workspace(tpw_knn_mask_workspace_size(n, m, count), a);
    check_rc(tpw_knn_mask_euclidean(a.data_ptr(), b.data_ptr(), dt, n, m, d, n1.data_ptr<float>(), n2.data_ptr<float>(),
                                    count, reinterpret_cast<uint8_t *>(mask.data_ptr<bool>()), ws.data_ptr(), s),
             "_knn_mask_euclidean");
    return mask;
}

at::Tensor pw_inner_cuda(const at::Tensor &x1, const at::Tensor &x2, int64_t epilogue) {
    check_cuda_pair("_pw_inner", x1, x2);
    TORCH_CHECK(x1.scalar_type() == x2.scalar_type(), "_pw_inner: x1 and x2 dtypes differ");
    const int dt = float_dtype("_pw_inner", x1);
    TORCH_CHECK(epilogue >= TPW_EPI_DOT && epilogue <= TPW_EPI_CORRELATION, "_pw_inner: bad epilogue");
    DeviceGuard guard(x1.device());
    auto a = as3(x1), b = as3(x2);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options());
    at::Tensor n1, n2;
    void *s = current_stream();
    if (epilogue != TPW_EPI_DOT) {
        const int squared = (epilogue == TPW_EPI_EUCLIDEAN || epilogue == TPW_EPI_SQEUCLIDEAN);
        n1 = at::empty({B, n}, a.options().dtype(at::kFloat));
        check_rc(tpw_row_norms(a.data_ptr(), dt, B * n, d, squared, n1.data_ptr<float>(), s), "row norms");
        if (x2.is_same(x1)) {
            n2 = n1;  // x2 = None: one set of norms
        } else {
            n2 = at::empty({B, m}, a.options().dtype(at::kFloat));
            check_rc(tpw_row_norms(b.data_ptr(), dt, B * m, d, squared, n2.data_ptr<float>(), s), "row norms");
        }
    }
    // Rows that are not whole 128-byte chunks (or operands not 16-byte aligned) would take the
    // register-staged kernel, whose element loads run 1.3-4x slower; for outputs of 2^20 entries
    // or more the operands are copied zero-padded to whole chunks for the tile kernel instead.
    // The staged kernel zero-fills its last chunk the same way, so the products are the same.
    at::Tensor ap = a, bp = b;
    int64_t dk = d;
    const int64_t chunk = 128 / (int64_t)a.element_size();
    const auto misaligned = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 != 0; };
    if (d > 0 && B * n * m >= (int64_t(1) << 20) &&
        (d % chunk != 0 || misaligned(a.data_ptr()) || misaligned(b.data_ptr()))) {
        dk = (d + chunk - 1) / chunk * chunk;
        ap = at::zeros({B, n, dk}, a.options());
        ap.narrow(2, 0, d).copy_(a);
        if (x2.is_same(x1)) {
            bp = ap;
        } else {
            bp = at::zeros({B, m, dk}, b.options());
            bp.narrow(2, 0, d).copy_(b);
        }
    }
    check_rc(tpw_pairwise_inner(ap.data_ptr(), bp.data_ptr(), dt, B, n, m, dk,
                                n1.defined() ? n1.data_ptr<float>() : nullptr,
                                n2.defined() ? n2.data_ptr<float>() : nullptr, (int)epilogue,
                                out.data_ptr(), s),
             "_pw_inner");
    return out_shape(out, x1);
}

std::tuple<at::Tensor, at::Tensor> pw_inner_backward_cuda(const at::Tensor &grad,
                                                          const at::Tensor &x1,
                                                          const at::Tensor &x2,
                                                          const at::Tensor &res, int64_t epilogue) {
    check_cuda_pair("_pw_inner_backward", x1, x2);
    const int dt = float_dtype("_pw_inner_backward", x1);
    DeviceGuard guard(x1.device());
    auto a = as3(x1), b = as3(x2);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto g = grad.to(a.scalar_type()).reshape({B, n, m}).contiguous();
    auto gx1 = at::empty_like(a), gx2 = at::empty_like(b);
    auto ws = workspace(tpw_inner_backward_workspace_size(B, n, m, d), a);
    void *s = current_stream();
    if (epilogue == TPW_EPI_EUCLIDEAN) {
        auto r = res.reshape({B, n, m}).contiguous();
        check_rc(tpw_euclidean_backward(g.data_ptr(), a.data_ptr(), b.data_ptr(), r.data_ptr(), dt, B,
                                        n, m, d, gx1.data_ptr(), gx2.data_ptr(), ws.data_ptr(), s),
                 "euclidean backward");
    } else if (epilogue == TPW_EPI_SQEUCLIDEAN) {
        check_rc(tpw_sqeuclidean_backward(g.data_ptr(), a.data_ptr(), b.data_ptr(), dt, B, n, m, d,
                                          gx1.data_ptr(), gx2.data_ptr(), ws.data_ptr(), s),
                 "sqeuclidean backward");
    } else if (epilogue == TPW_EPI_DOT) {
        check_rc(tpw_linear_backward(g.data_ptr(), a.data_ptr(), b.data_ptr(), dt, B, n, m, d,
                                     gx1.data_ptr(), gx2.data_ptr(), ws.data_ptr(), s),
                 "linear backward");
    } else if (epilogue == TPW_EPI_COSINE_SIM || epilogue == TPW_EPI_COSINE_DIST ||
               epilogue == TPW_EPI_CORRELATION) {
        auto n1 = at::empty({B, n}, a.options().dtype(at::kFloat));
        auto n2 = at::empty({B, m}, a.options().dtype(at::kFloat));
        check_rc(tpw_row_norms(a.data_ptr(), dt, B * n, d, 0, n1.data_ptr<float>(), s), "row norms");
        check_rc(tpw_row_norms(b.data_ptr(), dt, B * m, d, 0, n2.data_ptr<float>(), s), "row norms");
        // the forward's output, when autograd saved it: the weights come from it
        at::Tensor o = res.defined() ? res.reshape({B, n, m}).contiguous() : at::Tensor();
        check_rc(tpw_cosine_backward(g.data_ptr(), a.data_ptr(), b.data_ptr(), n1.data_ptr<float>(),
                                     n2.data_ptr<float>(), o.defined() ? o.data_ptr() : nullptr, dt, B, n, m, d,
                                     epilogue == TPW_EPI_CORRELATION ? 2 : epilogue == TPW_EPI_COSINE_SIM,
                                     gx1.data_ptr(), gx2.data_ptr(), ws.data_ptr(), s),
                 "cosine backward");
    } else {
        TORCH_CHECK(false, "_pw_inner_backward: epilogue ", epilogue, " has no backward");
    }
    return {gx1.reshape(x1.sizes()), gx2.reshape(x2.sizes())};
}

// ---------------------------------------------------------------- kernel functions (MFMA)
at::Tensor pw_kernel_cuda(const at::Tensor &x1, const at::Tensor &x2, int64_t kind, double gamma,
                          double coef0, int64_t degree) {
    check_cuda_pair("_pw_kernel", x1, x2);
    TORCH_CHECK(x1.scalar_type() == x2.scalar_type(), "_pw_kernel: x1 and x2 dtypes differ");
    const int dt = float_dtype("_pw_kernel", x1);
    DeviceGuard guard(x1.device());
    auto a = as3(x1), b = as3(x2);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options());
    check_rc(tpw_pairwise_kernel(a.data_ptr(), b.data_ptr(), dt, B, n, m, d, (int)kind, (float)gamma,
                                 (float)coef0, (int)degree, out.data_ptr(), current_stream()),
             "_pw_kernel");
    return out_shape(out, x1);
}

std::tuple<at::Tensor, at::Tensor> pw_kernel_backward_cuda(const at::Tensor &grad, const at::Tensor &x1,
                                                           const at::Tensor &x2, const at::Tensor &res,
                                                           int64_t kind, double gamma, double coef0,
                                                           int64_t degree) {
    check_cuda_pair("_pw_kernel_backward", x1, x2);
    const int dt = float_dtype("_pw_kernel_backward", x1);
    DeviceGuard guard(x1.device());
    auto a = as3(x1), b = as3(x2);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto g = grad.to(a.scalar_type()).reshape({B, n, m}).contiguous();
    at::Tensor r;
    if (res.defined()) r = res.to(a.scalar_type()).reshape({B, n, m}).contiguous();
    auto gx1 = at::empty_like(a), gx2 = at::empty_like(b);
    auto ws = workspace(tpw_inner_backward_workspace_size(B, n, m, d), a);
    check_rc(tpw_pairwise_kernel_backward(g.data_ptr(), a.data_ptr(), b.data_ptr(),
                                          r.defined() ? r.data_ptr() : nullptr, dt, B, n, m, d, (int)kind,
                                          (float)gamma, (float)coef0, (int)degree, gx1.data_ptr(),
                                          gx2.data_ptr(), ws.data_ptr(), current_stream()),
             "_pw_kernel_backward");
    return {gx1.reshape(x1.sizes()), gx2.reshape(x2.sizes())};
}

// ---------------------------------------------------------------- Minkowski (VALU)
at::Tensor pw_lp_cuda(const at::Tensor &x1, const at::Tensor &x2, double p) {
    check_cuda_pair("_pw_lp", x1, x2);
    TORCH_CHECK(x1.scalar_type() == at::kFloat && x2.scalar_type() == at::kFloat,
                "_pw_lp: supports float32 on the GPU");
    TORCH_CHECK(p >= 0, "cdist only supports non-negative p values");
    DeviceGuard guard(x1.device());
    auto a = as3(x1), b = as3(x2);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options());
    check_rc(tpw_lp_distances(a.data_ptr<float>(), b.data_ptr<float>(), B, n, m, d, p,
                              out.data_ptr<float>(), current_stream()),
             "_pw_lp");
    return out_shape(out, x1);
}

std::tuple<at::Tensor, at::Tensor> pw_lp_backward_cuda(const at::Tensor &grad, const at::Tensor &x1,
                                                       const at::Tensor &x2, const at::Tensor &dist,
                                                       double p) {
    check_cuda_pair("_pw_lp_backward", x1, x2);
    TORCH_CHECK(x1.scalar_type() == at::kFloat, "_pw_lp_backward: supports float32 on the GPU");
    DeviceGuard guard(x1.device());
    auto a = as3(x1), b = as3(x2);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto g = grad.to(at::kFloat).reshape({B, n, m}).contiguous();
    auto dd = dist.reshape({B, n, m}).contiguous();
    auto gx1 = at::empty_like(a), gx2 = at::empty_like(b);
    auto ws = workspace(tpw_lp_backward_workspace_size(B, n, m, d), a);
    check_rc(tpw_lp_distances_backward2(g.data_ptr<float>(), a.data_ptr<float>(), b.data_ptr<float>(),
                                        dd.data_ptr<float>(), B, n, m, d, p, gx1.data_ptr<float>(),
                                        gx2.data_ptr<float>(), ws.data_ptr(), current_stream()),
             "_pw_lp_backward");
    return {gx1.reshape(x1.sizes()), gx2.reshape(x2.sizes())};
}

// ---------------------------------------------------------------- boolean family
void check_binary_shapes(const at::Tensor &x1, const at::Tensor &x2) {
    // csrc/ops/cpu/pairwise_binary_kernels.cpp:123-133
    const bool unbatched = x1.dim() == 2;
    TORCH_CHECK(unbatched || x1.dim() == 3, "x1 must be 2-D (unbatched) or 3-D (batched) tensor.")
    TORCH_CHECK(unbatched || x2.dim() == 3, "x2 must be 2-D (unbatched) or 3-D (batched) tensor.")
    TORCH_CHECK(unbatched || x1.size(0) == x2.size(0), "batch_size of x1 and x2 do not match.")
    TORCH_CHECK((unbatched && x1.size(1) == x2.size(1)) || (!unbatched && x1.size(2) == x2.size(2)),
                "feature dimension of x1 and x2 do not match.")
}

// Packs [rows, d] bool rows into uint32 words (+ row popcounts).
std::pair<at::Tensor, at::Tensor> pack(const at::Tensor &x3, bool with_pops) {
    const int64_t rows = x3.size(0) * x3.size(1), d = x3.size(2);
    auto words = at::empty({rows, tpw_packed_words(d)}, x3.options().dtype(at::kInt));
    at::Tensor pops;
    if (with_pops) pops = at::empty({rows}, x3.options().dtype(at::kInt));
    check_rc(tpw_pack_bool_rows(reinterpret_cast<const uint8_t *>(x3.data_ptr<bool>()), rows, d,
                                reinterpret_cast<uint32_t *>(words.data_ptr<int32_t>()),
                                with_pops ? pops.data_ptr<int32_t>() : nullptr, current_stream()),
             "pack bool rows");
    return {words, pops};
}

}  // namespace

void bool_bytes_cuda(const at::Tensor &a, const at::Tensor &b, int bmet, int op, int red, at::Tensor &out) {
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    const bool same = b.is_same(a);
    if (d < (int64_t(1) << 24) && std::max(n, m) * tpw_packed_words(d) * 4 < (int64_t(1) << 32)) {
        // bit-packed rows and row popcounts (one pack pass per operand); the count metrics, and
        // the reductions over more than 256 features, then take the bit tile kernel on the fp4
        // matrix cores (any m), the rest the popcount kernel; the results equal the int8 byte
        // path's bit for bit
        auto pa = pack(a, true);
        auto pb = same ? pa : pack(b, true);
        const uint32_t *wa = reinterpret_cast<const uint32_t *>(pa.first.data_ptr<int32_t>());
        const uint32_t *wb = reinterpret_cast<const uint32_t *>(pb.first.data_ptr<int32_t>());
        if (bmet >= 0)
            check_rc(tpw_bool_count_metric(wa, wb, pa.second.data_ptr<int32_t>(), pb.second.data_ptr<int32_t>(), B, n, m,
                                           d, bmet, out.data_ptr<float>(), current_stream()),
                     "boolean count metric");
        else
            check_rc(tpw_bool_pairwise_reduce_counted(wa, wb, pa.second.data_ptr<int32_t>(),
                                                      pb.second.data_ptr<int32_t>(), B, n, m, d, op, red,
                                                      out.data_ptr<float>(), current_stream()),
                     "pairwise bool reduction");
        return;
    }
    const int64_t rb = tpw_bool_fp4_row_bytes(d);
    if (d < (int64_t(1) << 24) && std::max(n, m) * rb < (int64_t(1) << 31)) {
        // fp4 rows (one pack pass per operand: nibbles and row counts), then the scaled matrix
        // cores; the results equal the int8 byte path's bit for bit
        auto fa = at::empty({B * n, rb}, a.options().dtype(at::kByte));
        auto ca = at::empty({B * n}, a.options().dtype(at::kInt));
        check_rc(tpw_pack_bool_fp4(reinterpret_cast<const uint8_t *>(a.data_ptr<bool>()), B * n, d, fa.data_ptr<uint8_t>(),
                                   ca.data_ptr<int32_t>(), current_stream()),
                 "pack bool fp4");
        at::Tensor fb = fa, cb = ca;
        if (!same) {
            fb = at::empty({B * m, rb}, b.options().dtype(at::kByte));
            cb = at::empty({B * m}, b.options().dtype(at::kInt));
            check_rc(tpw_pack_bool_fp4(reinterpret_cast<const uint8_t *>(b.data_ptr<bool>()), B * m, d,
                                       fb.data_ptr<uint8_t>(), cb.data_ptr<int32_t>(), current_stream()),
                     "pack bool fp4");
        }
        if (bmet >= 0)
            check_rc(tpw_bool_fp4_count_metric(fa.data_ptr<uint8_t>(), fb.data_ptr<uint8_t>(), ca.data_ptr<int32_t>(),
                                               cb.data_ptr<int32_t>(), B, n, m, d, bmet, out.data_ptr<float>(),
                                               current_stream()),
                     "boolean count metric");
        else
            check_rc(tpw_bool_fp4_reduce(fa.data_ptr<uint8_t>(), fb.data_ptr<uint8_t>(), ca.data_ptr<int32_t>(),
                                         cb.data_ptr<int32_t>(), B, n, m, d, op, red, out.data_ptr<float>(),
                                         current_stream()),
                     "pairwise bool reduction");
        return;
    }
    auto ca = at::empty({B * n}, a.options().dtype(at::kInt));
    auto cb = same ? ca : at::empty({B * m}, b.options().dtype(at::kInt));
    const uint8_t *pa = reinterpret_cast<const uint8_t *>(a.data_ptr<bool>());
    const uint8_t *pb = reinterpret_cast<const uint8_t *>(b.data_ptr<bool>());
    check_rc(tpw_bool_row_counts(pa, B * n, d, ca.data_ptr<int32_t>(), current_stream()), "bool row counts");
    if (!same)
        check_rc(tpw_bool_row_counts(pb, B * m, d, cb.data_ptr<int32_t>(), current_stream()), "bool row counts");
    if (bmet >= 0)
        check_rc(tpw_bool_bytes_count_metric(pa, pb, ca.data_ptr<int32_t>(), cb.data_ptr<int32_t>(), B, n, m, d,
                                             bmet, out.data_ptr<float>(), current_stream()),
                 "boolean count metric");
    else
        check_rc(tpw_bool_bytes_reduce(pa, pb, ca.data_ptr<int32_t>(), cb.data_ptr<int32_t>(), B, n, m, d, op,
                                       red, out.data_ptr<float>(), current_stream()),
                 "pairwise bool reduction");
}

namespace {

template <int OP, int RED>
at::Tensor pw_reduce_cuda(const at::Tensor &x1, const at::Tensor &x2) {
    TORCH_CHECK(x1.is_cuda() && x2.is_cuda(), "expected GPU tensors");
    check_binary_shapes(x1, x2);
    DeviceGuard guard(x1.device());
    const auto common = at::result_type(x1, x2);
    pw_check_dispatch(OP, common, "pairwise_binary_reduction_forward_cuda");
    auto a = as3(x1.to(common)), b = as3(x2.to(common));
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options().dtype(at::kFloat));
    if (B * n * m == 0) return out_shape(out, x1);
    if (d == 0) {  // empty reduction: sum 0, mean 0/0
        out.fill_(RED == TPW_RED_SUM ? 0.0 : std::numeric_limits<double>::quiet_NaN());
        return out_shape(out, x1);
    }
    if (common == at::kBool && d >= kBoolBytesMinFeatures) {
        a = a.contiguous();
        b = x2.is_same(x1) ? a : b.contiguous();
        bool_bytes_cuda(a, b, -1, OP, RED, out);
    } else if (common == at::kBool) {
        auto wa = pack(a, false).first, wb = pack(b, false).first;
        check_rc(tpw_bool_pairwise_reduce(reinterpret_cast<const uint32_t *>(wa.data_ptr<int32_t>()),
                                          reinterpret_cast<const uint32_t *>(wb.data_ptr<int32_t>()),
                                          B, n, m, d, OP, RED, out.data_ptr<float>(), current_stream()),
                 "pairwise bool reduction");
    } else {
        const int code = float_code(common);
        TORCH_CHECK(code >= 0, "pairwise comparison not implemented for ", common);
        check_rc(tpw_compare_reduce(a.data_ptr(), b.data_ptr(), code, B, n, m, d, OP, RED,
                                    out.data_ptr<float>(), current_stream()),
                 "pairwise comparison reduction");
    }
    return out_shape(out, x1);
}

at::Tensor jaccard_cuda(const at::Tensor &x1, const at::Tensor &x2) {
    TORCH_CHECK(x1.is_cuda() && x2.is_cuda(), "expected GPU tensors");
    check_binary_shapes(x1, x2);
    DeviceGuard guard(x1.device());
    auto a = as3(x1.to(at::kBool)), b = as3(x2.to(at::kBool));
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options().dtype(at::kFloat));
    if (B * n * m == 0) return out_shape(out, x1);
    if (d == 0) {
        out.zero_();
        return out_shape(out, x1);
    }
    a = a.contiguous();
    b = x2.is_same(x1) ? a : b.contiguous();
    bool_bytes_cuda(a, b, TPW_BMET_JACCARD, 0, 0, out);
    return out_shape(out, x1);
}

// ---------------------------------------------------------------- neighbour mask
// Bool mask of each row's `count` smallest entries (stable order: ties to the lower column).
at::Tensor row_smallest_mask_cuda(const at::Tensor &dist, int64_t count) {
    TORCH_CHECK(dist.is_cuda() && dist.dim() == 2, "_row_smallest_mask: expected a 2-D GPU tensor");
    TORCH_CHECK(count >= 0, "_row_smallest_mask: count must be non-negative, got ", count);
    const int code = float_code(dist.scalar_type());
    TORCH_CHECK(code == TPW_F32 || code == TPW_BF16 || code == TPW_F16,
                "_row_smallest_mask: expected float32, bfloat16 or float16 distances, got ",
                dist.scalar_type());
    DeviceGuard guard(dist.device());
    auto d = dist.contiguous();
    auto mask = at::empty(d.sizes(), d.options().dtype(at::kBool));
    check_rc(tpw_row_smallest_mask(d.data_ptr(), code, d.size(0), d.size(1), count, mask.data_ptr(),
                                   current_stream()),
             "row_smallest_mask");
    return mask;
}

// ---------------------------------------------------------------- Hausdorff
struct HdRun {
    at::Tensor a, b, out, i1, i2;
};

// float32 takes the pruned cell-grid pipeline; float64 and float16 the reference's loop in
// its own order (tpw_directed_hausdorff_exact).  The reference serves the same three types
// (cuda/hausdorff_kernel.cu:150, AT_DISPATCH_FLOATING_TYPES_AND_HALF) and refuses the others.
int hd_exact_code(at::ScalarType t, const char *from) {
    TORCH_CHECK_NOT_IMPLEMENTED(t == at::kDouble || t == at::kHalf, "\"", from,
                                "\" not implemented for '", c10::toString(t), "'");
    return t == at::kDouble ? TPW_F64 : TPW_F16;
}

HdRun hausdorff_run(const at::Tensor &x1, const at::Tensor &x2, bool shuffle,
                    c10::optional<at::Generator> gen) {
    check_hausdorff_shapes(x1, x2);
    TORCH_CHECK(x1.is_cuda() && x2.is_cuda(), "_directed_hausdorff: expected GPU tensors");
    const bool exact = x1.scalar_type() != at::kFloat;
    const int code = exact ? hd_exact_code(x1.scalar_type(), "_directed_hausdorff_forward_cuda") : TPW_F32;
    HdRun r;
    r.a = x1.dim() == 3 ? x1.unsqueeze(0).contiguous() : x1.contiguous();
    r.b = x2.dim() == 3 ? x2.unsqueeze(0).contiguous() : x2.contiguous();
    const int64_t B = r.a.size(0), b1 = r.a.size(1), p1 = r.a.size(2), d = r.a.size(3);
    const int64_t b2 = r.b.size(1), p2 = r.b.size(2);
    r.out = at::empty({B, b1, b2}, r.a.options());
    r.i1 = at::empty({B, b1, b2}, r.a.options().dtype(at::kLong));
    r.i2 = at::empty({B, b1, b2}, r.a.options().dtype(at::kLong));
    at::Tensor perm1, perm2;
    if (shuffle) std::tie(perm1, perm2) = hausdorff_perms(B, p1, p2, r.a.options(), gen);
    if (exact) {
        check_rc(tpw_directed_hausdorff_exact(code, r.a.data_ptr(), r.b.data_ptr(), B, b1, p1, b2, p2, d,
                                              shuffle ? perm1.data_ptr<int64_t>() : nullptr,
                                              shuffle ? perm2.data_ptr<int64_t>() : nullptr, r.out.data_ptr(),
                                              r.i1.data_ptr<int64_t>(), r.i2.data_ptr<int64_t>(),
                                              current_stream()),
                 "_directed_hausdorff");
        return r;
    }
    auto ws = workspace(tpw_hausdorff_workspace_size(B, b1, p1, b2, p2, d), r.a);
    check_rc(tpw_directed_hausdorff(r.a.data_ptr<float>(), r.b.data_ptr<float>(), B, b1, p1, b2, p2, d,
                                    shuffle ? perm1.data_ptr<int64_t>() : nullptr,
                                    shuffle ? perm2.data_ptr<int64_t>() : nullptr,
                                    r.out.data_ptr<float>(), r.i1.data_ptr<int64_t>(),
                                    r.i2.data_ptr<int64_t>(), ws.data_ptr(), current_stream()),
             "_directed_hausdorff");
    return r;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> directed_hausdorff_cuda(
    const at::Tensor &x1, const at::Tensor &x2, bool shuffle, c10::optional<at::Generator> gen) {
    DeviceGuard guard(x1.device());
    HdRun r = hausdorff_run(x1, x2, shuffle, gen);
    if (x1.dim() == 3) return {r.out.squeeze(0), r.i1.squeeze(0), r.i2.squeeze(0)};
    return {r.out, r.i1, r.i2};
}

std::tuple<at::Tensor, at::Tensor> directed_hausdorff_backward_cuda(
    const at::Tensor &grad, const at::Tensor &x1, const at::Tensor &x2, bool shuffle,
    c10::optional<at::Generator> gen) {
    DeviceGuard guard(x1.device());
    // the reference re-runs the forward here (csrc/ops/cpu/hausdorff_kernel.cpp:269-306)
    HdRun r = hausdorff_run(x1, x2, shuffle, gen);
    if (r.a.scalar_type() != at::kFloat) {
        auto g = grad.to(r.a.scalar_type()).reshape(r.out.sizes()).contiguous();
        auto gx1 = at::empty_like(r.a), gx2 = at::empty_like(r.b);
        check_rc(tpw_directed_hausdorff_exact_backward(
                     hd_exact_code(r.a.scalar_type(), "_directed_hausdorff_backward_cuda"), g.data_ptr(),
                     r.a.data_ptr(), r.b.data_ptr(), r.out.data_ptr(), r.i1.data_ptr<int64_t>(),
                     r.i2.data_ptr<int64_t>(), r.a.size(0), r.a.size(1), r.a.size(2), r.b.size(1), r.b.size(2),
                     r.a.size(3), gx1.data_ptr(), gx2.data_ptr(), current_stream()),
                 "__directed_hausdorff_backward");
        if (x1.dim() == 3) return {gx1.squeeze(0), gx2.squeeze(0)};
        return {gx1, gx2};
    }
    auto g = grad.to(at::kFloat).reshape(r.out.sizes()).contiguous();
    auto gx1 = at::empty_like(r.a), gx2 = at::empty_like(r.b);  // written whole by the kernel
    check_rc(tpw_directed_hausdorff_backward(
                 g.data_ptr<float>(), r.a.data_ptr<float>(), r.b.data_ptr<float>(),
                 r.out.data_ptr<float>(), r.i1.data_ptr<int64_t>(), r.i2.data_ptr<int64_t>(),
                 r.a.size(0), r.a.size(1), r.a.size(2), r.b.size(1), r.b.size(2), r.a.size(3),
                 gx1.data_ptr<float>(), gx2.data_ptr<float>(), current_stream()),
             "__directed_hausdorff_backward");
    if (x1.dim() == 3) return {gx1.squeeze(0), gx2.squeeze(0)};
    return {gx1, gx2};
}

}  // namespace

at::Tensor lp_distances_bf16_cuda(const at::Tensor &x1, const at::Tensor &x2, double p) {
    check_cuda_pair("cdist", x1, x2);
    TORCH_CHECK(x1.scalar_type() == at::kFloat && x2.scalar_type() == at::kFloat, "cdist: float32 rows expected");
    DeviceGuard guard(x1.device());
    auto a = as3(x1), b = as3(x2);
    const int64_t B = a.size(0), n = a.size(1), m = b.size(1), d = a.size(2);
    auto out = at::empty({B, n, m}, a.options().dtype(at::kBFloat16));
    check_rc(tpw_lp_distances_bf16(a.data_ptr<float>(), b.data_ptr<float>(), B, n, m, d, p,
                                   reinterpret_cast<uint16_t *>(out.data_ptr()), current_stream()),
             "cdist");
    return out_shape(out, x1);
}

std::tuple<at::Tensor, at::Tensor> directed_hausdorff_backward_indexed_cuda(
    const at::Tensor &grad, const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &out,
    const at::Tensor &i1, const at::Tensor &i2) {
    DeviceGuard guard(x1.device());
    auto a = x1.dim() == 3 ? x1.unsqueeze(0).contiguous() : x1.contiguous();
    auto b = x2.dim() == 3 ? x2.unsqueeze(0).contiguous() : x2.contiguous();
    const int64_t B = a.size(0), b1 = a.size(1), b2 = b.size(1);
    auto o = out.reshape({B, b1, b2}).contiguous();
    auto m1 = i1.reshape({B, b1, b2}).contiguous(), m2 = i2.reshape({B, b1, b2}).contiguous();
    if (a.scalar_type() != at::kFloat) {
        auto g = grad.to(a.scalar_type()).reshape({B, b1, b2}).contiguous();
        auto gx1 = at::empty_like(a), gx2 = at::empty_like(b);
        check_rc(tpw_directed_hausdorff_exact_backward(
                     hd_exact_code(a.scalar_type(), "_directed_hausdorff_backward_cuda"), g.data_ptr(),
                     a.data_ptr(), b.data_ptr(), o.data_ptr(), m1.data_ptr<int64_t>(), m2.data_ptr<int64_t>(), B,
                     b1, a.size(2), b2, b.size(2), a.size(3), gx1.data_ptr(), gx2.data_ptr(), current_stream()),
                 "__directed_hausdorff_backward");
        if (x1.dim() == 3) return {gx1.squeeze(0), gx2.squeeze(0)};
        return {gx1, gx2};
    }
    auto g = grad.to(at::kFloat).reshape({B, b1, b2}).contiguous();
    auto gx1 = at::empty_like(a), gx2 = at::empty_like(b);  // written whole by the kernels
    check_rc(tpw_directed_hausdorff_backward(
                 g.data_ptr<float>(), a.data_ptr<float>(), b.data_ptr<float>(), o.data_ptr<float>(),
                 m1.data_ptr<int64_t>(), m2.data_ptr<int64_t>(), B, b1, a.size(2), b2, b.size(2), a.size(3),
                 gx1.data_ptr<float>(), gx2.data_ptr<float>(), current_stream()),
             "__directed_hausdorff_backward");
    if (x1.dim() == 3) return {gx1.squeeze(0), gx2.squeeze(0)};
    return {gx1, gx2};
}

namespace {

// ---------------------------------------------------------------- unreduced pw ops
template <int OP>
at::Tensor pw_binary_cuda(const at::Tensor &x1, const at::Tensor &x2) {
    TORCH_CHECK(x1.device() == x2.device(), "pairwise_binary_forward: x1 and x2 must be on the same device");
    DeviceGuard guard(x1.device());
    auto r = pw_binary_prepare(OP, x1, x2, "pairwise_binary_forward_cuda");
    const int64_t B = r.a.size(0), n = r.a.size(1), m = r.b.size(1), d = r.a.size(2);
    auto out = at::empty({B, n, m, d}, r.a.options().dtype(at::kBool));
    const int code = r.a.scalar_type() == at::kBool ? TPW_U8 : float_code(r.a.scalar_type());
    check_rc(tpw_pairwise_binary(r.a.data_ptr(), r.b.data_ptr(), code, OP, B, n, m, d,
                                 reinterpret_cast<uint8_t *>(out.data_ptr()), current_stream()),
             "pairwise_binary_forward");
    return out.view(r.out_shape);
}

}  // namespace

TORCH_LIBRARY_IMPL(torchpairwise, CUDA, m) {
    m.impl("_pw_inner", TORCH_FN(pw_inner_cuda));
    m.impl("_radius_mask_euclidean", TORCH_FN(radius_mask_euclidean_cuda));
    m.impl("_knn_mask_euclidean", TORCH_FN(knn_mask_euclidean_cuda));
    m.impl("_pw_inner_backward", TORCH_FN(pw_inner_backward_cuda));
    m.impl("_pw_kernel", TORCH_FN(pw_kernel_cuda));
    m.impl("_pw_kernel_backward", TORCH_FN(pw_kernel_backward_cuda));
    m.impl("_pw_lp", TORCH_FN(pw_lp_cuda));
    m.impl("_pw_lp_backward", TORCH_FN(pw_lp_backward_cuda));
    m.impl("_jaccard", TORCH_FN(jaccard_cuda));
    m.impl("_row_smallest_mask", TORCH_FN(row_smallest_mask_cuda));
    m.impl("pwand_sum", TORCH_FN((pw_reduce_cuda<TPW_BIT_AND, TPW_RED_SUM>)));
    m.impl("pwor_sum", TORCH_FN((pw_reduce_cuda<TPW_BIT_OR, TPW_RED_SUM>)));
    m.impl("pwxor_sum", TORCH_FN((pw_reduce_cuda<TPW_BIT_XOR, TPW_RED_SUM>)));
    m.impl("pweq_sum", TORCH_FN((pw_reduce_cuda<TPW_BIT_EQ, TPW_RED_SUM>)));
    m.impl("pwne_sum", TORCH_FN((pw_reduce_cuda<TPW_BIT_NE, TPW_RED_SUM>)));
    m.impl("pweq_mean", TORCH_FN((pw_reduce_cuda<TPW_BIT_EQ, TPW_RED_MEAN>)));
    m.impl("pwne_mean", TORCH_FN((pw_reduce_cuda<TPW_BIT_NE, TPW_RED_MEAN>)));
    m.impl("_directed_hausdorff", TORCH_FN(directed_hausdorff_cuda));
    m.impl("__directed_hausdorff_backward", TORCH_FN(directed_hausdorff_backward_cuda));
    m.impl("pwand", TORCH_FN(pw_binary_cuda<TPW_BIT_AND>));
    m.impl("pwor", TORCH_FN(pw_binary_cuda<TPW_BIT_OR>));
    m.impl("pwxor", TORCH_FN(pw_binary_cuda<TPW_BIT_XOR>));
    m.impl("pweq", TORCH_FN(pw_binary_cuda<TPW_BIT_EQ>));
    m.impl("pwne", TORCH_FN(pw_binary_cuda<TPW_BIT_NE>));
    m.impl("pwlt", TORCH_FN(pw_binary_cuda<TPW_CMP_LT>));
    m.impl("pwgt", TORCH_FN(pw_binary_cuda<TPW_CMP_GT>));
    m.impl("pwle", TORCH_FN(pw_binary_cuda<TPW_CMP_LE>));
    m.impl("pwge", TORCH_FN(pw_binary_cuda<TPW_CMP_GE>));
}

}  // namespace tpw_ext
