// Shared helpers of the PyTorch extension (host side only; kernels live behind the C ABI).
#pragma once

#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "torchpairwise_amd.h"

namespace tpw_ext {

// PyTorch-ROCm tensors report device type "cuda"; its HIP streams and device guards are
// the *MasqueradingAsCUDA variants.
using DeviceGuard = c10::hip::HIPGuardMasqueradingAsCUDA;

// Launch stream of the current device (PyTorch's current HIP stream).
inline void *current_stream() {
    return reinterpret_cast<void *>(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
}

inline void check_rc(int rc, const char *what) {
    TORCH_CHECK(rc == TPW_OK, what, ": ", tpw_last_error());
}

// Scratch memory from the caching allocator on `like`'s device.
inline at::Tensor workspace(size_t bytes, const at::Tensor &like) {
    return at::empty({(int64_t)(bytes > 0 ? bytes : 1)}, like.options().dtype(at::kByte));
}

inline int float_code(at::ScalarType t) {
    switch (t) {
        case at::kFloat: return TPW_F32;
        case at::kBFloat16: return TPW_BF16;
        case at::kHalf: return TPW_F16;
        case at::kDouble: return TPW_F64;
        case at::kChar: return TPW_I8;
        case at::kByte: return TPW_U8;
        case at::kShort: return TPW_I16;
        case at::kInt: return TPW_I32;
        case at::kLong: return TPW_I64;
        default: return -1;
    }
}

// The unreduced pairwise binary ops (pwand ... pwge), as the reference's
// pairwise_binary_forward_kernel prepares them (cpu/pairwise_binary_kernels.cpp:52-108,
// cuda/pairwise_binary_kernels.cu:61-141): 2-D inputs are unbatched, others [b, n, ...] with
// the trailing dims flattened into the features; both in at::result_type; the output
// [b, n, m, trailing...] (unbatched: [n, m, d]).  Element types as the reference dispatches
// them: logical ops bool only, eq / ne every integer and floating type and bool, the ordering
// comparisons every integer and floating type (no bool); others raise NotImplementedError
// with the reference's dispatch message.
// The reference's dtype dispatch of its own metric kernels (cpu/ and cuda/<op>_kernel.*):
// floating types and half, and bfloat16 where `bf16` (AT_DISPATCH_FLOATING_TYPES_AND2 rather
// than _AND_HALF); others raise its dispatch message for kernel `name`.
inline void check_float_dispatch(at::ScalarType t, bool bf16, const std::string &name) {
    const bool ok = t == at::kFloat || t == at::kDouble || t == at::kHalf || (bf16 && t == at::kBFloat16);
    TORCH_CHECK_NOT_IMPLEMENTED(ok, "\"", name, "\" not implemented for '", c10::toString(t), "'");
}

// Whether the reference dispatches binary op `op` (TPW_BIT_* / TPW_CMP_*) for element type t
// (common/binary_ops.h:69-78); if not, raise its dispatch message for kernel `name`.
inline void pw_check_dispatch(int op, at::ScalarType t, const char *name) {
    bool ok;
    if (op <= TPW_BIT_XOR) ok = t == at::kBool;
    else ok = t == at::kByte || t == at::kChar || t == at::kShort || t == at::kInt || t == at::kLong ||
              t == at::kFloat || t == at::kDouble || t == at::kHalf || t == at::kBFloat16 ||
              (t == at::kBool && (op == TPW_BIT_EQ || op == TPW_BIT_NE));
    TORCH_CHECK_NOT_IMPLEMENTED(ok, "\"", name, "\" not implemented for '", c10::toString(t), "'");
}

struct PwBinaryArgs {
    at::Tensor a, b;  // [B, n, D] and [B, m, D], contiguous, common type
    std::vector<int64_t> out_shape;
};
inline PwBinaryArgs pw_binary_prepare(int op, const at::Tensor &x1, const at::Tensor &x2, const char *name) {
    const bool unbatched = x1.dim() == 2;
    TORCH_CHECK(x1.dim() >= 2, "x1 must have at least 2 dimensions.")
    TORCH_CHECK(x2.dim() >= 2, "x2 must have at least 2 dimensions.")
    TORCH_CHECK(unbatched || x1.size(0) == x2.size(0), "batch_size of x1 and x2 do not match.")
    bool same = !unbatched && x1.dim() == x2.dim();
    for (int64_t d = 2; same && d < x1.dim(); ++d) same = x1.size(d) == x2.size(d);
    TORCH_CHECK((unbatched && x1.size(1) == x2.size(1)) || (!unbatched && same),
                "feature dimensions of x1 and x2 do not match.")
    const auto t = at::result_type(x1, x2);
    pw_check_dispatch(op, t, name);
    PwBinaryArgs r;
    r.a = x1.to(t).contiguous();
    r.b = x2.to(t).contiguous();
    if (unbatched) {
        r.a = r.a.unsqueeze(0);
        r.b = r.b.unsqueeze(0);
    }
    r.a = r.a.flatten(2);
    r.b = r.b.flatten(2);
    if (unbatched) {
        r.out_shape = {r.a.size(1), r.b.size(1), r.a.size(2)};
    } else {
        r.out_shape = {r.a.size(0), r.a.size(1), r.b.size(1)};
        for (int64_t d = 2; d < x1.dim(); ++d) r.out_shape.push_back(x1.size(d));
    }
    return r;
}

// [n, d] -> [1, n, d]; [b, n, d] unchanged (contiguous either way).
inline at::Tensor as3(const at::Tensor &x) {
    return x.dim() == 2 ? x.unsqueeze(0).contiguous() : x.contiguous();
}

// Epilogue codes of the inner-product internal op (same values as TPW_EPI_*).
constexpr int64_t kEuclidean = TPW_EPI_EUCLIDEAN;
constexpr int64_t kSqEuclidean = TPW_EPI_SQEUCLIDEAN;
constexpr int64_t kCosineSim = TPW_EPI_COSINE_SIM;
constexpr int64_t kCosineDist = TPW_EPI_COSINE_DIST;
constexpr int64_t kCorrelation = TPW_EPI_CORRELATION;
constexpr int64_t kDot = TPW_EPI_DOT;

// Dispatcher handles of the internal ops (defined in registration.cpp).
at::Tensor pw_inner(const at::Tensor &x1, const at::Tensor &x2, int64_t epilogue);
std::tuple<at::Tensor, at::Tensor> pw_inner_backward(const at::Tensor &grad, const at::Tensor &x1,
                                                     const at::Tensor &x2, const at::Tensor &res,
                                                     int64_t epilogue);
// the polynomial / sigmoid kernel functions on the MFMA kernel (TPW_KER_*)
at::Tensor pw_kernel(const at::Tensor &x1, const at::Tensor &x2, int64_t kind, double gamma,
                     double coef0, int64_t degree);
std::tuple<at::Tensor, at::Tensor> pw_kernel_backward(const at::Tensor &grad, const at::Tensor &x1,
                                                      const at::Tensor &x2, const at::Tensor &res,
                                                      int64_t kind, double gamma, double coef0,
                                                      int64_t degree);
at::Tensor pw_lp(const at::Tensor &x1, const at::Tensor &x2, double p);
// at::cdist's Lp distances of float32 GPU rows with the output written as bfloat16 by the kernel
// (no autograd: for callers that need no gradient; hip_impl.cpp)
at::Tensor lp_distances_bf16_cuda(const at::Tensor &x1, const at::Tensor &x2, double p);
std::tuple<at::Tensor, at::Tensor> pw_lp_backward(const at::Tensor &grad, const at::Tensor &x1,
                                                  const at::Tensor &x2, const at::Tensor &dist,
                                                  double p);
at::Tensor pw_binary_reduce(const char *name, const at::Tensor &x1, const at::Tensor &x2);
at::Tensor jaccard_fused(const at::Tensor &x1, const at::Tensor &x2);
at::Tensor row_smallest_mask(const at::Tensor &dist, int64_t count);
// the reference's VALU metric ops (family.cpp)
at::Tensor ppminkowski(const at::Tensor &x1, const at::Tensor &x2, double p);
at::Tensor wminkowski(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &w, double p);
at::Tensor canberra(const at::Tensor &x1, const at::Tensor &x2);
at::Tensor braycurtis(const at::Tensor &x1, const at::Tensor &x2);
at::Tensor additive_chi2(const at::Tensor &x1, const at::Tensor &x2);
at::Tensor sqjensenshannon(const at::Tensor &x1, const at::Tensor &x2, c10::optional<double> base);
// rbf / laplacian with the exponential fused into the VALU kernel (TPW_KER_RBF / _LAPLACIAN)
at::Tensor pw_exp_kernel(const at::Tensor &x1, const at::Tensor &x2, int64_t kind, double gamma);
// haversine, snr, squared mahalanobis (special.cpp)
at::Tensor haversine(const at::Tensor &x1, const at::Tensor &x2);
at::Tensor snr(const at::Tensor &x1, const at::Tensor &x2);
at::Tensor sqmahalanobis(const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &VI);
// bit-packed boolean rows and the one-pass boolean count metrics (packed_bool.cpp);
// bool_count_metric returns an undefined tensor where the fused GPU path does not apply
std::tuple<at::Tensor, at::Tensor> pack_bool(const at::Tensor &x);
at::Tensor packed_bool_metric(const at::Tensor &w1, const at::Tensor &p1, const at::Tensor &w2,
                              const at::Tensor &p2, int64_t d, c10::string_view metric);
at::Tensor bool_count_metric(const at::Tensor &x1, const at::Tensor &x2, c10::string_view metric);
// Boolean count metric (bmet = TPW_BMET_*) or, with bmet < 0, the pw reduction (op, red) of
// GPU bool rows a [B, n, d], b [B, m, d] (contiguous, d >= 1) straight from the bytes on the
// int8 matrix cores, into out [B, n, m] float32.  b may be the same tensor as a.
// Gradients of _directed_hausdorff on GPU float32 from the forward's output and indices (what
// the reference's re-run of the forward returns when it replays the same point order).
std::tuple<at::Tensor, at::Tensor> directed_hausdorff_backward_indexed_cuda(
    const at::Tensor &grad, const at::Tensor &x1, const at::Tensor &x2, const at::Tensor &out,
    const at::Tensor &i1, const at::Tensor &i2);
void bool_bytes_cuda(const at::Tensor &a, const at::Tensor &b, int bmet, int op, int red, at::Tensor &out);
// Plain pw reductions of bool rows take the packed popcount kernel up to this many features
// and the int8 matrix cores above (the count metrics always take the matrix cores): the
// packed rows are 8x smaller, which wins while the output write dominates.
constexpr int64_t kBoolBytesMinFeatures = 257;
at::Tensor prf_div(const at::Tensor &x, const at::Tensor &y, c10::string_view mode);
// prf_div of two tensors without the dispatcher (for other ops' CPU / GPU bodies; prf_div.cpp)
at::Tensor prf_div_cpu(const at::Tensor &x, const at::Tensor &y, c10::string_view mode);
std::tuple<at::Tensor, at::Tensor> prf_div_backward(const at::Tensor &g, const at::Tensor &x,
                                                    const at::Tensor &y, c10::string_view mode);
std::tuple<at::Tensor, at::Tensor, at::Tensor> directed_hausdorff(
    const at::Tensor &x1, const at::Tensor &x2, bool shuffle, c10::optional<at::Generator> gen);
std::tuple<at::Tensor, at::Tensor> directed_hausdorff_backward(
    const at::Tensor &grad, const at::Tensor &x1, const at::Tensor &x2, bool shuffle,
    c10::optional<at::Generator> gen);

// prf_div mode string -> identity flag (common/prf_div_mode.h:13-23 of the reference).
inline bool prf_identity(c10::string_view mode) {
    if (mode == "zero") return false;
    if (mode == "identity") return true;
    TORCH_CHECK(false, "mode must be either zero or identity. Got ", std::string(mode));
}

// Shared shape checks of the Hausdorff ops (csrc/ops/cpu/hausdorff_kernel.cpp:109-123).
inline void check_hausdorff_shapes(const at::Tensor &x1, const at::Tensor &x2) {
    at::CheckedFrom c = "_directed_hausdorff_forward";
    auto args = {at::TensorArg(x1, "x1", 1), at::TensorArg(x2, "x2", 2)};
    at::checkAllSameType(c, args);
    const bool unbatched = x1.dim() == 3;
    TORCH_CHECK(unbatched || x1.dim() == 4, "x1 must be 3-D (unbatched) or 4-D (batched) tensor.")
    TORCH_CHECK(unbatched || x2.dim() == 4, "x2 must be 3-D (unbatched) or 4-D (batched) tensor.")
    TORCH_CHECK(unbatched || (x1.size(0) == x2.size(0)), "batch_size of x1 and x2 do not match.")
    TORCH_CHECK((unbatched && x1.size(2) == x2.size(2)) || (!unbatched && x1.size(3) == x2.size(3)),
                "feature dimension of x1 and x2 do not match.")
}

// Hausdorff iteration orders drawn as the reference draws them: per batch, x1's then x2's
// permutation from `gen` on the inputs' device (csrc/ops/cpu/hausdorff_kernel.cpp:149-158).
inline std::pair<at::Tensor, at::Tensor> hausdorff_perms(int64_t batch, int64_t p1, int64_t p2,
                                                         const at::TensorOptions &opts,
                                                         c10::optional<at::Generator> gen) {
    auto perm1 = at::empty({batch, p1}, opts.dtype(at::kLong));
    auto perm2 = at::empty({batch, p2}, opts.dtype(at::kLong));
    for (int64_t b = 0; b < batch; ++b) {
        auto r1 = perm1[b], r2 = perm2[b];
        at::randperm_outf(p1, gen, r1);
        at::randperm_outf(p2, gen, r2);
    }
    return {perm1, perm2};
}

}  // namespace tpw_ext
