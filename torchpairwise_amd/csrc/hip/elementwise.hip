// prf_div: elementwise "pseudo-reciprocal-free" divide, y != 0 ? x / y : (zero: 0 |
// identity: x) (csrc/ops/cpu/prf_divide.h:8-16), its tensor / scalar forms
// (csrc/ops/cpu/prf_div_kernel.cpp:14-54) and their backward (prf_div_kernel.cpp:258-312:
// g / y and (g / y) * -x / y where y != 0, else g for identity and 0 otherwise; g / c for a
// scalar divisor; g * -c / (y * y) for a scalar dividend).  Memory-bound grid-stride kernels;
// half / bf16 round after every operation as c10::Half / c10::BFloat16 arithmetic does,
// float / double are native.  Outputs may alias inputs (the in-place forms write into x).
#include "common.hpp"

namespace tpw {
namespace {

struct F16 {
    uint16_t bits;
};
struct B16 {
    uint16_t bits;
};

template <typename T>
struct Num {
    using C = T;  // compute type
    __device__ static C load(const T *p, int64_t i) { return p[i]; }
    __device__ static void store(T *p, int64_t i, C v) { p[i] = v; }
    __device__ static C rnd(C v) { return v; }
};
template <>
struct Num<F16> {
    using C = float;
    __device__ static float load(const F16 *p, int64_t i) {
        return (float)__builtin_bit_cast(_Float16, p[i].bits);
    }
    __device__ static void store(F16 *p, int64_t i, float v) {
        p[i].bits = __builtin_bit_cast(uint16_t, (_Float16)v);
    }
    __device__ static float rnd(float v) { return (float)(_Float16)v; }
};
template <>
struct Num<B16> {
    using C = float;
    __device__ static float load(const B16 *p, int64_t i) { return bf16_to_f32(p[i].bits); }
    __device__ static void store(B16 *p, int64_t i, float v) { p[i].bits = f32_to_bf16_rne(v); }
    __device__ static float rnd(float v) { return bf16_to_f32(f32_to_bf16_rne(v)); }
};

template <typename T, bool IDENTITY>
__global__ void prf_div_kernel(const T *x, const T *y, int64_t numel, T *out) {
    using N = Num<T>;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < numel;
         i += (int64_t)gridDim.x * blockDim.x) {
        const auto xv = N::load(x, i), yv = N::load(y, i);
        typename N::C r;
        if (yv != 0) r = N::rnd(xv / yv);
        else r = IDENTITY ? xv : typename N::C(0);
        N::store(out, i, r);
    }
}

template <typename T, bool IDENTITY>
__global__ void prf_div_backward_kernel(const T *g, const T *x, const T *y, int64_t numel, T *gx,
                                        T *gy) {
    using N = Num<T>;
    using C = typename N::C;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < numel;
         i += (int64_t)gridDim.x * blockDim.x) {
        const C gv = N::load(g, i), xv = N::load(x, i), yv = N::load(y, i);
        C a = C(0), bq = C(0);
        if (yv != 0) {
            const C gs = N::rnd(gv / yv);
            a = gs;
            bq = N::rnd(N::rnd(gs * -xv) / yv);
        } else if (IDENTITY) {
            a = gv;
        }
        N::store(gx, i, a);
        N::store(gy, i, bq);
    }
}

// The scalar operand in the element type, rounded as c10::Scalar::to<T>() rounds a double
// (to float first, then to the half type).
template <typename T>
__host__ __device__ typename Num<T>::C scalar_as(double c) {
    return (typename Num<T>::C)c;
}
template <>
__host__ __device__ float scalar_as<F16>(double c) {
    return (float)(_Float16)(float)c;
}
template <>
__host__ __device__ float scalar_as<B16>(double c) {
    const float f = (float)c;
    if (f != f) return f;
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even on the upper 16 bits
    return __builtin_bit_cast(float, u & 0xffff0000u);
}

// SCALAR_FIRST: out = prf_divide(c, x[i]); else out = prf_divide(x[i], c).
template <typename T, bool IDENTITY, bool SCALAR_FIRST>
__global__ void prf_div_scalar_kernel(const T *x, typename Num<T>::C c, int64_t numel, T *out) {
    using N = Num<T>;
    using C = typename N::C;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < numel;
         i += (int64_t)gridDim.x * blockDim.x) {
        const C xv = N::load(x, i);
        const C num = SCALAR_FIRST ? c : xv, den = SCALAR_FIRST ? xv : c;
        C r;
        if (den != 0) r = N::rnd(num / den);
        else r = IDENTITY ? num : C(0);
        N::store(out, i, r);
    }
}

// SCALAR_FIRST (z = c / x): gx = x != 0 ? (g * -c) / (x * x) : 0; else (z = x / c):
// gx = c != 0 ? g / c : (identity ? g : 0).
template <typename T, bool IDENTITY, bool SCALAR_FIRST>
__global__ void prf_div_scalar_backward_kernel(const T *g, const T *x, typename Num<T>::C c,
                                               int64_t numel, T *gx) {
    using N = Num<T>;
    using C = typename N::C;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < numel;
         i += (int64_t)gridDim.x * blockDim.x) {
        const C gv = N::load(g, i);
        C r = C(0);
        if constexpr (SCALAR_FIRST) {
            const C o = N::load(x, i);
            if (o != 0) r = N::rnd(N::rnd(gv * -c) / N::rnd(o * o));
        } else {
            if (c != 0) r = N::rnd(gv / c);
            else if (IDENTITY) r = gv;
        }
        N::store(gx, i, r);
    }
}

unsigned grid_for(int64_t numel) {
    int64_t blocks = cdiv(numel, 256);
    return (unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

template <typename T>
int launch_fwd(const void *x, const void *y, int64_t numel, int identity, void *out, hipStream_t s) {
    auto *X = static_cast<const T *>(x);
    auto *Y = static_cast<const T *>(y);
    auto *O = static_cast<T *>(out);
    if (identity) hipLaunchKernelGGL((prf_div_kernel<T, true>), dim3(grid_for(numel)), dim3(256), 0, s, X, Y, numel, O);
    else hipLaunchKernelGGL((prf_div_kernel<T, false>), dim3(grid_for(numel)), dim3(256), 0, s, X, Y, numel, O);
    return check_launch("prf_div_kernel");
}

template <typename T>
int launch_bwd(const void *g, const void *x, const void *y, int64_t numel, int identity, void *gx,
               void *gy, hipStream_t s) {
    auto *G = static_cast<const T *>(g);
    auto *X = static_cast<const T *>(x);
    auto *Y = static_cast<const T *>(y);
    if (identity) hipLaunchKernelGGL((prf_div_backward_kernel<T, true>), dim3(grid_for(numel)), dim3(256), 0, s, G, X, Y, numel, static_cast<T *>(gx), static_cast<T *>(gy));
    else hipLaunchKernelGGL((prf_div_backward_kernel<T, false>), dim3(grid_for(numel)), dim3(256), 0, s, G, X, Y, numel, static_cast<T *>(gx), static_cast<T *>(gy));
    return check_launch("prf_div_backward_kernel");
}

template <typename T>
int launch_scalar(const void *x, double c, int64_t numel, int identity, int scalar_first, void *out,
                  hipStream_t s) {
    auto *X = static_cast<const T *>(x);
    auto *O = static_cast<T *>(out);
    const auto cv = scalar_as<T>(c);
    const dim3 grid(grid_for(numel)), block(256);
    if (scalar_first) {
        if (identity) hipLaunchKernelGGL((prf_div_scalar_kernel<T, true, true>), grid, block, 0, s, X, cv, numel, O);
        else hipLaunchKernelGGL((prf_div_scalar_kernel<T, false, true>), grid, block, 0, s, X, cv, numel, O);
    } else {
        if (identity) hipLaunchKernelGGL((prf_div_scalar_kernel<T, true, false>), grid, block, 0, s, X, cv, numel, O);
        else hipLaunchKernelGGL((prf_div_scalar_kernel<T, false, false>), grid, block, 0, s, X, cv, numel, O);
    }
    return check_launch("prf_div_scalar_kernel");
}

template <typename T>
int launch_scalar_bwd(const void *g, const void *x, double c, int64_t numel, int identity,
                      int scalar_first, void *gx, hipStream_t s) {
    auto *G = static_cast<const T *>(g);
    auto *X = static_cast<const T *>(x);
    auto *GX = static_cast<T *>(gx);
    const auto cv = scalar_as<T>(c);
    const dim3 grid(grid_for(numel)), block(256);
    if (scalar_first) {
        hipLaunchKernelGGL((prf_div_scalar_backward_kernel<T, false, true>), grid, block, 0, s, G, X, cv, numel, GX);
    } else {
        if (identity) hipLaunchKernelGGL((prf_div_scalar_backward_kernel<T, true, false>), grid, block, 0, s, G, X, cv, numel, GX);
        else hipLaunchKernelGGL((prf_div_scalar_backward_kernel<T, false, false>), grid, block, 0, s, G, X, cv, numel, GX);
    }
    return check_launch("prf_div_scalar_backward_kernel");
}

}  // namespace
}  // namespace tpw

using namespace tpw;

extern "C" int tpw_prf_div(const void *x, const void *y, int dtype, int64_t numel, int identity,
                           void *out, void *stream) {
    TPW_REQUIRE(numel >= 0, "invalid numel");
    if (numel == 0) return TPW_OK;
    TPW_REQUIRE(x && y && out, "null pointer");
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case TPW_F32: return launch_fwd<float>(x, y, numel, identity, out, s);
        case TPW_F64: return launch_fwd<double>(x, y, numel, identity, out, s);
        case TPW_F16: return launch_fwd<F16>(x, y, numel, identity, out, s);
        case TPW_BF16: return launch_fwd<B16>(x, y, numel, identity, out, s);
        default: tpw::set_error("prf_div: unsupported dtype %d", dtype); return TPW_ERR_INVALID;
    }
}

extern "C" int tpw_prf_div_backward(const void *grad, const void *x, const void *y, int dtype,
                                    int64_t numel, int identity, void *grad_x, void *grad_y,
                                    void *stream) {
    TPW_REQUIRE(numel >= 0, "invalid numel");
    if (numel == 0) return TPW_OK;
    TPW_REQUIRE(grad && x && y && grad_x && grad_y, "null pointer");
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case TPW_F32: return launch_bwd<float>(grad, x, y, numel, identity, grad_x, grad_y, s);
        case TPW_F64: return launch_bwd<double>(grad, x, y, numel, identity, grad_x, grad_y, s);
        case TPW_F16: return launch_bwd<F16>(grad, x, y, numel, identity, grad_x, grad_y, s);
        case TPW_BF16: return launch_bwd<B16>(grad, x, y, numel, identity, grad_x, grad_y, s);
        default: tpw::set_error("prf_div: unsupported dtype %d", dtype); return TPW_ERR_INVALID;
    }
}

extern "C" int tpw_prf_div_scalar(const void *x, double c, int dtype, int64_t numel, int identity,
                                  int scalar_first, void *out, void *stream) {
    TPW_REQUIRE(numel >= 0, "invalid numel");
    if (numel == 0) return TPW_OK;
    TPW_REQUIRE(x && out, "null pointer");
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case TPW_F32: return launch_scalar<float>(x, c, numel, identity, scalar_first, out, s);
        case TPW_F64: return launch_scalar<double>(x, c, numel, identity, scalar_first, out, s);
        case TPW_F16: return launch_scalar<F16>(x, c, numel, identity, scalar_first, out, s);
        case TPW_BF16: return launch_scalar<B16>(x, c, numel, identity, scalar_first, out, s);
        default: tpw::set_error("prf_div: unsupported dtype %d", dtype); return TPW_ERR_INVALID;
    }
}

extern "C" int tpw_prf_div_scalar_backward(const void *grad, const void *x, double c, int dtype,
                                           int64_t numel, int identity, int scalar_first,
                                           void *grad_x, void *stream) {
    TPW_REQUIRE(numel >= 0, "invalid numel");
    if (numel == 0) return TPW_OK;
    TPW_REQUIRE(grad && grad_x && (x || !scalar_first), "null pointer");
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case TPW_F32: return launch_scalar_bwd<float>(grad, x, c, numel, identity, scalar_first, grad_x, s);
        case TPW_F64: return launch_scalar_bwd<double>(grad, x, c, numel, identity, scalar_first, grad_x, s);
        case TPW_F16: return launch_scalar_bwd<F16>(grad, x, c, numel, identity, scalar_first, grad_x, s);
        case TPW_BF16: return launch_scalar_bwd<B16>(grad, x, c, numel, identity, scalar_first, grad_x, s);
        default: tpw::set_error("prf_div: unsupported dtype %d", dtype); return TPW_ERR_INVALID;
    }
}
