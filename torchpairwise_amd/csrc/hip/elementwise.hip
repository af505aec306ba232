// prf_div: elementwise "pseudo-reciprocal-free" divide, y != 0 ? x / y : (zero: 0 |
// identity: x) (csrc/ops/cpu/prf_divide.h:8-16), and its backward (csrc/ops/cpu/
// prf_div_kernel.cpp:258-277: g / y and (g / y) * -x / y where y != 0; else g for identity,
// 0 otherwise).  Memory-bound grid-stride kernels; half / bf16 round after every operation
// as c10::Half / c10::BFloat16 arithmetic does, float / double are native.
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
__global__ void prf_div_kernel(const T *__restrict__ x, const T *__restrict__ y, int64_t numel,
                               T *__restrict__ out) {
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
__global__ void prf_div_backward_kernel(const T *__restrict__ g, const T *__restrict__ x,
                                        const T *__restrict__ y, int64_t numel,
                                        T *__restrict__ gx, T *__restrict__ gy) {
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
