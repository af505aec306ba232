// Pairwise equal / not-equal counts for non-bool element types (pweq_*/pwne_* and
// hamming_distances on integer or floating inputs, which the reference compares with ==/!=
// without a bool coercion: csrc/ops/common/binary_ops.h, pairwise_metrics.cpp:206-213).
//
// 256-thread blocks own a 64 x 64 output tile; both panels are staged in LDS feature-major
// as the native element type; each thread owns 4 x 4 outputs and counts in uint32.  Floating
// types compare by value (so -0 == +0 and NaN != NaN, as C++ ==/!= do).  The epilogue is the
// float accumulator / mean of the bit-packed path.
#include "common.hpp"

namespace tpw {
namespace {

constexpr int kT = 64;
constexpr int kK = 32;
constexpr uint32_t kFloatExactLimit = 1u << 24;

template <typename T>
struct Cmp {
    __device__ static bool eq(T a, T b) { return a == b; }
};
struct Half {
    uint16_t bits;
};
struct BF16 {
    uint16_t bits;
};
__device__ __forceinline__ float half_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}
template <>
struct Cmp<Half> {
    __device__ static bool eq(Half a, Half b) { return half_to_f32(a.bits) == half_to_f32(b.bits); }
};
template <>
struct Cmp<BF16> {
    __device__ static bool eq(BF16 a, BF16 b) { return bf16_to_f32(a.bits) == bf16_to_f32(b.bits); }
};

template <typename T, bool NE, bool MEAN>
__global__ __launch_bounds__(256) void compare_reduce_kernel(const T *__restrict__ x1,
                                                             const T *__restrict__ x2, int64_t n,
                                                             int64_t m, int64_t d, double inv_d,
                                                             float *__restrict__ out) {
    __shared__ T As[kK][kT + 1];
    __shared__ T Bs[kK][kT + 1];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int64_t b = blockIdx.z;
    const int64_t row0 = (int64_t)blockIdx.y * kT, col0 = (int64_t)blockIdx.x * kT;
    const T *A = x1 + b * n * d;
    const T *B = x2 + b * m * d;
    uint32_t acc[4][4] = {};
    for (int64_t k0 = 0; k0 < d; k0 += kK) {
#pragma unroll
        for (int q = 0; q < (kT * kK) / 256; ++q) {
            const int idx = tid + 256 * q;
            const int r = idx / kK, kk = idx % kK;
            const int64_t gk = k0 + kk;
            T va{}, vb{};
            if (row0 + r < n && gk < d) va = A[(row0 + r) * d + gk];
            if (col0 + r < m && gk < d) vb = B[(col0 + r) * d + gk];
            As[kk][r] = va;
            Bs[kk][r] = vb;
        }
        __syncthreads();
        const int kmax = d - k0 < kK ? (int)(d - k0) : kK;
        for (int kk = 0; kk < kmax; ++kk) {
            T a[4], bv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) a[r] = As[kk][4 * ty + r];
#pragma unroll
            for (int c = 0; c < 4; ++c) bv[c] = Bs[kk][4 * tx + c];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[r][c] += Cmp<T>::eq(a[r], bv[c]) ? 0u : 1u;
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t row = row0 + 4 * ty + r;
        if (row >= n) continue;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int64_t col = col0 + 4 * tx + c;
            if (col >= m) continue;
            uint32_t cnt = acc[r][c];  // not-equal count
            if (!NE) cnt = (uint32_t)d - cnt;
            float v;
            if (!MEAN) {
                v = (float)(cnt < kFloatExactLimit ? cnt : kFloatExactLimit);
            } else if (inv_d > 0.0) {
                v = (float)((double)cnt * inv_d);
            } else {
                v = __fdiv_rn((float)(cnt < kFloatExactLimit ? cnt : kFloatExactLimit), (float)d);
            }
            out[(b * n + row) * m + col] = v;
        }
    }
}

template <typename T>
int launch(const void *x1, const void *x2, int64_t batch, int64_t n, int64_t m, int64_t d,
           bool ne, bool mean, float *out, hipStream_t s) {
    dim3 grid((unsigned)cdiv(m, kT), (unsigned)cdiv(n, kT), (unsigned)batch);
    const double inv_d = d < (int64_t)kFloatExactLimit ? 1.0 / (double)d : 0.0;
    const T *a = static_cast<const T *>(x1);
    const T *b = static_cast<const T *>(x2);
    if (ne && mean) hipLaunchKernelGGL((compare_reduce_kernel<T, true, true>), grid, dim3(256), 0, s, a, b, n, m, d, inv_d, out);
    else if (ne) hipLaunchKernelGGL((compare_reduce_kernel<T, true, false>), grid, dim3(256), 0, s, a, b, n, m, d, inv_d, out);
    else if (mean) hipLaunchKernelGGL((compare_reduce_kernel<T, false, true>), grid, dim3(256), 0, s, a, b, n, m, d, inv_d, out);
    else hipLaunchKernelGGL((compare_reduce_kernel<T, false, false>), grid, dim3(256), 0, s, a, b, n, m, d, inv_d, out);
    return check_launch("compare_reduce_kernel");
}

}  // namespace
}  // namespace tpw

using namespace tpw;

extern "C" int tpw_compare_reduce(const void *x1, const void *x2, int elem_type, int64_t batch,
                                  int64_t n, int64_t m, int64_t d, int op, int reduction,
                                  float *out, void *stream) {
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 1, "invalid sizes");
    TPW_REQUIRE(op == TPW_BIT_EQ || op == TPW_BIT_NE, "tpw_compare_reduce supports EQ and NE only");
    TPW_REQUIRE(reduction == TPW_RED_SUM || reduction == TPW_RED_MEAN, "unknown reduction %d", reduction);
    TPW_REQUIRE(cdiv(n, kT) <= kMaxGridYZ && batch <= kMaxGridYZ, "too many rows or batches");
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    const bool ne = op == TPW_BIT_NE, mean = reduction == TPW_RED_MEAN;
    hipStream_t s = as_stream(stream);
    switch (elem_type) {
        case TPW_F32: return launch<float>(x1, x2, batch, n, m, d, ne, mean, out, s);
        case TPW_BF16: return launch<BF16>(x1, x2, batch, n, m, d, ne, mean, out, s);
        case TPW_F16: return launch<Half>(x1, x2, batch, n, m, d, ne, mean, out, s);
        case TPW_F64: return launch<double>(x1, x2, batch, n, m, d, ne, mean, out, s);
        case TPW_I8: return launch<int8_t>(x1, x2, batch, n, m, d, ne, mean, out, s);
        case TPW_U8: return launch<uint8_t>(x1, x2, batch, n, m, d, ne, mean, out, s);
        case TPW_I16: return launch<int16_t>(x1, x2, batch, n, m, d, ne, mean, out, s);
        case TPW_I32: return launch<int32_t>(x1, x2, batch, n, m, d, ne, mean, out, s);
        case TPW_I64: return launch<int64_t>(x1, x2, batch, n, m, d, ne, mean, out, s);
        default: tpw::set_error("unsupported element type %d", elem_type); return TPW_ERR_INVALID;
    }
}
