// Squared Mahalanobis distance d^T VI d with d = x1[i] - x2[j]
// (reference: csrc/ops/cpu/sqmahalanobis_kernel.cpp:13-33, an O(d^2) loop per pair).
//
// Here VI d = VI x1[i] - VI x2[j], so with the per-row projections P = x VI^T (one small
// product per row, O(rows d^2) in total) the per-pair work is O(d):
//
//     out[i, j] = sum_k (x1[i,k] - x2[j,k]) * (P1[i,k] - P2[j,k]).
//
// The difference is formed before the product, as in the reference, so identical rows give
// exactly 0 and near rows keep their relative accuracy.  For float the projections are
// computed in double and carried as two floats (hi = rn(P), lo = rn(P - hi)); the pair term
// uses (hi1 - hi2) + (lo1 - lo2), which is exact to a few float roundings of the true
// VI d even when the rows nearly coincide (hi1 - hi2 is then exact).  Double inputs keep P in
// double.  A register-tiled VALU kernel does the pairs: 64 x 64 outputs per 256-thread block,
// 4 x 4 per thread, 16-feature chunks of the six operand panels staged feature-major in LDS.
#include <type_traits>

#include "common.hpp"

namespace tpw {
namespace {

constexpr int kTile = 64, kKC = 16, kPad = 68;  // LDS row stride: 16-byte aligned float4 reads

// P[r, k] = sum_l x[r, l] * VI[b, k, l] in double; float: hi / lo split, double: hi only.
template <typename T>
__global__ void project_kernel(const T *__restrict__ x, const T *__restrict__ VI, int64_t rows_per_batch,
                               int64_t total, int64_t d, T *__restrict__ hi, T *__restrict__ lo) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total * d) return;
    const int64_t r = t / d, k = t - r * d, b = r / rows_per_batch;
    const T *xr = x + r * d, *vk = VI + (b * d + k) * d;
    double s = 0.0;
    for (int64_t l = 0; l < d; ++l) s = fma((double)xr[l], (double)vk[l], s);
    const T h = (T)s;
    hi[t] = h;
    if (lo) lo[t] = (T)(s - (double)h);
}

template <typename T>
struct Vec4;
template <>
struct Vec4<float> {
    typedef float type __attribute__((ext_vector_type(4)));
};
template <>
struct Vec4<double> {
    typedef double type __attribute__((ext_vector_type(4)));
};

// out[b, i, j] = sum_k (a[i,k] - c[j,k]) * ((ha[i,k] - hc[j,k]) + (la[i,k] - lc[j,k]))
template <typename T, bool LO>
__global__ __launch_bounds__(256) void mahalanobis_pairs_kernel(
    const T *__restrict__ x1, const T *__restrict__ h1, const T *__restrict__ l1, const T *__restrict__ x2,
    const T *__restrict__ h2, const T *__restrict__ l2, int64_t n, int64_t m, int64_t d, T *__restrict__ out) {
    using V4 = typename Vec4<T>::type;
    constexpr int kPanels = LO ? 3 : 2;
    __shared__ __align__(16) T sa[kPanels][kKC][kPad];
    __shared__ __align__(16) T sc[kPanels][kKC][kPad];
    const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
    const int64_t b = blockIdx.z, i0 = (int64_t)blockIdx.y * kTile, j0 = (int64_t)blockIdx.x * kTile;
    const T *A[3] = {x1 + b * n * d, h1 + b * n * d, LO ? l1 + b * n * d : nullptr};
    const T *C[3] = {x2 + b * m * d, h2 + b * m * d, LO ? l2 + b * m * d : nullptr};
    T acc[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] = T(0);

    for (int64_t k0 = 0; k0 < d; k0 += kKC) {
        // stage: 64 rows x 16 features of every panel, feature-major; zero past the edges
#pragma unroll
        for (int e = tid; e < kTile * kKC; e += 256) {
            const int row = e / kKC, kk = e % kKC;
            const int64_t k = k0 + kk;
            const bool ka = k < d;
            const bool ra = i0 + row < n, rc = j0 + row < m;
#pragma unroll
            for (int p = 0; p < kPanels; ++p) {
                sa[p][kk][row] = (ra && ka) ? A[p][(i0 + row) * d + k] : T(0);
                sc[p][kk][row] = (rc && ka) ? C[p][(j0 + row) * d + k] : T(0);
            }
        }
        __syncthreads();
#pragma unroll 4
        for (int kk = 0; kk < kKC; ++kk) {
            const V4 xa = *reinterpret_cast<const V4 *>(&sa[0][kk][tr * 4]);
            const V4 ha = *reinterpret_cast<const V4 *>(&sa[1][kk][tr * 4]);
            const V4 xc = *reinterpret_cast<const V4 *>(&sc[0][kk][tc * 4]);
            const V4 hc = *reinterpret_cast<const V4 *>(&sc[1][kk][tc * 4]);
            V4 la = {0, 0, 0, 0}, lc = {0, 0, 0, 0};
            if constexpr (LO) {
                la = *reinterpret_cast<const V4 *>(&sa[2][kk][tr * 4]);
                lc = *reinterpret_cast<const V4 *>(&sc[2][kk][tc * 4]);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const T dk = xa[r] - xc[c];
                    T u = ha[r] - hc[c];
                    if constexpr (LO) u += la[r] - lc[c];
                    acc[r][c] = fma(dk, u, acc[r][c]);
                }
        }
        __syncthreads();
    }
    T *o = out + b * n * m;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t i = i0 + tr * 4 + r;
        if (i >= n) continue;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int64_t j = j0 + tc * 4 + c;
            if (j < m) o[i * m + j] = acc[r][c];
        }
    }
}

size_t ws_elems(int64_t batch, int64_t n, int64_t m, int64_t d, bool lo) {
    return (size_t)(lo ? 2 : 1) * (size_t)(batch * (n + m) * d);
}

template <typename T>
int run(const T *x1, const T *x2, const T *VI, int64_t batch, int64_t n, int64_t m, int64_t d, T *out,
        void *workspace, hipStream_t s) {
    constexpr bool LO = std::is_same_v<T, float>;
    T *w = static_cast<T *>(workspace);
    T *h1 = w, *h2 = h1 + batch * n * d;
    T *l1 = LO ? h2 + batch * m * d : nullptr, *l2 = LO ? l1 + batch * n * d : nullptr;
    const bool same = x1 == x2 && n == m;
    if (d > 0) {  // d == 0: the empty sum; the pair kernel reads no panel and writes zeros
        hipLaunchKernelGGL(project_kernel<T>, dim3((unsigned)cdiv(batch * n * d, 256)), dim3(256), 0, s, x1, VI,
                           n, batch * n, d, h1, l1);
        if (!same)
            hipLaunchKernelGGL(project_kernel<T>, dim3((unsigned)cdiv(batch * m * d, 256)), dim3(256), 0, s, x2,
                               VI, m, batch * m, d, h2, l2);
    }
    if (same) {
        h2 = h1;
        l2 = l1;
    }
    const dim3 grid((unsigned)cdiv(m, kTile), (unsigned)cdiv(n, kTile), (unsigned)batch);
    hipLaunchKernelGGL((mahalanobis_pairs_kernel<T, LO>), grid, dim3(256), 0, s, x1, h1, l1, x2, h2, l2, n, m, d,
                       out);
    return check_launch("mahalanobis_pairs_kernel");
}

}  // namespace
}  // namespace tpw

using namespace tpw;

extern "C" size_t tpw_sqmahalanobis_workspace_size(int dtype, int64_t batch, int64_t n, int64_t m, int64_t d) {
    if (batch < 0 || n < 0 || m < 0 || d < 0) return 0;
    if (dtype == TPW_F32) return 4 * ws_elems(batch, n, m, d, true);
    if (dtype == TPW_F64) return 8 * ws_elems(batch, n, m, d, false);
    return 0;
}

extern "C" int tpw_sqmahalanobis(const void *x1, const void *x2, const void *VI, int dtype, int64_t batch,
                                 int64_t n, int64_t m, int64_t d, void *out, void *workspace, void *stream) {
    TPW_REQUIRE(dtype == TPW_F32 || dtype == TPW_F64, "sqmahalanobis: dtype must be TPW_F32 or TPW_F64 (got %d)",
                dtype);
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(out && (d == 0 || (x1 && x2 && VI && workspace)), "null pointer");
    TPW_REQUIRE(cdiv(n, kTile) <= kMaxGridYZ && batch <= kMaxGridYZ && cdiv(m, kTile) <= 0x7fffffffLL,
                "sizes exceed the launch grid");
    hipStream_t s = as_stream(stream);
    if (dtype == TPW_F32)
        return run<float>(static_cast<const float *>(x1), static_cast<const float *>(x2),
                          static_cast<const float *>(VI), batch, n, m, d, static_cast<float *>(out), workspace, s);
    return run<double>(static_cast<const double *>(x1), static_cast<const double *>(x2),
                       static_cast<const double *>(VI), batch, n, m, d, static_cast<double *>(out), workspace, s);
}
