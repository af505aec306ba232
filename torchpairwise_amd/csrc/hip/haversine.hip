// Haversine distances between points given as (latitude, longitude) in radians, and their
// gradient (the reference's _haversine / __haversine_backward, cpu/haversine_kernel.cpp).
//
//   out[i,j] = 2 asin(sqrt(sin^2((lat_i - lat_j) / 2) + cos lat_i cos lat_j sin^2((lon_i - lon_j) / 2)))
//
// D is 2, so there is no feature loop to tile: the forward is one thread per output with the
// points' latitude sines / cosines precomputed once, each output written once (non-temporal).  The backward follows
// the reference's formulas: grad_x1 row i sums over j (one wave per row, lanes over j, a
// fixed-shape wave reduction), grad_x2 column j sums over i (one thread per column, i in
// order).  Both are deterministic.
#include "common.hpp"

#include <math.h>

namespace tpw {
namespace {

// sin / cos of the latitude of every point: sc[r] = (sin lat, cos lat)
__global__ void lat_trig_kernel(const float *__restrict__ x, int64_t rows, float2 *__restrict__ sc) {
    const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (r >= rows) return;
    float s, c;
    sincosf(x[2 * r], &s, &c);
    sc[r] = make_float2(s, c);
}

__device__ __forceinline__ float hav_val(float lat1, float lon1, float c1, float lat2, float lon2,
                                         float c2) {
    const float sa = sinf((lat1 - lat2) * 0.5f), so = sinf((lon1 - lon2) * 0.5f);
    return sa * sa + c1 * c2 * (so * so);
}

// out[b, i, j]; block 64 x 4 threads covers 4 rows x 64 columns.
__global__ __launch_bounds__(256) void haversine_kernel(const float *__restrict__ x1,
                                                        const float *__restrict__ x2,
                                                        const float2 *__restrict__ sc1,
                                                        const float2 *__restrict__ sc2, int64_t n,
                                                        int64_t m, float *__restrict__ out) {
    const int64_t b = blockIdx.z;
    const int64_t i = (int64_t)blockIdx.y * 4 + (threadIdx.x >> 6);
    const int64_t j = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
    if (i >= n || j >= m) return;
    const float *p = x1 + (b * n + i) * 2, *q = x2 + (b * m + j) * 2;
    const float v = hav_val(p[0], p[1], sc1[b * n + i].y, q[0], q[1], sc2[b * m + j].y);
    store_nt(out + (b * n + i) * m + j, 2.0f * asinf(sqrtf(v)));
}

__global__ void zero_kernel(float *__restrict__ p, int64_t len) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t < len) p[t] = 0.0f;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Per-pair factor g / (sqrt(val) sqrt(1 - val)) and the pair's trigonometric terms.
struct PairTerms {
    float w, so, co, sd;  // weight, sin(dlon/2), cos(dlon/2), sin(dlat)
};
__device__ __forceinline__ PairTerms pair_terms(float g, float lat1, float lon1, float c1, float lat2,
                                                float lon2, float c2) {
    PairTerms t;
    const float sa = sinf((lat1 - lat2) * 0.5f);
    sincosf((lon1 - lon2) * 0.5f, &t.so, &t.co);
    const float val = sa * sa + c1 * c2 * (t.so * t.so);
    t.w = g / (sqrtf(val) * sqrtf(1.0f - val));
    t.sd = sinf(lat1 - lat2);
    return t;
}

// grad_x1[b, i, :]: one wave per row i (4 rows per block), lanes stride over j.
__global__ __launch_bounds__(256) void haversine_grad_x1_kernel(
    const float *__restrict__ g, const float *__restrict__ x1, const float *__restrict__ x2,
    const float2 *__restrict__ sc1, const float2 *__restrict__ sc2, int64_t n, int64_t m,
    float *__restrict__ gx1) {
    const int64_t b = blockIdx.y;
    const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (i >= n) return;
    const float lat1 = x1[(b * n + i) * 2], lon1 = x1[(b * n + i) * 2 + 1];
    const float s1 = sc1[b * n + i].x, c1 = sc1[b * n + i].y;
    float dlat = 0.0f, dlon = 0.0f;
    for (int64_t j = lane; j < m; j += 64) {
        const float lat2 = x2[(b * m + j) * 2], lon2 = x2[(b * m + j) * 2 + 1];
        const float c2 = sc2[b * m + j].y;
        const PairTerms t = pair_terms(g[(b * n + i) * m + j], lat1, lon1, c1, lat2, lon2, c2);
        dlat += t.w * (-s1 * (t.so * t.so) * c2 + t.sd * 0.5f);   // haversine_kernel.cpp:111-113
        dlon += t.w * (t.so * c1 * c2 * t.co);                    // :114-116
    }
    dlat = wave_sum(dlat);
    dlon = wave_sum(dlon);
    if (lane == 0) {
        gx1[(b * n + i) * 2] = dlat;
        gx1[(b * n + i) * 2 + 1] = dlon;
    }
}

// grad_x2[b, j, :]: one thread per column j, i in order (coalesced along j).
__global__ __launch_bounds__(256) void haversine_grad_x2_kernel(
    const float *__restrict__ g, const float *__restrict__ x1, const float *__restrict__ x2,
    const float2 *__restrict__ sc1, const float2 *__restrict__ sc2, int64_t n, int64_t m,
    float *__restrict__ gx2) {
    const int64_t b = blockIdx.y;
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= m) return;
    const float lat2 = x2[(b * m + j) * 2], lon2 = x2[(b * m + j) * 2 + 1];
    const float s2 = sc2[b * m + j].x, c2 = sc2[b * m + j].y;
    float dlat = 0.0f, dlon = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        const float lat1 = x1[(b * n + i) * 2], lon1 = x1[(b * n + i) * 2 + 1];
        const float c1 = sc1[b * n + i].y;
        const PairTerms t = pair_terms(g[(b * n + i) * m + j], lat1, lon1, c1, lat2, lon2, c2);
        dlat += t.w * (-s2 * (t.so * t.so) * c1 - t.sd * 0.5f);   // haversine_kernel.cpp:138-140
        dlon += t.w * (-t.so * c1 * c2 * t.co);                   // :141-143
    }
    gx2[(b * m + j) * 2] = dlat;
    gx2[(b * m + j) * 2 + 1] = dlon;
}

int launch_trig(const float *x, int64_t rows, float2 *sc, hipStream_t s) {
    if (rows == 0) return TPW_OK;
    hipLaunchKernelGGL(lat_trig_kernel, dim3((unsigned)cdiv(rows, 256)), dim3(256), 0, s, x, rows, sc);
    return check_launch("lat_trig_kernel");
}

}  // namespace
}  // namespace tpw

using namespace tpw;

extern "C" size_t tpw_haversine_workspace_size(int64_t batch, int64_t n, int64_t m) {
    return sizeof(float2) * (size_t)(batch * (n + m)) + 256;
}

extern "C" int tpw_haversine(const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m,
                             float *out, void *workspace, void *stream) {
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0, "invalid sizes");
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out && workspace, "null pointer");
    TPW_REQUIRE(cdiv(n, 4) <= kMaxGridYZ && batch <= kMaxGridYZ, "too many rows or batches");
    hipStream_t s = as_stream(stream);
    float2 *sc1 = static_cast<float2 *>(workspace), *sc2 = sc1 + batch * n;
    int rc = launch_trig(x1, batch * n, sc1, s);
    if (rc == TPW_OK) rc = launch_trig(x2, batch * m, sc2, s);
    if (rc != TPW_OK) return rc;
    hipLaunchKernelGGL(haversine_kernel, dim3((unsigned)cdiv(m, 64), (unsigned)cdiv(n, 4), (unsigned)batch),
                       dim3(256), 0, s, x1, x2, sc1, sc2, n, m, out);
    return check_launch("haversine_kernel");
}

extern "C" int tpw_haversine_backward(const float *grad, const float *x1, const float *x2,
                                      int64_t batch, int64_t n, int64_t m, float *grad_x1,
                                      float *grad_x2, void *workspace, void *stream) {
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0, "invalid sizes");
    if (batch == 0 || (n == 0 && m == 0)) return TPW_OK;
    TPW_REQUIRE(cdiv(n, 4) <= 0x7fffffffLL && batch <= kMaxGridYZ, "too many rows or batches");
    hipStream_t s = as_stream(stream);
    if (n == 0 || m == 0) {  // nothing to sum: zero gradients (the empty side may be null)
        float *g = n ? grad_x1 : grad_x2;
        const int64_t len = 2 * batch * (n ? n : m);
        TPW_REQUIRE(g, "null pointer");
        hipLaunchKernelGGL(zero_kernel, dim3((unsigned)cdiv(len, 256)), dim3(256), 0, s, g, len);
        return check_launch("zero_kernel");
    }
    TPW_REQUIRE(grad && x1 && x2 && grad_x1 && grad_x2 && workspace, "null pointer");
    float2 *sc1 = static_cast<float2 *>(workspace), *sc2 = sc1 + batch * n;
    int rc = launch_trig(x1, batch * n, sc1, s);
    if (rc == TPW_OK) rc = launch_trig(x2, batch * m, sc2, s);
    if (rc != TPW_OK) return rc;
    hipLaunchKernelGGL(haversine_grad_x1_kernel, dim3((unsigned)cdiv(n, 4), (unsigned)batch), dim3(256), 0, s,
                       grad, x1, x2, sc1, sc2, n, m, grad_x1);
    rc = check_launch("haversine_grad_x1_kernel");
    if (rc != TPW_OK) return rc;
    hipLaunchKernelGGL(haversine_grad_x2_kernel, dim3((unsigned)cdiv(m, 256), (unsigned)batch), dim3(256), 0, s,
                       grad, x1, x2, sc1, sc2, n, m, grad_x2);
    return check_launch("haversine_grad_x2_kernel");
}
