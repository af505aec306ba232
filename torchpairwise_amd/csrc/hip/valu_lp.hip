// Non-GEMM pairwise reductions on the VALU: Minkowski distances for p = 0, 1, 2, 3, inf and
// general p, and their gradient (at::_cdist_forward / at::_cdist_backward semantics).
//
// Forward: 256-thread blocks own a 128 x 128 output tile; thread (ty, tx) owns rows
// 8 ty + r (r < 8) and columns 64 h + 4 tx + c (h < 2, c < 4).  Both operand panels are
// staged in LDS feature-major ([k][row], 4-float pad), so one k step costs a thread four
// 16-byte LDS reads (8 x1 values broadcast over tx, 8 x2 values) for 64 pair-features.
// Per pair-feature the VALU does a subtract and an abs-modified accumulate (p = 1: add,
// p = inf: max), three ops for p = 3 (d * |d| fused into the accumulate), one exp2/log2
// pair more for general p.  Stores are non-temporal float4 rows (256 B per 16 lanes).
//
// Backward (grad of x1; x2 by the transposed call): out[i,k] = sum_j F(x1[i,k] - x2[j,k],
// g[i,j], dist[i,j]).  A block owns 128 rows x 64 features with its x1 values held in
// registers, streams 32 j at a time (x2 panel [j][k] and the per-pair weight
// w = g / dist^(p-1) computed while staging into LDS), thread block 8 rows x 4 features.
// The j range is split over several blocks when the row/feature grid alone would not fill
// the GPU; the per-split partial sums are then added in split order by a second kernel,
// so the result is deterministic.
#include <math.h>

#include "common.hpp"

namespace tpw {
namespace {

enum PKind { kP0 = 0, kP1, kP2, kP3, kPInf, kPLt2, kPGen };

constexpr int kThreads = 256;
constexpr int kTile = 128;
constexpr int kBK = 32;
constexpr int kPad = 4;

template <int PK>
__device__ __forceinline__ float lp_step(float acc, float a, float b, float p) {
    const float d = a - b;
    if constexpr (PK == kP1) return acc + fabsf(d);
    else if constexpr (PK == kPInf) return fmaxf(acc, fabsf(d));
    else if constexpr (PK == kP2) return fmaf(d, d, acc);
    else if constexpr (PK == kP3) return fmaf(d * d, fabsf(d), acc);
    else if constexpr (PK == kP0) return acc + (d != 0.0f ? 1.0f : 0.0f);
    else return acc + exp2f(p * __log2f(fabsf(d)));
}

template <int PK>
__device__ __forceinline__ float lp_finish(float acc, float inv_p) {
    if constexpr (PK == kP2) return sqrt_rn(acc);
    else if constexpr (PK == kP3) return cbrtf(acc);
    else if constexpr (PK == kPGen || PK == kPLt2) return powf(acc, inv_p);
    else return acc;
}

template <int PK, bool VEC>
__global__ __launch_bounds__(kThreads, 2) void lp_forward_kernel(
    const float *__restrict__ x1, const float *__restrict__ x2, int64_t n, int64_t m, int64_t d,
    float p, float inv_p, float *__restrict__ out, int64_t tiles_m) {
    __shared__ float As[kBK][kTile + kPad];
    __shared__ float Bs[kBK][kTile + kPad];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int64_t b = blockIdx.z;
    const int64_t row0 = (int64_t)blockIdx.y * kTile, col0 = (int64_t)blockIdx.x * kTile;
    const float *A = x1 + b * n * d;
    const float *B = x2 + b * m * d;

    float acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.0f;

    // staging: 128 rows x 32 features per operand = 1024 float4, 4 per thread
    auto load = [&](const float *X, int64_t rows, int64_t r0, int64_t k0, floatx4 (&v)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int idx = tid + kThreads * q;
            const int r = idx >> 3, c4 = idx & 7;
            const int64_t gr = r0 + r, gk = k0 + 4 * c4;
            floatx4 t = {0.0f, 0.0f, 0.0f, 0.0f};
            if (gr < rows) {
                const float *src = X + gr * d + gk;
                if constexpr (VEC) {
                    if (gk < d) t = *reinterpret_cast<const floatx4 *>(src);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (gk + e < d) t[e] = src[e];
                }
            }
            v[q] = t;
        }
    };
    floatx4 pa[4], pb[4];
    load(A, n, row0, 0, pa);
    load(B, m, col0, 0, pb);
    for (int64_t k0 = 0; k0 < d; k0 += kBK) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int idx = tid + kThreads * q;
            const int r = idx >> 3, c4 = idx & 7;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                As[4 * c4 + e][r] = pa[q][e];
                Bs[4 * c4 + e][r] = pb[q][e];
            }
        }
        __syncthreads();
        if (k0 + kBK < d) {
            load(A, n, row0, k0 + kBK, pa);
            load(B, m, col0, k0 + kBK, pb);
        }
        const int kmax = d - k0 < kBK ? (int)(d - k0) : kBK;
        for (int k = 0; k < kmax; ++k) {
            const floatx4 a0 = *reinterpret_cast<const floatx4 *>(&As[k][8 * ty]);
            const floatx4 a1 = *reinterpret_cast<const floatx4 *>(&As[k][8 * ty + 4]);
            const floatx4 b0 = *reinterpret_cast<const floatx4 *>(&Bs[k][4 * tx]);
            const floatx4 b1 = *reinterpret_cast<const floatx4 *>(&Bs[k][64 + 4 * tx]);
            const float av[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
            const float bv[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[i][j] = lp_step<PK>(acc[i][j], av[i], bv[j], p);
        }
        __syncthreads();
    }

    const bool vec_store = VEC && (m % 4 == 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int64_t row = row0 + 8 * ty + i;
        if (row >= n) continue;
        float *orow = out + (b * n + row) * m;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t col = col0 + 64 * h + 4 * tx;
            floatx4 v;
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = lp_finish<PK>(acc[i][4 * h + c], inv_p);
            if (vec_store && col + 3 < m) {
                store_nt4(orow + col, v);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (col + c < m) store_nt(orow + col + c, v[c]);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------------------
constexpr int kBRows = 128;  // rows (i) per block
constexpr int kBFeat = 64;   // features (k) per block
constexpr int kBJ = 32;      // j per stage

// Weight of pair (i, j) given upstream grad g and distance dist (torch's _cdist_backward):
// p = 1, inf: g itself; p = 2: g / dist; other p: g / dist^(p-1); 0 where dist == 0 (except
// p = 1 and inf, whose formulas have no division).
template <int PK>
__device__ __forceinline__ float pair_weight(float g, float dist, float p) {
    if constexpr (PK == kP1 || PK == kPInf) return g;
    else if constexpr (PK == kP2) return dist == 0.0f ? 0.0f : __fdiv_rn(g, dist);
    else if constexpr (PK == kP3) return dist == 0.0f ? 0.0f : __fdiv_rn(g, dist * dist);
    else return dist == 0.0f ? 0.0f : __fdiv_rn(g, powf(dist, p - 1.0f));
}

__device__ __forceinline__ float signf(float d) {
    return d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f);
}

template <int PK>
__device__ __forceinline__ float grad_term(float d, float w, float dist, float p) {
    if constexpr (PK == kP1) return signf(d) * w;
    else if constexpr (PK == kP2) return d * w;
    else if constexpr (PK == kP3) return d * fabsf(d) * w;
    else if constexpr (PK == kPInf) return fabsf(d) == dist ? signf(d) * w : 0.0f;
    else if constexpr (PK == kPLt2) {
        if (d == 0.0f && p < 1.0f) return 0.0f;
        return signf(d) * exp2f((p - 1.0f) * __log2f(fabsf(d))) * w;
    } else {
        return d * exp2f((p - 2.0f) * __log2f(fabsf(d))) * w;
    }
}

// out[(split, b, i, k)] = sum over this split's j of grad_term.  G(b,i,j) and Dist(b,i,j)
// are read at g[b*n*m + i*gs_i + j*gs_j] (gs = (m, 1) direct, (1, n) transposed).
template <int PK, bool TR>
__global__ __launch_bounds__(kThreads, 2) void lp_backward_kernel(
    const float *__restrict__ g, const float *__restrict__ dist, const float *__restrict__ x1,
    const float *__restrict__ x2, int64_t n, int64_t m, int64_t d, float p, int64_t j_per_split,
    int64_t batch, float *__restrict__ out) {
    __shared__ float Ws[kBJ][kBRows + kPad];
    __shared__ float Ds[PK == kPInf ? kBJ : 1][kBRows + kPad];
    __shared__ float Xs[kBJ][kBFeat + kPad];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int64_t split = blockIdx.z / batch, b = blockIdx.z - split * batch;
    const int64_t i0 = (int64_t)blockIdx.y * kBRows, k0 = (int64_t)blockIdx.x * kBFeat;
    const int64_t jbeg = split * j_per_split;
    const int64_t jend = jbeg + j_per_split < m ? jbeg + j_per_split : m;
    const float *G = g + b * n * m;
    const float *Dm = dist + b * n * m;
    const float *X1 = x1 + b * n * d;
    const float *X2 = x2 + b * m * d;

    float xv[8][4], acc[8][4];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const int64_t i = i0 + 8 * ty + r;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int64_t k = k0 + 4 * tx + c;
            xv[r][c] = (i < n && k < d) ? X1[i * d + k] : 0.0f;
            acc[r][c] = 0.0f;
        }
    }

    for (int64_t j0 = jbeg; j0 < jend; j0 += kBJ) {
        // weights: 128 i x 32 j
        if constexpr (!TR) {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int idx = tid + kThreads * q;
                const int ii = idx >> 5, jj = idx & 31;
                const int64_t i = i0 + ii, j = j0 + jj;
                float w = 0.0f, dd = 0.0f;
                if (i < n && j < jend) {
                    const float gv = G[i * m + j];
                    dd = Dm[i * m + j];
                    w = pair_weight<PK>(gv, dd, p);
                }
                Ws[jj][ii] = w;
                if constexpr (PK == kPInf) Ds[jj][ii] = dd;
            }
        } else {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int idx = tid + kThreads * q;
                const int jj = idx >> 7, ii = idx & 127;
                const int64_t i = i0 + ii, j = j0 + jj;
                float w = 0.0f, dd = 0.0f;
                if (i < n && j < jend) {
                    const float gv = G[j * n + i];
                    dd = Dm[j * n + i];
                    w = pair_weight<PK>(gv, dd, p);
                }
                Ws[jj][ii] = w;
                if constexpr (PK == kPInf) Ds[jj][ii] = dd;
            }
        }
        // x2 panel: 32 j x 64 k
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int idx = tid + kThreads * q;
            const int jj = idx >> 6, kk = idx & 63;
            const int64_t j = j0 + jj, k = k0 + kk;
            Xs[jj][kk] = (j < jend && k < d) ? X2[j * d + k] : 0.0f;
        }
        __syncthreads();
        const int jmax = jend - j0 < kBJ ? (int)(jend - j0) : kBJ;
        for (int jj = 0; jj < jmax; ++jj) {
            const floatx4 w0 = *reinterpret_cast<const floatx4 *>(&Ws[jj][8 * ty]);
            const floatx4 w1 = *reinterpret_cast<const floatx4 *>(&Ws[jj][8 * ty + 4]);
            const floatx4 x = *reinterpret_cast<const floatx4 *>(&Xs[jj][4 * tx]);
            const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
            float dv[8];
            if constexpr (PK == kPInf) {
                const floatx4 d0 = *reinterpret_cast<const floatx4 *>(&Ds[jj][8 * ty]);
                const floatx4 d1 = *reinterpret_cast<const floatx4 *>(&Ds[jj][8 * ty + 4]);
                dv[0] = d0[0]; dv[1] = d0[1]; dv[2] = d0[2]; dv[3] = d0[3];
                dv[4] = d1[0]; dv[5] = d1[1]; dv[6] = d1[2]; dv[7] = d1[3];
            } else {
#pragma unroll
                for (int r = 0; r < 8; ++r) dv[r] = 0.0f;
            }
#pragma unroll
            for (int r = 0; r < 8; ++r)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    acc[r][c] += grad_term<PK>(xv[r][c] - x[c], wv[r], dv[r], p);
        }
        __syncthreads();
    }

    float *o = out + (split * batch + b) * n * d;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const int64_t i = i0 + 8 * ty + r;
        if (i >= n) continue;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int64_t k = k0 + 4 * tx + c;
            if (k < d) o[i * d + k] = acc[r][c];
        }
    }
}

__global__ void sum_splits_kernel(const float *__restrict__ part, int64_t splits, int64_t len,
                                  float *__restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= len) return;
    float s = part[t];
    for (int64_t q = 1; q < splits; ++q) s += part[q * len + t];
    out[t] = s;
}

__global__ void fill_zero_kernel(float *__restrict__ p, int64_t len) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < len) p[t] = 0.0f;
}

int pkind_of(double p) {
    if (p == 0.0) return kP0;
    if (p == 1.0) return kP1;
    if (p == 2.0) return kP2;
    if (p == 3.0) return kP3;
    if (isinf(p)) return kPInf;
    if (p < 2.0) return kPLt2;
    return kPGen;
}

template <int PK>
int launch_forward(const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m,
                   int64_t d, double p, float *out, hipStream_t s) {
    const int64_t tiles_m = cdiv(m, kTile);
    dim3 grid((unsigned)tiles_m, (unsigned)cdiv(n, kTile), (unsigned)batch);
    const bool vec = (d % 4 == 0) && aligned16(x1) && aligned16(x2) && aligned16(out);
    const float pf = (float)p, inv_p = (float)(1.0 / p);
    if (vec)
        hipLaunchKernelGGL((lp_forward_kernel<PK, true>), grid, dim3(kThreads), 0, s, x1, x2, n, m,
                           d, pf, inv_p, out, tiles_m);
    else
        hipLaunchKernelGGL((lp_forward_kernel<PK, false>), grid, dim3(kThreads), 0, s, x1, x2, n,
                           m, d, pf, inv_p, out, tiles_m);
    return check_launch("lp_forward_kernel");
}

}  // namespace

// Number of j splits used by the backward for these sizes (1 = no partial buffer).
int64_t lp_backward_splits(int64_t batch, int64_t n, int64_t m, int64_t d) {
    const int64_t base = cdiv(n, kBRows) * cdiv(d, kBFeat) * batch;
    int64_t splits = cdiv(1024, base);
    const int64_t max_by_m = cdiv(m, 512);
    if (splits > max_by_m) splits = max_by_m;
    if (splits > 16) splits = 16;
    if (splits < 1) splits = 1;
    while (splits > 1 && splits * batch > kMaxGridYZ) --splits;
    return splits;
}

template <int PK, bool TR>
static int launch_backward(const float *g, const float *dist, const float *x1, const float *x2,
                           int64_t batch, int64_t n, int64_t m, int64_t d, double p,
                           float *grad, float *part, int64_t splits, hipStream_t s) {
    const int64_t jps = cdiv(cdiv(m, splits), kBJ) * kBJ;
    dim3 grid((unsigned)cdiv(d, kBFeat), (unsigned)cdiv(n, kBRows), (unsigned)(splits * batch));
    float *dst = splits > 1 ? part : grad;
    hipLaunchKernelGGL((lp_backward_kernel<PK, TR>), grid, dim3(kThreads), 0, s, g, dist, x1, x2,
                       n, m, d, (float)p, jps, batch, dst);
    int rc = check_launch("lp_backward_kernel");
    if (rc != TPW_OK || splits == 1) return rc;
    const int64_t len = batch * n * d;
    hipLaunchKernelGGL(sum_splits_kernel, dim3((unsigned)cdiv(len, 256)), dim3(256), 0, s, part,
                       splits, len, grad);
    return check_launch("sum_splits_kernel");
}

template <bool TR>
static int dispatch_backward(int pk, const float *g, const float *dist, const float *x1,
                             const float *x2, int64_t batch, int64_t n, int64_t m, int64_t d,
                             double p, float *grad, float *part, int64_t splits, hipStream_t s) {
    switch (pk) {
        case kP1: return launch_backward<kP1, TR>(g, dist, x1, x2, batch, n, m, d, p, grad, part, splits, s);
        case kP2: return launch_backward<kP2, TR>(g, dist, x1, x2, batch, n, m, d, p, grad, part, splits, s);
        case kP3: return launch_backward<kP3, TR>(g, dist, x1, x2, batch, n, m, d, p, grad, part, splits, s);
        case kPInf: return launch_backward<kPInf, TR>(g, dist, x1, x2, batch, n, m, d, p, grad, part, splits, s);
        case kPLt2: return launch_backward<kPLt2, TR>(g, dist, x1, x2, batch, n, m, d, p, grad, part, splits, s);
        default: return launch_backward<kPGen, TR>(g, dist, x1, x2, batch, n, m, d, p, grad, part, splits, s);
    }
}

}  // namespace tpw

using namespace tpw;

extern "C" int tpw_lp_distances(const float *x1, const float *x2, int64_t batch, int64_t n,
                                int64_t m, int64_t d, double p, float *out, void *stream) {
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    TPW_REQUIRE(p >= 0.0, "p must be non-negative, got %g", p);
    TPW_REQUIRE(cdiv(n, kTile) <= kMaxGridYZ && batch <= kMaxGridYZ, "too many rows or batches");
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    hipStream_t s = as_stream(stream);
    switch (pkind_of(p)) {
        case kP0: return launch_forward<kP0>(x1, x2, batch, n, m, d, p, out, s);
        case kP1: return launch_forward<kP1>(x1, x2, batch, n, m, d, p, out, s);
        case kP2: return launch_forward<kP2>(x1, x2, batch, n, m, d, p, out, s);
        case kP3: return launch_forward<kP3>(x1, x2, batch, n, m, d, p, out, s);
        case kPInf: return launch_forward<kPInf>(x1, x2, batch, n, m, d, p, out, s);
        case kPLt2: return launch_forward<kPLt2>(x1, x2, batch, n, m, d, p, out, s);
        default: return launch_forward<kPGen>(x1, x2, batch, n, m, d, p, out, s);
    }
}

extern "C" size_t tpw_lp_backward_workspace_size(int64_t batch, int64_t n, int64_t m, int64_t d) {
    const int64_t splits = lp_backward_splits(batch, n, m, d);
    return splits > 1 ? (size_t)(splits * batch * n * d) * sizeof(float) : 0;
}

extern "C" int tpw_lp_distances_backward(const float *grad, const float *x1, const float *x2,
                                         const float *dist, int64_t batch, int64_t n, int64_t m,
                                         int64_t d, double p, int transposed, float *grad_x1,
                                         void *workspace, void *stream) {
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    TPW_REQUIRE(p >= 0.0, "p must be non-negative, got %g", p);
    TPW_REQUIRE(cdiv(n, kBRows) <= kMaxGridYZ, "too many rows");
    if (batch == 0 || n == 0 || d == 0) return TPW_OK;
    TPW_REQUIRE(grad_x1, "null pointer");
    hipStream_t s = as_stream(stream);
    const int64_t len = batch * n * d;
    if (p == 0.0 || m == 0) {  // zero gradient, as _cdist_backward returns for p == 0
        hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)cdiv(len, 256)), dim3(256), 0, s,
                           grad_x1, len);
        return check_launch("fill_zero_kernel");
    }
    TPW_REQUIRE(grad && x1 && x2 && dist, "null pointer");
    const int64_t splits = lp_backward_splits(batch, n, m, d);
    TPW_REQUIRE(splits == 1 || workspace, "workspace of %zu bytes required",
                tpw_lp_backward_workspace_size(batch, n, m, d));
    float *part = static_cast<float *>(workspace);
    const int pk = pkind_of(p);
    if (transposed)
        return dispatch_backward<true>(pk, grad, dist, x1, x2, batch, n, m, d, p, grad_x1, part, splits, s);
    return dispatch_backward<false>(pk, grad, dist, x1, x2, batch, n, m, d, p, grad_x1, part, splits, s);
}
