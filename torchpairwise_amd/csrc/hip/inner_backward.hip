// Backward of the inner-product family (euclidean via _euclidean_dist, cosine distance and
// cosine similarity, and the polynomial / sigmoid kernel functions), fp32 and bf16.
//
// Both gradients have the shape  grad_x1 = sign * (W @ x2) + coef1[i] * x1[i],
//                                grad_x2 = sign * (W^T @ x1) + coef2[j] * x2[j],
// with a per-pair weight matrix W [n, m] and per-row coefficients:
//   euclidean (derivatives.yaml _euclidean_dist_backward):
//     W = grad / res (0 where res == 0), sign = -1, coef1 = sum_j W, coef2 = sum_i W;
//   cosine (autograd graph of csrc/ops/pairwise_metrics.cpp:51-56,112-122):
//     q = prf_div(S, n1 n2^T, identity), gq = -grad [0 <= 1 - q <= 2] (clip mask; for
//     cosine_similarity gq = grad), gS = prf_div backward (gq / den, or gq where den == 0),
//     gden = gS * -S / den (0 where den == 0), W = gS, sign = +1,
//     coef1 = sum_j gden n2[j] / n1[i], coef2 = sum_i gden n1[i] / n2[j] (0 where the norm
//     is 0, as torch's norm backward);
//   polynomial (pairwise_metrics.cpp:67-78, (S gamma + coef0)^degree):
//     W = grad * degree * (S gamma + coef0)^(degree - 1) * gamma (S recomputed), sign = +1,
//     no coefficients;
//   sigmoid (pairwise_metrics.cpp:80-90, tanh(S gamma + coef0)): W = grad * (1 - out^2) *
//     gamma from the output.
//
// Pass 1 (VALU, memory-bound) forms W in the workspace and writes per-tile partial row and
// column sums; pass 2 adds the partials in a fixed order (deterministic); pass 3 runs the
// two products on the matrix cores with the sign/coef epilogue fused.  For cosine, S is
// first recomputed on the MFMA path.
//   fp32: W in fp32; both products on the forward's tile kernel (v_mfma_f32_32x32x2_f32),
//         which reads x2 (for grad_x1) and W, x1 (for grad_x2) k-major in place
//         (grad_product_f32); other shapes take bwd_gemm_kernel, operands staged k-major
//         in LDS, split over K when the output tiles alone would not fill the GPU.  For the
//         modes whose row terms are the weights (or zero), passes 1-2 and the grad_x1
//         product are one kernel (fused_grad1_kernel) and grad_x2 sums W's columns from its
//         own operand.
//   bf16: W rounded to bf16 (the precision of the reference's bf16 autograd); both products on
//         the tile kernel (v_mfma_f32_32x32x16_bf16), which reads x2 (for grad_x1) and W, x1 (for
//         grad_x2) k-major through transposing LDS reads (grad_product_bf16); other shapes
//         write W^T and transposed x1, x2 so that both products are A . B^T with k-contiguous
//         rows (inner_grad_gemm).
#include "common.hpp"
#include "tile_mfma.hpp"

namespace tpw {
namespace {

enum Mode {
    kEuclid = 0, kCosDist = 1, kCosSim = 2, kSqEuclid = 3, kPoly = 4, kSigmoid = 5, kCosCorr = 6, kDot = 7,
    // the cosine modes with the weights formed from the forward's output instead of a recomputed S
    kCosDistO = 8, kCosSimO = 9, kCosCorrO = 10
};
// S-based cosine modes, output-based ones, and either
template <int MODE> constexpr bool kCosS = MODE == kCosDist || MODE == kCosSim || MODE == kCosCorr;
template <int MODE> constexpr bool kCosO = MODE == kCosDistO || MODE == kCosSimO || MODE == kCosCorrO;
template <int MODE> constexpr bool kCosAny = kCosS<MODE> || kCosO<MODE>;

// x^k for an integral k as ATen's pow with a scalar exponent computes it on the GPU.
__device__ __forceinline__ float ipow(float x, int k) {
#pragma clang fp contract(off)
    if (k == 2) return x * x;
    if (k == 3) return x * x * x;
    if (k == 1) return x;
    if (k == 0) return 1.0f;
    return powf(x, (float)k);
}

constexpr int kPWRows = 128;
constexpr int kPWCols = 256;

// One pair's stored weight w (for BF16W the euclidean / sqeuclidean weight is already rounded
// to bf16, as the reference's bf16 autograd rounds its ratio tensor), its row-sum term rt and
// column-sum term ct, from the upstream grad gv, av (res for euclid / sigmoid, S for the
// polynomial and the S-based cosine modes, the forward's output o for the output-based ones),
// and for cosine the row and column norms nv, a2.  Quotients by res and by the norm product
// use fast_div (the reciprocal, within 2 ulp of the reference's divide).
template <int MODE, bool BF16W>
__device__ __forceinline__ void weight_terms(float gv, float av, float nv, float a2, const KerParams &kp, float &w,
                                             float &rt, float &ct) {
#pragma clang fp contract(off)
    rt = 0.0f;
    ct = 0.0f;
    if constexpr (MODE == kEuclid) {
        w = av == 0.0f ? 0.0f : fast_div(gv, av);
        if constexpr (BF16W) w = bf16_to_f32(f32_to_bf16_rne(w));
        rt = w;
        ct = w;
    } else if constexpr (MODE == kSqEuclid) {
        w = 2.0f * gv;
        if constexpr (BF16W) w = bf16_to_f32(f32_to_bf16_rne(w));
        rt = w;
        ct = w;
    } else if constexpr (MODE == kPoly) {
        // autograd of matmul(...).mul_(gamma).add_(coef0).pow_(degree): pow's
        // backward grad * (degree * base^(degree - 1)) (zero for degree 0), then * gamma
        const float base = av * kp.gamma + kp.coef0;
        const float fd = kp.degree == 0 ? 0.0f : (float)kp.degree * ipow(base, kp.degree - 1);
        w = (gv * fd) * kp.gamma;
    } else if constexpr (MODE == kSigmoid) {
        // tanh's backward from its output t: grad * (1 - t * t), then * gamma
        w = (gv * (1.0f - av * av)) * kp.gamma;
    } else if constexpr (MODE == kDot) {
        w = gv;  // matmul's backward: the products with grad itself
    } else if constexpr (kCosO<MODE>) {
        // q = S / den from the output o: o itself (similarity), 1 - o (distance, correlation).
        // The distance's clip passes the gradient where 0 <= 1 - q <= 2; from o alone the
        // bounds o = 0 and o = 2 cannot tell an exact 1 - q = 0 (or 2) from a clipped one, and
        // both count as clipped.  (An unclipped q of exactly +-1 belongs to a pair whose
        // gradient terms cancel to rounding level: gS (x2 - q (n2 / n1) x1) for parallel rows.)
        const float a1 = nv, den = a1 * a2;
        const float q = MODE == kCosSimO ? av : 1.0f - av;
        float gq = MODE == kCosSimO ? gv : -gv;
        if constexpr (MODE == kCosDistO) gq = (av > 0.0f && av < 2.0f) ? gq : 0.0f;
        const float gS = den != 0.0f ? fast_div(gq, den) : gq;
        // gden = gS * -S / den = -gS q (0 where den == 0, as prf_div's backward)
        const float gden = den != 0.0f ? -(gS * q) : 0.0f;
        w = gS;
        rt = gden * a2;
        ct = gden * a1;
    } else {
        const float sv = av, a1 = nv;
        const float den = a1 * a2;
        const float q = den != 0.0f ? __fdiv_rn(sv, den) : sv;
        float gq = gv;
        if constexpr (MODE == kCosDist) {
            const float v = 1.0f - q;
            gq = (v >= 0.0f && v <= 2.0f) ? -gv : 0.0f;
        } else if constexpr (MODE == kCosCorr) {
            gq = -gv;  // neg_ then add_(1): no clamp
        }
        const float gS = den != 0.0f ? fast_div(gq, den) : gq;
        const float gden = den != 0.0f ? fast_div(gS * -sv, den) : 0.0f;
        w = gS;
        rt = gden * a2;
        ct = gden * a1;
    }
}

// The output-based cosine terms for a pair whose norms both lie in [2^-60, 2^60] (so den = n1 n2
// is a normal nonzero float and weight_terms takes its quotient branch), from the reciprocals
// r1 = RN(1 / n1), r2 = RN(1 / n2): gS = gq r1 r2, rt = gden n2 = -gq q r1, ct = gden n1 =
// -gq q r2.  Within 2 ulp of weight_terms's values (which divide by the rounded n1 n2), with
// seven VALU operations against its twenty and a reciprocal.
template <int MODE>
__device__ __forceinline__ void cos_terms_fast(float gv, float av, float r1, float r2, float &w, float &rt,
                                               float &ct) {
#pragma clang fp contract(off)
    const float q = MODE == kCosSimO ? av : 1.0f - av;
    float gq = MODE == kCosSimO ? gv : -gv;
    if constexpr (MODE == kCosDistO) gq = (av > 0.0f && av < 2.0f) ? gq : 0.0f;
    const float t = gq * q;
    w = gq * (r1 * r2);
    rt = -(t * r1);
    ct = -(t * r2);
}

// Norms in [2^-60, 2^60] (NaN excluded): the pairs of two such rows take cos_terms_fast.
__device__ __forceinline__ bool cos_norm_fast(float v) { return v >= 0x1p-60f && v <= 0x1p60f; }

// rn2[t] = RN(1 / n2[t]); *slow |= 1 when one of the len1 + len2 norms n1, n2 lies outside
// [2^-60, 2^60] (*slow preset to 0; one atomic per wave that finds one).
__global__ void cos_norm_prep_kernel(const float *__restrict__ n1, int64_t len1, const float *__restrict__ n2,
                                     int64_t len2, float *__restrict__ rn2, uint32_t *__restrict__ slow) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool in = t < len1 + len2;
    const float v = !in ? 1.0f : t < len1 ? n1[t] : n2[t - len1];
    if (in && t >= len1) rn2[t - len1] = __fdiv_rn(1.0f, v);
    if (__ballot(!cos_norm_fast(v)) != 0ull && (threadIdx.x & 63) == 0) atomicOr(slow, 1u);
}

// bf16 cosine: grad_x2[j] = P[j] + coef2[j] x2[j], with P = W^T x1 as the product wrote it (bf16,
// in gx2) and coef2[j] = sum_i gden[i][j] n1[i] / n2[j].  Since gden = -gS q and q n1 / n2 =
// S / n2^2, coef2[j] = -(x2[j] . sum_i gS[i][j] x1[i]) / n2[j]^2 = -(x2[j] . P[j]) / n2[j]^2
// (0 where n2[j] = 0): one wave per row, the dot product in fp32, d % 8 == 0.
__global__ __launch_bounds__(256) void cos_proj_finish_kernel(uint16_t *__restrict__ gx2,
                                                              const uint16_t *__restrict__ x2,
                                                              const float *__restrict__ n2, int64_t rows, int64_t d) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;  // the same in every lane
    uint16_t *P = gx2 + row * d;
    const uint16_t *X = x2 + row * d;
    float dot = 0.0f;
    for (int64_t k = 8 * lane; k < d; k += 512) {
        const uint4 pv = *reinterpret_cast<const uint4 *>(P + k), xv = *reinterpret_cast<const uint4 *>(X + k);
        const uint32_t pw[4] = {pv.x, pv.y, pv.z, pv.w}, xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            dot += __uint_as_float(pw[e] << 16) * __uint_as_float(xw[e] << 16);
            dot += __uint_as_float(pw[e] & 0xffff0000u) * __uint_as_float(xw[e] & 0xffff0000u);
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) dot += __shfl_xor(dot, off, 64);
    const float nv = n2[row];
    const float coef = nv == 0.0f ? 0.0f : -__fdiv_rn(__fdiv_rn(dot, nv), nv);
    for (int64_t k = 8 * lane; k < d; k += 512) {
        const uint4 pv = *reinterpret_cast<const uint4 *>(P + k), xv = *reinterpret_cast<const uint4 *>(X + k);
        const uint32_t pw[4] = {pv.x, pv.y, pv.z, pv.w}, xw[4] = {xv.x, xv.y, xv.z, xv.w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = f32x2_to_bf16x2_rne(__uint_as_float(pw[e] << 16) + coef * __uint_as_float(xw[e] << 16),
                                       __uint_as_float(pw[e] & 0xffff0000u) +
                                           coef * __uint_as_float(xw[e] & 0xffff0000u));
        *reinterpret_cast<uint4 *>(P + k) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// Pass 1.  W (type T: fp32, or bf16 rounded as the reference's bf16 autograd rounds its
// ratio tensor) is written [n, m] to Wo and, when WTo is given, transposed [m, n] to WTo,
// so that both gradient products read their operands k-contiguous.  The row / column sums
// are taken of the stored values.  For cosine, S is read from the fp32 buffer S.
template <typename T, int MODE>
__global__ __launch_bounds__(256) void pair_weights_kernel(
    const T *__restrict__ g, const T *__restrict__ res, const float *__restrict__ n1,
    const float *__restrict__ n2, int64_t n, int64_t m, const float *__restrict__ S,
    float *__restrict__ rowpart, float *__restrict__ colpart, int64_t tiles_i, int64_t tiles_j,
    T *__restrict__ Wo, T *__restrict__ WTo, KerParams kp) {
#pragma clang fp contract(off)
    constexpr bool BF16W = sizeof(T) == 2;
    constexpr int kGrp = BF16W ? 8 : 4;  // rows per 16-byte transposed store
    __shared__ float red[4][kPWRows];
    // bf16 W^T through LDS: 64 rows x 256 columns as [column][8 x 16 bytes] (144-byte stride),
    // written out as row segments; needs 16-byte aligned W^T rows (n % 8 == 0)
    __shared__ uint4 tr[BF16W ? kPWCols * 9 : 1];
    const bool lds_t = BF16W && (n % 8) == 0;
    const int64_t b = blockIdx.z, ti = blockIdx.y, tj = blockIdx.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t j = tj * kPWCols + tid;
    const bool jok = j < m;
    float a2 = 0.0f;
    if constexpr (kCosAny<MODE>) a2 = jok ? n2[b * m + j] : 0.0f;
    float csum = 0.0f;
    // One element from its loaded operands (gv = grad; av = res for euclid / sigmoid, S for
    // polynomial / cosine; nv = n1[i] for cosine): the stored weight (wf, or its bf16 bits wb)
    // and the row-sum term rt.
    constexpr bool kRes = MODE == kEuclid || MODE == kSigmoid || kCosO<MODE>;
    constexpr bool kS = MODE == kPoly || kCosS<MODE>;
    constexpr bool kCos = kCosAny<MODE>;
    auto element = [&](bool ok, int64_t idx, float gv, float av, float nv, float &wf, uint16_t &wb, float &rt) {
        wf = 0.0f;
        wb = 0;
        rt = 0.0f;
        if (!ok) return;
        float w, ct;
        weight_terms<MODE, BF16W>(gv, av, nv, a2, kp, w, rt, ct);
        if constexpr (MODE == kEuclid || MODE == kSqEuclid || kCos) csum += ct;
        if constexpr (BF16W) {
            wb = f32_to_bf16_rne(w);
            Wo[idx] = wb;
        } else {
            Wo[idx] = w;
            wf = w;
        }
    };
    // Rows in groups of 8.  The group's 8 row sums over this wave's 64 columns take a
    // transposing butterfly: xor 32, 16, 8 each hand half of the remaining values to the
    // partner (4 + 2 + 1 shuffles), leaving lane l with a partial of group row
    // (l >> 3) & 7 (bits 5, 4, 3 of l), which xor 4, 2, 1 complete: 10 shuffles per 8 rows
    // instead of 6 per row.
    const int grow = ((lane >> 5) & 1) * 4 + ((lane >> 4) & 1) * 2 + ((lane >> 3) & 1);
    for (int r0 = 0; r0 < kPWRows; r0 += 8) {
        float wf[8], rt[8];
        uint16_t wb[8];
        // the group's loads first (an invalid element reads element 0 of the batch, which
        // exists whenever the grid does, and is then dropped), so their latencies overlap
        float gv[8], av[8], nv[8];
        bool ok[8];
        int64_t idx[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t i = ti * kPWRows + r0 + u;
            ok[u] = i < n && jok;
            idx[u] = ok[u] ? (b * n + i) * m + j : b * n * m;
            gv[u] = to_f32(g[idx[u]]);
            av[u] = 0.0f;
            nv[u] = 0.0f;
            if constexpr (kRes) av[u] = to_f32(res[idx[u]]);
            if constexpr (kS) av[u] = S[idx[u]];
            if constexpr (kCos) nv[u] = n1[b * n + (ok[u] ? i : 0)];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) element(ok[u], idx[u], gv[u], av[u], nv[u], wf[u], wb[u], rt[u]);
        if (WTo && lds_t) {
            // bf16 rows r0 .. r0 + 7 of column j -> the LDS transpose tile (written out below)
            uint4 pk;
            pk.x = (uint32_t)wb[0] | ((uint32_t)wb[1] << 16);
            pk.y = (uint32_t)wb[2] | ((uint32_t)wb[3] << 16);
            pk.z = (uint32_t)wb[4] | ((uint32_t)wb[5] << 16);
            pk.w = (uint32_t)wb[6] | ((uint32_t)wb[7] << 16);
            tr[tid * 9 + ((r0 & 63) >> 3)] = pk;
        } else if (WTo) {  // rows r0 .. r0 + 7 of column j: 16 bytes (bf16) or 2 x 16 bytes of WTo row j
            const int64_t i0 = ti * kPWRows + r0;
            if (jok && i0 < n) {
                T *dst = WTo + (b * m + j) * n + i0;
#pragma unroll
                for (int hlf = 0; hlf < 8 / kGrp; ++hlf) {
                    const int e0 = hlf * kGrp;
                    uint32_t pk[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if constexpr (BF16W) pk[e] = (uint32_t)wb[2 * e] | ((uint32_t)wb[2 * e + 1] << 16);
                        else pk[e] = __float_as_uint(wf[e0 + e]);
                    }
                    if (i0 + e0 + kGrp <= n && (n % kGrp) == 0) {
                        *reinterpret_cast<uint4 *>(dst + e0) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
                    } else {
                        for (int e = 0; e < kGrp && i0 + e0 + e < n; ++e) {
                            if constexpr (BF16W) dst[e0 + e] = wb[e0 + e];
                            else dst[e0 + e] = wf[e0 + e];
                        }
                    }
                }
            }
        }
        float v4[4], v2[2];
        const bool hi32 = (lane & 32) != 0, hi16 = (lane & 16) != 0, hi8 = (lane & 8) != 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float mine = hi32 ? rt[4 + k] : rt[k], other = hi32 ? rt[k] : rt[4 + k];
            v4[k] = mine + __shfl_xor(other, 32, 64);
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const float mine = hi16 ? v4[2 + k] : v4[k], other = hi16 ? v4[k] : v4[2 + k];
            v2[k] = mine + __shfl_xor(other, 16, 64);
        }
        float v1;
        {
            const float mine = hi8 ? v2[1] : v2[0], other = hi8 ? v2[0] : v2[1];
            v1 = mine + __shfl_xor(other, 8, 64);
        }
        v1 += __shfl_xor(v1, 4, 64);
        v1 += __shfl_xor(v1, 2, 64);
        v1 += __shfl_xor(v1, 1, 64);
        if ((lane & 7) == 0) red[wave][r0 + grow] = v1;
        if (WTo && lds_t && (r0 & 63) == 56) {
            // the 64-row half is complete: write W^T rows j0 .. j0 + 255, 128 contiguous bytes
            // (rows i0 .. i0 + 63) each, 8 lanes per row segment
            __syncthreads();
            const int64_t i0 = ti * kPWRows + (r0 & ~63);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int idx = tid + 256 * q, col = idx >> 3, c = idx & 7;
                const int64_t jj = tj * kPWCols + col, ii = i0 + 8 * c;
                if (jj < m && ii < n) {
                    T *dst = WTo + (b * m + jj) * n + ii;
                    const uint4 v = tr[col * 9 + c];
                    if (ii + 8 <= n) {
                        *reinterpret_cast<uint4 *>(dst) = v;
                    } else {
                        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
                        for (int e = 0; ii + e < n; ++e) dst[e] = (uint16_t)(w4[e >> 1] >> (16 * (e & 1)));
                    }
                }
            }
            __syncthreads();
        }
    }
    __syncthreads();
    if (tid < kPWRows) {
        const int64_t i = ti * kPWRows + tid;
        if (i < n)
            rowpart[(b * tiles_j + tj) * n + i] = red[0][tid] + red[1][tid] + red[2][tid] + red[3][tid];
    }
    if (jok) colpart[(b * tiles_i + ti) * m + j] = csum;
}

// Pass 1 for fp32 weights without a transposed copy, with 16-byte accesses: the 128 x 256
// tile of pair_weights_kernel, wave w on rows 32 w .. 32 w + 31, lane l on columns 4 l .. 4 l + 3
// (m % 4 == 0 and 16-byte aligned arrays, so a lane's 4 columns are all inside or all
// outside), rows in groups of 4 with the group's loads issued first.  The group's 4 row sums
// take a transposing butterfly (xor 32 and 16 hand half of the values to the partner, xor 8,
// 4, 2, 1 complete them): lane l then holds row 2 ((l >> 5) & 1) + ((l >> 4) & 1) of the
// group.  Column sums meet in LDS.  Same weights (weight_terms) and partials layout as
// pair_weights_kernel.
template <int MODE>
__global__ __launch_bounds__(256) void pair_weights_vec_kernel(
    const float *__restrict__ g, const float *__restrict__ res, const float *__restrict__ n1,
    const float *__restrict__ n2, int64_t n, int64_t m, const float *__restrict__ S,
    float *__restrict__ rowpart, float *__restrict__ colpart, int64_t tiles_i, int64_t tiles_j,
    float *__restrict__ Wo, KerParams kp) {
#pragma clang fp contract(off)
    constexpr bool kRes = MODE == kEuclid || MODE == kSigmoid || kCosO<MODE>;
    constexpr bool kS = MODE == kPoly || kCosS<MODE>;
    constexpr bool kCos = kCosAny<MODE>;
    __shared__ floatx4 red[4][64];
    const int64_t b = blockIdx.z, ti = blockIdx.y, tj = blockIdx.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t j0 = tj * kPWCols + 4 * lane;
    const bool jok = j0 < m;
    floatx4 a2 = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (kCos)
        if (jok) a2 = *reinterpret_cast<const floatx4 *>(n2 + b * m + j0);
    floatx4 csum = {0.0f, 0.0f, 0.0f, 0.0f};
    const float *Av = kRes ? res : S;
    const int grow = ((lane >> 5) & 1) * 2 + ((lane >> 4) & 1);
    const int64_t wrow0 = ti * kPWRows + wave * 32;
    for (int r0 = 0; r0 < 32; r0 += 4) {
        floatx4 gv[4], av[4];
        float nv[4];
        bool ok[4];
        int64_t idx[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t i = wrow0 + r0 + u;
            ok[u] = i < n && jok;
            idx[u] = ok[u] ? (b * n + i) * m + j0 : b * n * m;  // element 0 of the batch when invalid
            gv[u] = *reinterpret_cast<const floatx4 *>(g + idx[u]);
            av[u] = (kRes || kS) ? *reinterpret_cast<const floatx4 *>(Av + idx[u]) : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            nv[u] = kCos ? n1[b * n + (ok[u] ? i : 0)] : 0.0f;
        }
        float rs[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            floatx4 wv = {0.0f, 0.0f, 0.0f, 0.0f};
            float r = 0.0f;
            if (ok[u]) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float w, rt, ct;
                    weight_terms<MODE, false>(gv[u][c], av[u][c], nv[u], a2[c], kp, w, rt, ct);
                    wv[c] = w;
                    r += rt;
                    csum[c] += ct;
                }
                *reinterpret_cast<floatx4 *>(Wo + idx[u]) = wv;
            }
            rs[u] = r;
        }
        const bool hi32 = (lane & 32) != 0, hi16 = (lane & 16) != 0;
        float v2[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const float mine = hi32 ? rs[2 + k] : rs[k], other = hi32 ? rs[k] : rs[2 + k];
            v2[k] = mine + __shfl_xor(other, 32, 64);
        }
        float v1;
        {
            const float mine = hi16 ? v2[1] : v2[0], other = hi16 ? v2[0] : v2[1];
            v1 = mine + __shfl_xor(other, 16, 64);
        }
        v1 += __shfl_xor(v1, 8, 64);
        v1 += __shfl_xor(v1, 4, 64);
        v1 += __shfl_xor(v1, 2, 64);
        v1 += __shfl_xor(v1, 1, 64);
        const int64_t i = wrow0 + r0 + grow;
        if ((lane & 15) == 0 && i < n) rowpart[(b * tiles_j + tj) * n + i] = v1;
    }
    // column partials (zero for the kernel functions, whose W carries the whole gradient)
    red[wave][lane] = csum;
    __syncthreads();
    if (tid < 64) {
        const int64_t j = tj * kPWCols + 4 * tid;
        floatx4 t = red[0][tid];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            const floatx4 o = red[w][tid];
            t[0] += o[0];
            t[1] += o[1];
            t[2] += o[2];
            t[3] += o[3];
        }
        if (j < m) *reinterpret_cast<floatx4 *>(colpart + (b * tiles_i + ti) * m + j) = t;
    }
}

// coef[b][r] = sum_t part[b][t][r] (t in order), divided by norms[b][r] when given
// (0 where that norm is 0).
__global__ void reduce_parts_kernel(const float *__restrict__ part, int64_t tiles, int64_t rows,
                                    int64_t batch, const float *__restrict__ norms,
                                    float *__restrict__ coef) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= batch * rows) return;
    const int64_t b = t / rows, r = t - b * rows;
    const float *p = part + b * tiles * rows + r;
    float s = 0.0f;
    for (int64_t q = 0; q < tiles; ++q) s += p[q * rows];
    if (norms) {
        const float nv = norms[t];
        s = nv == 0.0f ? 0.0f : __fdiv_rn(s, nv);
    }
    coef[t] = s;
}

constexpr int kGT = 128;     // output tile rows and cols
constexpr int kGK = 32;      // k per chunk
constexpr int kGStride = kGT + 32;  // LDS row stride (floats): lanes 0-31 / 32-63 on disjoint banks

template <typename T>
__device__ __forceinline__ floatx4 load4(const T *p);
template <>
__device__ __forceinline__ floatx4 load4<float>(const float *p) {
    return *reinterpret_cast<const floatx4 *>(p);
}
template <>
__device__ __forceinline__ floatx4 load4<uint16_t>(const uint16_t *p) {
    const uint2 v = *reinterpret_cast<const uint2 *>(p);
    floatx4 r = {__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                 __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u)};
    return r;
}

// out = sign * (A @ B) + coef[row] * X[row]  (or raw partial sums when part != nullptr).
// A is fp32 [M][K] (A_T: stored [K][M]); B and X are T [K][N] / [M][N]; batch strides are
// M*K, K*N and M*N.  grid = (tiles_N, tiles_M, batch * splits).
template <typename T, bool A_T, bool VEC>
__global__ __launch_bounds__(256, 2) void bwd_gemm_kernel(
    const float *__restrict__ A, const T *__restrict__ B, int64_t M, int64_t N, int64_t K,
    int64_t k_per_split, int64_t batch, float sign, const float *__restrict__ coef,
    const T *__restrict__ X, T *__restrict__ out, float *__restrict__ part) {
    constexpr int kAStride = A_T ? kGStride : kGStride + 2;
    __shared__ float As[kGK * kAStride];
    __shared__ float Bs[kGK * kGStride];
    const int64_t split = blockIdx.z / batch, b = blockIdx.z - split * batch;
    const int64_t row0 = (int64_t)blockIdx.y * kGT, col0 = (int64_t)blockIdx.x * kGT;
    const int64_t kbeg = split * k_per_split;
    const int64_t kend = kbeg + k_per_split < K ? kbeg + k_per_split : K;
    const float *Ab = A + b * M * K;
    const T *Bb = B + b * K * N;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
    const int l32 = lane & 31, h = lane >> 5;

    floatx16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.0f;

    // Staging is software-pipelined: chunk k0 + kGK is loaded into registers while chunk k0
    // is multiplied from LDS.  A chunk: 128 rows x 32 k -> As[k][row]; B chunk: 32 k x 128
    // cols -> Bs[k][col].  Global reads are 16 bytes along the stored rows.  Direct A is
    // transposed on its way to LDS: 8 lanes per row, 8 rows per 64 lanes, one float store per
    // k; its row stride kGStride + 2 (4 * 162 = 8 mod 64) puts the 64 lanes of such a store
    // on 64 distinct banks (with 160 they would share 8).
    floatx4 va[4], vb[4];
    auto load = [&](int64_t k0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int idx = tid + 256 * q;
            floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (!A_T) {
                const int r = idx >> 3, c4 = idx & 7;
                const int64_t gr = row0 + r, gk = k0 + 4 * c4;
                if (gr < M) {
                    const float *src = Ab + gr * K + gk;
                    if (VEC && gk + 3 < kend) {
                        v = *reinterpret_cast<const floatx4 *>(src);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (gk + e < kend) v[e] = src[e];
                    }
                }
            } else {
                const int kk = idx >> 5, r4 = idx & 31;
                const int64_t gk = k0 + kk, gr = row0 + 4 * r4;
                if (gk < kend) {
                    const float *src = Ab + gk * M + gr;
                    if (VEC && gr + 3 < M) {
                        v = *reinterpret_cast<const floatx4 *>(src);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (gr + e < M) v[e] = src[e];
                    }
                }
            }
            va[q] = v;
        }
        // B chunk: 32 k x 128 cols -> Bs[k][col]
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int idx = tid + 256 * q;
            const int kk = idx >> 5, c4 = idx & 31;
            const int64_t gk = k0 + kk, gc = col0 + 4 * c4;
            floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
            if (gk < kend) {
                const T *src = Bb + gk * N + gc;
                if (VEC && gc + 3 < N) {
                    v = load4<T>(src);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (gc + e < N) v[e] = to_f32(src[e]);
                }
            }
            vb[q] = v;
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int idx = tid + 256 * q;
            if constexpr (!A_T) {
                const int r = idx >> 3, c4 = idx & 7;
#pragma unroll
                for (int e = 0; e < 4; ++e) As[(4 * c4 + e) * kAStride + r] = va[q][e];
            } else {
                const int kk = idx >> 5, r4 = idx & 31;
                *reinterpret_cast<floatx4 *>(&As[kk * kAStride + 4 * r4]) = va[q];
            }
            const int kk = idx >> 5, c4 = idx & 31;
            *reinterpret_cast<floatx4 *>(&Bs[kk * kGStride + 4 * c4]) = vb[q];
        }
    };

    if (kbeg < kend) load(kbeg);
    for (int64_t k0 = kbeg; k0 < kend; k0 += kGK) {
        store();
        __syncthreads();
        if (k0 + kGK < kend) load(k0 + kGK);
#pragma unroll
        for (int s = 0; s < kGK / 2; ++s) {
            const int kk = 2 * s + h;
            float a[2], bv[2];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) a[mi] = As[kk * kAStride + wr + mi * 32 + l32];
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) bv[ni] = Bs[kk * kGStride + wc + ni * 32 + l32];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[mi], bv[ni], acc[mi][ni], 0, 0, 0);
        }
        __syncthreads();
    }

#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
        const int64_t col = col0 + wc + ni * 32 + l32;
        if (col >= N) continue;
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = row0 + wr + mi * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row >= M) continue;
                if (part) {
                    part[((split * batch + b) * M + row) * N + col] = acc[mi][ni][r];
                } else {
                    const int64_t o = (b * M + row) * N + col;
                    from_f32(out + o, sign * acc[mi][ni][r] + coef[b * M + row] * to_f32(X[o]));
                }
            }
        }
    }
}

template <typename T>
__global__ void gemm_finish_kernel(const float *__restrict__ part, int64_t splits, int64_t len,
                                   int64_t M, int64_t N, float sign, const float *__restrict__ coef,
                                   const T *__restrict__ X, T *__restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= len) return;
    float s = part[t];
    for (int64_t q = 1; q < splits; ++q) s += part[q * len + t];
    const int64_t row = t / N;  // (b * M + row) flattened
    from_f32(out + t, sign * s + coef[row] * to_f32(X[t]));
}

// Blocks of the fp32 product kernel resident at once on the current device (CUs x blocks
// per CU; every variant of the kernel has the same register and LDS footprint), cached per
// device.  Without a device (a size query on a host without one) 256 CUs x 3.
int64_t gemm_slots() {
    static int cache[16];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256 * 3;
    int &c = cache[dev & 15];
    if (c == 0) {
        int per_cu = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, bwd_gemm_kernel<float, false, true>, 256, 0) !=
                hipSuccess || per_cu <= 0)
            per_cu = 3;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        c = per_cu * cus;
    }
    return c;
}

// Compute units of the current device (256 when the query fails).
int64_t device_cus() {
    static int cache[16];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
    int &c = cache[dev & 15];
    if (c == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        c = cus;
    }
    return c;
}

// The tile-kernel gradient products have one block per 128 x 128 output tile and no split of K,
// so they run only where that grid gives every CU two blocks; smaller outputs (16384 x 128 from
// K = 16384: 128 tiles) take the split-K GEMM, whose splits fill the GPU.
bool tile_grid_fills(int64_t batch, int64_t M, int64_t N) {
    return cdiv(M, tile::kT) * cdiv(N, tile::kT) * batch >= 2 * device_cus();
}

// Number of K splits: the smallest whose blocks fill the resident rounds to at least 90 %
// (the output tiles alone are often a round and a third: C2's 1024 tiles on 768 slots run two
// rounds for 1.33 rounds of work), else the best fill, with at least 256 k per split.
int64_t gemm_splits(int64_t batch, int64_t M, int64_t N, int64_t K) {
    const int64_t base = cdiv(M, kGT) * cdiv(N, kGT) * batch;
    if (base == 0) return 1;  // no output tiles (an empty side): nothing to split
    const int64_t slots = gemm_slots();
    int64_t cap = K / 256;
    if (cap > 8) cap = 8;
    while (cap > 1 && cap * batch > kMaxGridYZ) --cap;
    int64_t best = 1;
    double best_fill = 0.0;
    for (int64_t sp = 1; sp <= (cap < 1 ? 1 : cap); ++sp) {
        const int64_t blocks = base * sp;
        const double fill = (double)blocks / (double)(cdiv(blocks, slots) * slots);
        if (fill >= 0.9) return sp;
        if (fill > best_fill + 1e-9) {
            best_fill = fill;
            best = sp;
        }
    }
    return best;
}

template <typename T, bool A_T>
int run_gemm(const float *A, const T *B, int64_t batch, int64_t M, int64_t N, int64_t K,
             float sign, const float *coef, const T *X, T *out, float *part, hipStream_t s) {
    const int64_t splits = gemm_splits(batch, M, N, K);
    const int64_t kps = cdiv(cdiv(K, splits), kGK) * kGK;
    dim3 grid((unsigned)cdiv(N, kGT), (unsigned)cdiv(M, kGT), (unsigned)(batch * splits));
    const bool vec = (K % 4 == 0) && (M % 4 == 0) && (N % 4 == 0) && aligned16(A) && aligned16(B);
    float *dst = splits > 1 ? part : nullptr;
    if (vec)
        hipLaunchKernelGGL((bwd_gemm_kernel<T, A_T, true>), grid, dim3(256), 0, s, A, B, M, N, K,
                           kps, batch, sign, coef, X, out, dst);
    else
        hipLaunchKernelGGL((bwd_gemm_kernel<T, A_T, false>), grid, dim3(256), 0, s, A, B, M, N, K,
                           kps, batch, sign, coef, X, out, dst);
    int rc = check_launch("bwd_gemm_kernel");
    if (rc != TPW_OK || splits == 1) return rc;
    const int64_t len = batch * M * N;
    hipLaunchKernelGGL((gemm_finish_kernel<T>), dim3((unsigned)cdiv(len, 256)), dim3(256), 0, s,
                       part, splits, len, M, N, sign, coef, X, out);
    return check_launch("gemm_finish_kernel");
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct BwdWs {
    float *S, *rowpart, *colpart, *coef1, *coef2, *part, *rn2;
    uint32_t *slow;
    void *W, *WT, *x1t, *x2t;  // element type of the inputs
};

// [S fp32 (cosine) | row partials | column partials | coef1 | coef2 | column reciprocals and
// the norm-range flag (fused fp32 cosine) | W | W^T | x1^T | x2^T |
// GEMM split partials], W and the transposes in the inputs' element type (sized for fp32;
// the fp32 path uses W and the split partials, the bf16 path W, W^T and the transposes).
BwdWs carve(void *ws, int64_t batch, int64_t n, int64_t m, int64_t d, size_t *total = nullptr) {
    char *base = static_cast<char *>(ws), *p = base;
    BwdWs w;
    auto take = [&](size_t bytes) {
        char *r = p;
        p += align256(bytes);
        return r;
    };
    w.S = reinterpret_cast<float *>(take(sizeof(float) * batch * n * m));
    // partials: the weight pass's tiles (256 columns, 128 rows) or the cosine tile kernel's
    // halves of 128 x 128 tiles, whichever are more
    const int64_t tjp = cdiv(m, kPWCols) > 2 * cdiv(m, 128) ? cdiv(m, kPWCols) : 2 * cdiv(m, 128);
    w.rowpart = reinterpret_cast<float *>(take(sizeof(float) * batch * tjp * n));
    // column partials: two per 128 x 128 tile (the cosine tile kernel), four per 128-row block
    // (the fused fp32 cosine kernel), or one per weight-pass tile
    w.colpart = reinterpret_cast<float *>(take(sizeof(float) * batch * 4 * cdiv(n, 128) * m));
    w.coef1 = reinterpret_cast<float *>(take(sizeof(float) * batch * n));
    w.coef2 = reinterpret_cast<float *>(take(sizeof(float) * batch * m));
    w.rn2 = reinterpret_cast<float *>(take(sizeof(float) * batch * m));
    w.slow = reinterpret_cast<uint32_t *>(take(sizeof(uint32_t)));
    w.W = take(sizeof(float) * batch * n * m);
    w.WT = take(sizeof(float) * batch * n * m);
    w.x1t = take(sizeof(float) * batch * n * d);
    w.x2t = take(sizeof(float) * batch * m * d);
    const int64_t s1 = gemm_splits(batch, n, d, m), s2 = gemm_splits(batch, m, d, n);
    const int64_t p1 = s1 > 1 ? s1 * batch * n * d : 0, p2 = s2 > 1 ? s2 * batch * m * d : 0;
    w.part = reinterpret_cast<float *>(take(sizeof(float) * (p1 > p2 ? p1 : p2)));
    if (total) *total = (size_t)(p - base);
    return w;
}

size_t workspace_bytes(int64_t batch, int64_t n, int64_t m, int64_t d) {
    size_t total = 0;
    carve(nullptr, batch, n, m, d, &total);
    return total;
}

// x [batch, rows, d] -> xt [batch, d, rows], through a 64 x 64 LDS tile.
template <typename T>
__global__ void transpose_kernel(const T *__restrict__ x, int64_t rows, int64_t d, T *__restrict__ xt) {
    __shared__ T t[64][65];
    const int64_t b = blockIdx.z, r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int rr = ty; rr < 64; rr += 4) {
        const int64_t r = r0 + rr, c = c0 + tx;
        t[rr][tx] = (r < rows && c < d) ? x[(b * rows + r) * d + c] : T(0);
    }
    __syncthreads();
    for (int cc = ty; cc < 64; cc += 4) {
        const int64_t c = c0 + cc, r = r0 + tx;
        if (c < d && r < rows) xt[(b * d + c) * rows + r] = t[tx][cc];
    }
}

// Zeroes len 16-bit words (fills with a kernel, not hipMemsetAsync).
__global__ void zero_words_kernel(uint16_t *__restrict__ p, int64_t len) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t < len) p[t] = 0;
}

// Weight pass and grad_x1 product in one kernel (fp32; euclidean, sqeuclidean, polynomial,
// sigmoid, and the output-based cosine modes).  A block owns a
// 128 x 256 tile of grad_x1 = sign * W . x2 + coef1 * x1, K = m in 32-column chunks: grad
// (and res / S) of the tile's rows travel by DMA into k-contiguous panels (tile_mfma.hpp's
// layout), x2's chunk (32 rows x 256 columns, k-major) into a third panel.  Wave w owns rows
// 32 w .. 32 w + 31 across all 256 columns (8 MFMA blocks), so each weight is formed once per
// block, by the lane that feeds it to the MFMA (weight_terms: the same values as the weight
// pass), and written once to W for the grad_x2 product; coef1[i] = sum_j rt accumulates per
// lane in K order (each lane sums its half of every chunk; the halves are added at the end).
// The weights of step q + 1 are formed while step q's products run.  One 64 KiB buffer, two
// blocks per CU.
// The cosine modes read the forward's output as the second panel and the norms: the lane's row
// norm n1 once, the chunk's 32 column norms n2 with the chunk's DMA.  Their row terms divide by
// n1 at the end (coef1 = sum_j rt / n1, 0 where n1 = 0, as reduce_parts_kernel does), and their
// column terms ct are summed per chunk over each wave's 32 rows (a butterfly over the lanes) and
// written as partials colpart[b][4 tr + wave][j] (column blocks tc > 0 repeat the same weights
// and write none); reduce_parts_kernel adds the 4 cdiv(n, 128) partials in order for coef2.
constexpr int kFCols = 256;

// The fused grad_x1 kernels own a 128 x 256 tile of grad_x1 ([n, d]) and loop over all of m,
// so their grid is only cdiv(n, 128) cdiv(d, 256) batch blocks: below two per CU they leave the
// GPU half idle (16384 x 16384 x 128 polynomial: 128 blocks, 3.5 ms against 1.1 ms for the weight
// pass and the two tile-kernel products), and the unfused path runs instead.
// (Their grad_x2 product, m x d on the tile kernel, has to fill the GPU as well.)
bool fused_grid_fills(int64_t batch, int64_t n, int64_t m, int64_t d) {
    return cdiv(n, tile::kT) * cdiv(d, kFCols) * batch >= 2 * device_cus() && tile_grid_fills(batch, m, d);
}
template <int MODE, bool FAST = false>
__global__ __launch_bounds__(256, 2) void fused_grad1_kernel(
    const float *__restrict__ g, const float *__restrict__ av, const float *__restrict__ x2,
    const float *__restrict__ x1, int64_t n, int64_t m, int64_t d, float *__restrict__ W, float *__restrict__ gx1,
    int64_t tiles_n, int64_t tiles_c, int64_t total, KerParams kp, float sign, const float *__restrict__ n1,
    const float *__restrict__ n2, float *__restrict__ colpart, const float *__restrict__ rn2,
    const uint32_t *__restrict__ slow) {
    using namespace tile;
    constexpr bool kCos = kCosO<MODE>;
    // column terms summed into partials: cosine's gden n1, and the weights themselves for
    // euclidean / sqeuclidean (coef2 = sum_i W)
    constexpr bool kColT = kCos || MODE == kEuclid || MODE == kSqEuclid;
    // the cosine pair of launches: the FAST instance runs when every norm lies in [2^-60, 2^60],
    // the other one otherwise (the flag is the same for every block)
    if constexpr (kCos)
        if ((__builtin_amdgcn_readfirstlane(*slow) != 0u) == FAST) return;
    constexpr bool kAv = MODE == kEuclid || MODE == kSigmoid || MODE == kPoly || kCos;
    __shared__ uint4 smem[4 * kPanel];  // grad | res or S | x2 (two panels)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave * 32;
    const int l32 = lane & 31, h = lane >> 5;
    int64_t b, tr, tc;
    xcd_tile_of(blockIdx.x, tiles_n, tiles_c, total, b, tr, tc);
    const int64_t row0 = tr * kT, col0 = tc * kFCols;
    const uint8_t *G = reinterpret_cast<const uint8_t *>(g + b * n * m);
    const uint8_t *AV = kAv ? reinterpret_cast<const uint8_t *>(av + b * n * m) : G;
    const uint8_t *X2 = reinterpret_cast<const uint8_t *>(x2 + b * m * d);
    // 16 DMA slots per lane and chunk: wave 0 the grad panel, wave 1 the res / S panel, waves
    // 2 and 3 the x2 panel (K row kr at 64 positions, columns xor 32 for K rows 16..31)
    uint32_t off[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int s = (wave * 16 + j) * 64 + lane;
        if (s < 2 * kPanel) {
            const int r = (s >> 3) & (kT - 1), p = s & 7;
            const int64_t row = row0 + r < n ? row0 + r : n - 1;
            off[j] = (uint32_t)(row * m * 4 + swz(r, p) * 16);
        } else {
            const int t = s - 2 * kPanel, kr = t >> 6, lp = (t & 63) ^ ((kr >> 4) << 3);
            int64_t c = col0 + 4 * lp;
            c = c < d ? c : d - 4;
            off[j] = (uint32_t)(kr * d * 4 + c * 4);
        }
    }
    floatx16 acc[8];
#pragma unroll
    for (int ni = 0; ni < 8; ++ni)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[ni][r] = 0.0f;
    float rsum = 0.0f;
    // the lane's row; rows past n read row n - 1 (the same clamped inputs) and store nothing; the
    // tiles of further column blocks store the same W values again
    const int r = wr + l32;
    const int64_t wrow = row0 + r < n ? row0 + r : n - 1;
    const uint4 *Gs = smem, *As = smem + kPanel, *Bs = smem + 2 * kPanel;
    const float a1 = kCos ? n1[b * n + wrow] : 0.0f;  // the lane's row norm
    const float r1 = kCos && FAST ? __fdiv_rn(1.0f, a1) : 0.0f;
    // the lane's 16 column norms (reciprocals for FAST) and column terms of the chunk (K = 16 h + v)
    floatx16 n2c, ctv;
    // the weights of the lane's piece at step q of the chunk (K = 16 h + 4 q + e), and their row
    // terms into rsum (vector types, not arrays: an array here is placed in LDS by the compiler)
    auto weights = [&](int q) {
        const int c = h * 4 + q;
        const floatx4 gv = __builtin_bit_cast(floatx4, piece(Gs, r, c));
        const floatx4 avv = kAv ? __builtin_bit_cast(floatx4, piece(As, r, c)) : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        floatx4 w;
        if constexpr (MODE == kEuclid) {
            // g / res by the reciprocal without fast_div's branch per pair: one test of the
            // piece's four denominators, and weight_terms itself (0 for res = 0, else fast_div)
            // when one of them lies outside [2^-126, 2^126] (0, inf and NaN included; the
            // forward's res is 0 only on a self-distance diagonal).  Inside the range the
            // product with the reciprocal is fast_div's value, so both routes give the same
            // weights; a range test per element (two compares) costs less than telling the
            // quotients that need fast_div's divide from those that do not (four compares and a
            // select per element: 0.16 ms of the C2 euclidean backward)
            bool ok = true;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ay = __builtin_fabsf(avv[e]);
                ok = ok && ay >= 0x1p-126f && ay <= 0x1p126f;
                w[e] = gv[e] * __builtin_amdgcn_rcpf(avv[e]);
            }
            if (__builtin_expect(__ballot(!ok) != 0ull, 0)) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float we, rt, ct;
                    weight_terms<MODE, false>(gv[e], avv[e], 0.0f, 0.0f, kp, we, rt, ct);
                    w[e] = we;
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                rsum += w[e];
                ctv[4 * q + e] = w[e];
            }
            return w;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float we, rt, ct;
            if constexpr (kCos && FAST) cos_terms_fast<MODE>(gv[e], avv[e], r1, n2c[4 * q + e], we, rt, ct);
            else weight_terms<MODE, false>(gv[e], avv[e], a1, kCos ? n2c[4 * q + e] : 0.0f, kp, we, rt, ct);
            w[e] = we;
            rsum += rt;
            if constexpr (kColT) ctv[4 * q + e] = ct;
        }
        return w;
    };
    // column partials: only the first column block, and zeros for a wave past the last row (n is
    // a multiple of 32, so a wave's rows are all valid or all past the end)
    const bool col_writer = tc == 0;
    const bool rows_ok = row0 + wr < n;
    float *cp = kColT ? colpart + (b * 4 * tiles_n + 4 * tr + wave) * m : nullptr;
    // W leaves as whole 128-byte lines.  Stored piece by piece from the lanes that formed them,
    // each instruction wrote 16-byte parts of 32 lines, which reached HBM in parts (1.5x W's
    // bytes).  Euclidean and the kernel functions: each lane puts its weight pieces into the grad
    // slots they were formed from (only that lane reads them), and at the end of the chunk lane
    // (lr, lp) = (lane / 8, lane % 8) stores piece lp of row wr + 8 i + lr (i < 4); element
    // offsets from the batch's W stay below 2^31 (n m 4 < 2^32).  Cosine, whose extra registers
    // leave no room for that (it spilled): each lane keeps its 16 weights of the chunk, its 64
    // contiguous bytes of the line (the partner lane has the other 64), and stores them together
    // one chunk later (after the next barrier, which would otherwise wait for them).
    constexpr bool kLdsW = !kCos;
    float *Wrow = kCos ? W + (b * n + wrow) * m : nullptr;
    floatx16 wst;
    auto store_w = [&](int kw) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<floatx4 *>(Wrow + (int64_t)kw * 32 + 4 * (h * 4 + q)) =
                floatx4{wst[4 * q], wst[4 * q + 1], wst[4 * q + 2], wst[4 * q + 3]};
    };
    const int lr = lane >> 3, lx = (lane & 7) ^ lr;
    float *Wb = W + b * n * m;
    const int64_t wrow_l = row0 + wr + lr < n ? row0 + wr + lr : n - 1;
    const uint32_t woff = (uint32_t)(wrow_l * m + 4 * (lane & 7));
    const uint32_t wstep = (uint32_t)(8 * m);
    const int nchunks = (int)(m / 32);
    for (int kc = 0; kc < nchunks; ++kc) {
        if (kc > 0) barrier_lds();  // every wave is done with chunk kc - 1
        if (wave != 1 || kAv) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int first = (wave * 16 + j) * 64;
                const uint8_t *base = first < kPanel       ? G + (int64_t)kc * 128
                                      : first < 2 * kPanel ? AV + (int64_t)kc * 128
                                                           : X2 + (int64_t)kc * 128 * d;
                dma16(base, off[j], lds_addr(smem + first));
            }
        }
        if constexpr (kCos) {
            const floatx4 *np = reinterpret_cast<const floatx4 *>((FAST ? rn2 : n2) + b * m + (int64_t)kc * 32 + 16 * h);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const floatx4 v = np[q];
#pragma unroll
                for (int e = 0; e < 4; ++e) n2c[4 * q + e] = v[e];
            }
        }
        barrier_all();
        // the previous chunk's W pieces, now that this chunk's barrier is behind them (the next
        // barrier waits for them, a chunk later)
        if constexpr (!kLdsW)
            if (kc > 0) store_w(kc - 1);
        floatx4 wn = weights(0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const floatx4 a = wn;
            floatx4 bv[8];
#pragma unroll
            for (int ni = 0; ni < 8; ++ni) {
                const float *f = reinterpret_cast<const float *>(Bs) + (16 * h + 4 * q) * kFCols +
                                 ((ni * 32 + l32) ^ (32 * h));
                bv[ni] = floatx4{f[0], f[kFCols], f[2 * kFCols], f[3 * kFCols]};
            }
            if constexpr (kLdsW) {
                smem[r * 8 + swz(r, h * 4 + q)] = __builtin_bit_cast(uint4, a);  // into its grad slot
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) wst[4 * q + e] = a[e];
            }
            if (q < 3) wn = weights(q + 1);  // formed while this step's products run
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int ni = 0; ni < 8; ++ni)
                    acc[ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(bv[ni][e], a[e], acc[ni], 0, 0, 0);
            if (q < 3) {
                // one product, then two VALU instructions, over the step
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
                }
            }
        }
        if constexpr (kLdsW) {
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes landed
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // row wr + 8 i + lr, piece lp: slot swz = lp ^ lr ^ (i & 1) (wr is a multiple of 32)
                const uint4 v = smem[(wr + 8 * i + lr) * 8 + (lx ^ (i & 1))];
                if (row0 + wr + 8 * i + lr < n)
                    *reinterpret_cast<uint4 *>(Wb + (uint32_t)(woff + i * wstep + kc * 32)) = v;
            }
        }
        if constexpr (kColT) {
            // the chunk's column terms summed over the wave's 32 rows (lanes of equal h): each
            // step hands half of the lane's values to its partner; lane (l32, h) ends with
            // column 16 h + (l32 >> 1), in both lanes of a pair
            float t8[8], t4[4], t2[2];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const bool up = (l32 & 16) != 0;
                const float mine = up ? ctv[8 + i] : ctv[i], other = up ? ctv[i] : ctv[8 + i];
                t8[i] = mine + __shfl_xor(other, 16, 64);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool up = (l32 & 8) != 0;
                const float mine = up ? t8[4 + i] : t8[i], other = up ? t8[i] : t8[4 + i];
                t4[i] = mine + __shfl_xor(other, 8, 64);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const bool up = (l32 & 4) != 0;
                const float mine = up ? t4[2 + i] : t4[i], other = up ? t4[i] : t4[2 + i];
                t2[i] = mine + __shfl_xor(other, 4, 64);
            }
            const bool up2 = (l32 & 2) != 0;
            float t1 = (up2 ? t2[1] : t2[0]) + __shfl_xor(up2 ? t2[0] : t2[1], 2, 64);
            t1 += __shfl_xor(t1, 1, 64);
            if (col_writer && (l32 & 1) == 0) cp[(int64_t)kc * 32 + 16 * h + (l32 >> 1)] = rows_ok ? t1 : 0.0f;
        }
    }
    if constexpr (!kLdsW) store_w(nchunks - 1);
    barrier_lds();  // the buffer becomes the output stage
    float a1v = rsum + __shfl_xor(rsum, 32, 64);  // both K halves
    if constexpr (kCos) a1v = a1 == 0.0f ? 0.0f : __fdiv_rn(a1v, a1);
    floatx4 *sl = reinterpret_cast<floatx4 *>(smem) + wave * 1024;  // 16 KiB per wave
#pragma unroll
    for (int half = 0; half < 2; ++half)
        store_wave_rows_f32<4>(
            sl,
            [&](int ni, int gq) {
                const int64_t row = row0 + r, col = col0 + half * 128 + ni * 32 + 8 * gq + 4 * h;
                floatx4 xv = {0.0f, 0.0f, 0.0f, 0.0f};
                if (row < n && col < d) xv = *reinterpret_cast<const floatx4 *>(x1 + (b * n + row) * d + col);
                floatx4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = sign * acc[half * 4 + ni][4 * gq + e] + a1v * xv[e];
                return o;
            },
            gx1, b, row0 + wr, col0 + half * 128, n, d);
}

// The same for bf16: 64-column K chunks (128 bytes of a row), grad and res / S as bf16 panels,
// x2's chunk (64 K rows x 256 columns) k-major, read through transposing LDS reads; each
// weight is formed in fp32 and rounded to bf16 as the weight pass stores it (weight_terms
// with BF16W, then round to nearest even), fed to v_mfma_f32_32x32x16_bf16 and written to W;
// coef1 sums the row terms (the rounded weights for euclidean).  grad_x1 leaves as bf16.
// The output-based cosine modes work as in the fp32 kernel (a FAST instance on reciprocal norms
// and a dividing one, the norm-range flag choosing): the second panel is the forward's bf16
// output and the chunk's 64 column reciprocals (or norms) come by DMA into LDS with the panels.
// Their column coefficients are left to cos_proj_finish_kernel (summing the column terms here
// took more registers than the two blocks per CU leave: the kernel spilled).
template <int MODE, bool FAST = false>
__global__ __launch_bounds__(256, 2) void fused_grad1_bf16_kernel(
    const uint16_t *__restrict__ g, const uint16_t *__restrict__ av, const uint16_t *__restrict__ x2,
    const uint16_t *__restrict__ x1, int64_t n, int64_t m, int64_t d, uint16_t *__restrict__ W,
    uint16_t *__restrict__ gx1, int64_t tiles_n, int64_t tiles_c, int64_t total, KerParams kp, float sign,
    const float *__restrict__ n1, const float *__restrict__ n2, const float *__restrict__ rn2,
    const uint32_t *__restrict__ slow) {
    using namespace tile;
    constexpr bool kCos = kCosO<MODE>;
    if constexpr (kCos)
        if ((__builtin_amdgcn_readfirstlane(*slow) != 0u) == FAST) return;
    constexpr bool kAv = MODE == kEuclid || MODE == kSigmoid || MODE == kPoly || kCos;
    __shared__ uint4 smem[4 * kPanel];  // grad | res or S | x2 (two panels)
    __shared__ __align__(16) float s_n2[64];  // cosine: the chunk's column reciprocals (FAST) or norms
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave * 32;
    const int l32 = lane & 31, h = lane >> 5;
    const int grp = ((lane >> 4) & 1) * 16;  // first row of the lane's 16-lane group
    int64_t b, tr, tc;
    xcd_tile_of(blockIdx.x, tiles_n, tiles_c, total, b, tr, tc);
    const int64_t row0 = tr * kT, col0 = tc * kFCols;
    const uint8_t *G = reinterpret_cast<const uint8_t *>(g + b * n * m);
    const uint8_t *AV = kAv ? reinterpret_cast<const uint8_t *>(av + b * n * m) : G;
    const uint8_t *X2 = reinterpret_cast<const uint8_t *>(x2 + b * m * d);
    // 16 DMA slots per lane and chunk, slot j at a wave-uniform stride from a per-lane offset
    // that depends only on j's parity (two registers): wave 0 the grad panel, wave 1 the res / S
    // panel (tile row 8 j + lane / 8, position lane % 8; n % 128 == 0, so no row clamps), waves
    // 2 and 3 the x2 panel (K row 32 (wave - 2) + 2 j + lane / 32 at position lane % 32, logical
    // piece position ^ 4 (kr & 3))
    uint32_t off_par[2];
    int64_t jstride;
    if (wave < 2) {
        jstride = 8 * m * 2;
#pragma unroll
        for (int par = 0; par < 2; ++par)
            off_par[par] = (uint32_t)((row0 + (lane >> 3)) * m * 2 + 16 * ((lane & 7) ^ ((lane >> 3) & 7) ^ par));
    } else {
        jstride = 2 * d * 2;
        const int kr0 = 32 * (wave - 2) + (lane >> 5);
#pragma unroll
        for (int par = 0; par < 2; ++par) {
            const int lp = (lane & 31) ^ (4 * ((kr0 + 2 * par) & 3));
            int64_t c = col0 + 8 * lp;
            c = c < d ? c : d - 8;
            off_par[par] = (uint32_t)(kr0 * d * 2 + c * 2);
        }
    }
    floatx16 acc[8];
#pragma unroll
    for (int ni = 0; ni < 8; ++ni)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[ni][r] = 0.0f;
    float rsum = 0.0f;
    // the lane's W row; rows past n store row n - 1, whose weights they duplicate exactly
    const int r = wr + l32;
    const int64_t wrow = row0 + r < n ? row0 + r : n - 1;
    const uint4 *Gs = smem, *As = smem + kPanel, *Bs = smem + 2 * kPanel;
    // the W line stores (euclidean and the kernel functions; the cosine kernel has no registers to
    // spare for them and stores each piece as it is formed): lane (lr, lp) = (lane / 8, lane % 8)
    // writes piece lp of row wr + 8 i + lr (i < 4) of each chunk; element offsets from the batch's
    // W below 2^31 (n m 2 < 2^32)
    constexpr bool kLdsW = !kCos;
    const int lr = lane >> 3, lx = (lane & 7) ^ lr;
    uint16_t *Wb = W + b * n * m;
    const uint32_t woff = (uint32_t)((row0 + wr + lr) * m + 8 * (lane & 7));
    // cosine: the lane's row norm and reciprocal
    const float a1 = kCos ? n1[b * n + wrow] : 0.0f;
    const float r1 = kCos && FAST ? __fdiv_rn(1.0f, a1) : 0.0f;
    const uint8_t *NC = kCos ? reinterpret_cast<const uint8_t *>((FAST ? rn2 : n2) + b * m) : nullptr;
    // the bf16 weights of the lane's piece at step q (K = 32 h + 8 q + e), their row terms
    // into rsum
    auto weights = [&](int q) {
        const int c = h * 4 + q;
        const uint4 gp = piece(Gs, r, c);
        const uint4 ap = kAv ? piece(As, r, c) : make_uint4(0, 0, 0, 0);
        const uint32_t gw[4] = {gp.x, gp.y, gp.z, gp.w}, aw[4] = {ap.x, ap.y, ap.z, ap.w};
        uint32_t o[4];
        if constexpr (kCos) {
            // the lane's 8 pairs (K = 32 h + 8 q + k): weights and row terms (the column
            // coefficients come from the grad_x2 product afterwards, cos_proj_finish_kernel)
            const floatx4 nA = *reinterpret_cast<const floatx4 *>(&s_n2[32 * h + 8 * q]);
            const floatx4 nB = *reinterpret_cast<const floatx4 *>(&s_n2[32 * h + 8 * q + 4]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float wv[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int k = 2 * e + u;
                    const float gvv = __uint_as_float(u ? gw[e] & 0xffff0000u : gw[e] << 16);
                    const float avv = __uint_as_float(u ? aw[e] & 0xffff0000u : aw[e] << 16);
                    const float nv = k < 4 ? nA[k] : nB[k - 4];
                    float we, rt, ct;
                    if constexpr (FAST) cos_terms_fast<MODE>(gvv, avv, r1, nv, we, rt, ct);
                    else weight_terms<MODE, true>(gvv, avv, a1, nv, kp, we, rt, ct);
                    wv[u] = we;
                    rsum += rt;
                }
                o[e] = f32x2_to_bf16x2_rne(wv[0], wv[1]);
            }
            return make_uint4(o[0], o[1], o[2], o[3]);
        }
        if constexpr (MODE == kEuclid) {
            // as the fp32 kernel: the reciprocal without a branch per pair, one range test of
            // the piece's eight denominators (weight_terms below when one lies outside
            // [2^-126, 2^126], 0, inf and NaN included); each weight rounded to bf16 once and
            // summed as rounded
            bool ok = true;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float wv[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const float gvv = __uint_as_float(u ? gw[e] & 0xffff0000u : gw[e] << 16);
                    const float avv = __uint_as_float(u ? aw[e] & 0xffff0000u : aw[e] << 16);
                    const float ay = __builtin_fabsf(avv);
                    ok = ok && ay >= 0x1p-126f && ay <= 0x1p126f;
                    wv[u] = gvv * __builtin_amdgcn_rcpf(avv);
                }
                o[e] = f32x2_to_bf16x2_rne(wv[0], wv[1]);
            }
            if (!__builtin_expect(__ballot(!ok) != 0ull, 0)) {
#pragma unroll
                for (int e = 0; e < 4; ++e) rsum += __uint_as_float(o[e] << 16) + __uint_as_float(o[e] & 0xffff0000u);
                return make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // rt: the rounded weight for euclidean / sqeuclidean (BF16W), 0 for the kernel functions
            float w0, w1, rt, ct;
            weight_terms<MODE, true>(__uint_as_float(gw[e] << 16), __uint_as_float(aw[e] << 16), 0.0f, 0.0f, kp,
                                     w0, rt, ct);
            rsum += rt;
            weight_terms<MODE, true>(__uint_as_float(gw[e] & 0xffff0000u), __uint_as_float(aw[e] & 0xffff0000u),
                                     0.0f, 0.0f, kp, w1, rt, ct);
            rsum += rt;
            o[e] = f32x2_to_bf16x2_rne(w0, w1);
        }
        return make_uint4(o[0], o[1], o[2], o[3]);
    };
    const int nchunks = (int)(m / 64);
    for (int kc = 0; kc < nchunks; ++kc) {
        if (kc > 0) barrier_lds();  // every wave is done with chunk kc - 1
        if (wave != 1 || kAv) {
            const uint8_t *base = wave == 0 ? G + (int64_t)kc * 128
                                  : wave == 1 ? AV + (int64_t)kc * 128
                                              : X2 + (int64_t)kc * 128 * d;
#pragma unroll
            for (int j = 0; j < 16; ++j)
                dma16(base + j * jstride, off_par[j & 1], lds_addr(smem + (wave * 16 + j) * 64));
        }
        if constexpr (kCos)
            if (wave == 3) dma4(NC + (int64_t)kc * 256, (uint32_t)lane * 4, lds_addr(s_n2));
        barrier_all();
        uint4 an = weights(0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint4 a = an;
            if constexpr (kLdsW) {
                // W's piece into the grad slot it was formed from (only this lane reads that
                // slot, and it has: the weights are formed from it)
                smem[r * 8 + swz(r, h * 4 + q)] = a;
            } else {
                *reinterpret_cast<uint4 *>(W + (b * n + wrow) * m + (int64_t)kc * 64 + 8 * (h * 4 + q)) = a;
            }
            if (q < 3) an = weights(q + 1);  // formed while this step's products run
#pragma unroll
            for (int ni = 0; ni < 8; ++ni) {
                const uint4 bv = kpiece_bf16<512>(Bs, ni * 32 + grp, lane, h, q);
                acc[ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, bv),
                                                                 __builtin_bit_cast(bf16x8, a), acc[ni], 0, 0, 0);
            }
            if (q < 3) {
                // one product, then eight VALU instructions, over the step
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
                }
            }
        }
        if constexpr (kLdsW) {
            // the wave's 32 W rows of the chunk (128 bytes each) leave as whole lines, 8 rows per
            // store: stored piece by piece from the lanes that formed them, each instruction wrote
            // 16-byte parts of 32 lines (W alone cost 0.27 ms of the kernel's 0.88 at C2)
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes landed
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // row wr + 8 i + lr, piece lp: slot swz = lp ^ lr ^ (i & 1) (wr is a multiple of 32)
                const uint4 v = smem[(wr + 8 * i + lr) * 8 + (lx ^ (i & 1))];
                *reinterpret_cast<uint4 *>(Wb + (uint32_t)(woff + i * 8 * (uint32_t)m + kc * 64)) = v;
            }
        }
    }
    barrier_lds();  // the buffer becomes the output stage
    float a1v = rsum + __shfl_xor(rsum, 32, 64);  // both K halves
    if constexpr (kCos) a1v = a1 == 0.0f ? 0.0f : __fdiv_rn(a1v, a1);
    uint4 *sl = smem + wave * 1024;  // 16 KiB per wave
    store_wave_rows_bf16<8>(
        sl,
        [&](int ni, int gq) {
            const int64_t row = row0 + r, col = col0 + ni * 32 + 8 * gq + 4 * h;
            floatx4 xv = {0.0f, 0.0f, 0.0f, 0.0f};
            if (row < n && col < d) {
                const uint2 qv = *reinterpret_cast<const uint2 *>(x1 + (b * n + row) * d + col);
                xv = floatx4{__uint_as_float(qv.x << 16), __uint_as_float(qv.x & 0xffff0000u),
                             __uint_as_float(qv.y << 16), __uint_as_float(qv.y & 0xffff0000u)};
            }
            floatx4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = sign * acc[ni][4 * gq + e] + a1v * xv[e];
            return o;
        },
        gx1, b, row0 + wr, col0, n, d);
}

// The bf16 fused path's shapes: whole 128-row tiles (n % 128 == 0), whole 64-element K chunks
// both ways, d a multiple of 8,
// 16-byte aligned arrays, per-batch byte offsets of grad below 2^32.
bool fused_bf16_fits(const void *g, const void *av, const uint16_t *x1, const uint16_t *x2, const uint16_t *W,
                     const uint16_t *gx1, const uint16_t *gx2, int64_t n, int64_t m, int64_t d) {
    return n > 0 && m > 0 && d > 0 && n % 128 == 0 && m % 64 == 0 && d % 8 == 0 && n * m * 2 < ((int64_t)1 << 32) &&
           aligned16(g) && aligned16(av) && aligned16(W) && aligned16(gx1) && aligned16(x1) && aligned16(x2) &&
           grad_product_bf16_fits(W, true, x1, true, m, d, n, x2, gx2);
}

// Cosine backward, S and the weight pass in one kernel: S = x1 . x2^T of a 128 x 128 tile on the
// matrix cores (the tile kernel's K loop), then per element the weight pass's weight_terms from
// S, grad and the row / column norms.  W leaves through the tile stage (type T; bf16 rounded as
// the pass stores it); the row terms of each wave's 64 columns go to rowpart (two partials per
// 128-column tile), the column terms of each wave's 64 rows to colpart (two per 128-row tile):
// a lane sums its two rows, then lane c sums column c over the 32 lanes through the wave's own
// LDS slice.  S never leaves the chip.  Two operand buffers (the next chunk's DMA in flight
// while the current one is multiplied) at two blocks per CU: the epilogue's divides need more
// than the 128 registers of four blocks.  Needs the tile kernel's direct-load shapes,
// m % (16 / sizeof(T)) == 0 and 16-byte aligned grad and W.
template <typename T, int MODE>
__global__ __launch_bounds__(tile::kThreads, 2) void cos_weights_tile_kernel(
    const T *__restrict__ x1, const T *__restrict__ x2, int64_t n, int64_t m, int64_t d, const float *__restrict__ n1,
    const float *__restrict__ n2, const T *__restrict__ g, T *__restrict__ Wo, float *__restrict__ rowpart,
    float *__restrict__ colpart, int64_t tiles_n, int64_t tiles_m, int64_t total) {
    using namespace tile;
    constexpr bool BF16W = sizeof(T) == 2;
    __shared__ uint4 smem[2 * kBuf];
    __shared__ __align__(16) float s_aux[2 * kT];  // row norms, then column norms
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
    const int l32 = lane & 31, h = lane >> 5;
    int64_t b, tr, tc;
    xcd_tile_of(blockIdx.x, tiles_n, tiles_m, total, b, tr, tc);
    const int64_t row0 = tr * kT, col0 = tc * kT;
    const int64_t row_bytes = d * (int64_t)sizeof(T);
    const uint8_t *A = reinterpret_cast<const uint8_t *>(x1 + b * n * d);
    const uint8_t *B = reinterpret_cast<const uint8_t *>(x2 + b * m * d);
    dma_tile_rows(n1 + b * n, n2 + b * m, true, wave, lane, row0, col0, n, m, s_aux);
    uint32_t off[kSlots];
    dma_offsets(off, wave, lane, row0, col0, n, m, row_bytes);
    dma_chunk(A, B, off, wave, 0, smem);
    floatx16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.0f;
    const int nchunks = (int)(row_bytes / 128);
    for (int kc = 0; kc < nchunks; ++kc) {
        barrier_all();  // chunk kc (and, the first time, the norms) has landed
        // chunk kc + 1 goes to the buffer chunk kc - 1 used, which every wave is done with
        if (kc + 1 < nchunks) dma_chunk(A, B, off, wave, (int64_t)(kc + 1) * 128, smem + ((kc + 1) & 1) * kBuf);
        const uint4 *As = smem + (kc & 1) * kBuf, *Bs = As + kPanel;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int c = h * 4 + q;
            uint4 a[2], bv[2];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) a[mi] = piece(As, wr + mi * 32 + l32, c);
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) bv[ni] = piece(Bs, wc + ni * 32 + l32, c);
            mfma_piece_t(acc, a, bv, T{});
        }
    }
    barrier_lds();  // the operand buffers become the column-sum slices, then the output stage

    // weights in place of S; row terms per lane; column terms per lane over its two rows, one
    // column block at a time, into the wave's slice as [row l32][unit u ^ (l32 & 15)]
    float rs[2] = {0.0f, 0.0f};
    floatx4 *sl = reinterpret_cast<floatx4 *>(smem) + wave * 512;
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
        floatx4 cs[4];
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) cs[gq] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
            const int64_t row = row0 + wr + mi * 32 + l32;
            const float a1 = s_aux[wr + mi * 32 + l32];
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                const int cl = wc + ni * 32 + 8 * gq + 4 * h;
                const int64_t col = col0 + cl;
                const bool ok = row < n && col < m;  // m % 4 == 0: the quad is all in or all out
                floatx4 gv = {0.0f, 0.0f, 0.0f, 0.0f};
                if (ok) {
                    const T *gp = g + (b * n + row) * m + col;
                    if constexpr (BF16W) {
                        const uint2 qv = *reinterpret_cast<const uint2 *>(gp);
                        gv = floatx4{__uint_as_float(qv.x << 16), __uint_as_float(qv.x & 0xffff0000u),
                                     __uint_as_float(qv.y << 16), __uint_as_float(qv.y & 0xffff0000u)};
                    } else {
                        gv = *reinterpret_cast<const floatx4 *>(gp);
                    }
                }
                const floatx4 a2 = *reinterpret_cast<const floatx4 *>(&s_aux[kT + cl]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float w = 0.0f, rt = 0.0f, ct = 0.0f;
                    if (ok) weight_terms<MODE, BF16W>(gv[e], acc[mi][ni][4 * gq + e], a1, a2[e], KerParams{}, w, rt, ct);
                    acc[mi][ni][4 * gq + e] = w;
                    rs[mi] += rt;
                    cs[gq][e] += ct;
                }
            }
        }
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
            const int u = ni * 8 + 2 * gq + h;
            sl[l32 * 16 + (u ^ (l32 & 15))] = cs[gq];
        }
    }
    // row partials over the wave's 64 columns
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
        const float v = rs[mi] + __shfl_xor(rs[mi], 32, 64);
        const int64_t row = row0 + wr + mi * 32 + l32;
        if (h == 0 && row < n) rowpart[(b * 2 * tiles_m + 2 * tc + (wave & 1)) * n + row] = v;
    }
    // column partials over the wave's 64 rows: lane c sums column c of the slice
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    {
        const float *f = reinterpret_cast<const float *>(sl);
        float v = 0.0f;
#pragma unroll
        for (int r = 0; r < 32; ++r) v += f[r * 64 + (((lane >> 2) ^ (r & 15)) << 2) + (lane & 3)];
        const int64_t col = col0 + wc + lane;
        if (col < m) colpart[(b * 2 * tiles_n + 2 * tr + (wave >> 1)) * m + col] = v;
    }
    barrier_lds();  // every wave's column reads are done before the stage is rewritten
    store_tile<T>(
        smem,
        [&](int mi, int ni, int gq) {
            return floatx4{acc[mi][ni][4 * gq], acc[mi][ni][4 * gq + 1], acc[mi][ni][4 * gq + 2],
                           acc[mi][ni][4 * gq + 3]};
        },
        Wo, b, row0, col0, n, m);
}

// cos_weights_tile_kernel's shapes (the tile kernel's direct-load conditions, whole 16-byte
// units per W row, 16-byte aligned grad and W).
template <typename T>
bool cos_fused_fits(const T *x1, const T *x2, const T *g, const T *W, int64_t n, int64_t m, int64_t d) {
    constexpr int64_t ES = (int64_t)sizeof(T);
    return n > 0 && m > 0 && d > 0 && (d * ES) % 128 == 0 && aligned16(x1) && aligned16(x2) && aligned16(g) &&
           aligned16(W) && m % (16 / ES) == 0 && (n > m ? n : m) * d * ES < ((int64_t)1 << 32);
}

// The fused path's shapes: whole K chunks both ways (m and n multiples of 32), d a multiple of
// 4, 16-byte aligned arrays, per-batch byte offsets of grad below 2^32.
bool fused_fits(const void *g, const void *av, const float *x1, const float *x2, const void *W, const void *gx1,
                const void *gx2, int64_t n, int64_t m, int64_t d) {
    return n > 0 && m > 0 && d > 0 && n % 32 == 0 && m % 32 == 0 && d % 4 == 0 && n * m * 4 < ((int64_t)1 << 32) &&
           aligned16(g) && aligned16(av) && aligned16(W) && aligned16(gx1) &&
           grad_product_f32_fits(static_cast<const float *>(W), true, x1, true, m, d, n, x2,
                                 static_cast<const float *>(gx2)) &&
           aligned16(x1) && aligned16(x2);
}

// fp32 gx1 = sign * W . x2 + coef1 * x1 and gx2 = sign * W^T . x1 + coef2 * x2.  The tile
// kernel reads the operands in place, x2 (for gx1) and W, x1 (for gx2) k-major, where the
// shapes allow; otherwise the split-K GEMM.
int products_f32(const float *W, const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m, int64_t d,
                 float sign, const BwdWs &w, float *gx1, float *gx2, hipStream_t s) {
    if (grad_product_f32_fits(W, false, x2, true, n, d, m, x1, gx1) &&
        grad_product_f32_fits(W, true, x1, true, m, d, n, x2, gx2) && tile_grid_fills(batch, n, d) &&
        tile_grid_fills(batch, m, d)) {
        const int rc = grad_product_f32(W, false, x2, true, batch, n, d, m, sign, w.coef1, x1, gx1, s);
        if (rc) return rc;
        return grad_product_f32(W, true, x1, true, batch, m, d, n, sign, w.coef2, x2, gx2, s);
    }
    const int rc = run_gemm<float, false>(W, x2, batch, n, d, m, sign, w.coef1, x1, gx1, w.part, s);
    if (rc) return rc;
    return run_gemm<float, true>(W, x1, batch, m, d, n, sign, w.coef2, x2, gx2, w.part, s);
}

template <typename T, int MODE>
int run_backward(const T *g, const T *x1, const T *x2, const T *res, const float *n1,
                 const float *n2, int dtype, int64_t batch, int64_t n, int64_t m, int64_t d, T *gx1,
                 T *gx2, void *ws, hipStream_t s, KerParams kp = {}) {
    BwdWs w = carve(ws, batch, n, m, d);
    T *W = static_cast<T *>(w.W), *WT = static_cast<T *>(w.WT);
    T *x1t = static_cast<T *>(w.x1t), *x2t = static_cast<T *>(w.x2t);
    int rc = TPW_OK;
    constexpr bool kBf16 = sizeof(T) == 2;
    constexpr bool kCosMode = kCosS<MODE>;  // S recomputed (the output-based modes read res)
    // bf16: the tile kernel reads x2 (for gx1) and W, x1 (for gx2) k-major in place where the
    // shapes allow (no W^T, no transposed inputs)
    bool bf16_kmajor = false;
    if constexpr (kBf16)
        bf16_kmajor = grad_product_bf16_fits(W, false, x2, true, n, d, m, x1, gx1) &&
                      grad_product_bf16_fits(W, true, x1, true, m, d, n, x2, gx2) &&
                      tile_grid_fills(batch, n, d) && tile_grid_fills(batch, m, d);
    // cosine: S and the weight pass in one kernel (cos_weights_tile_kernel) where it fits and,
    // for bf16, the products need no W^T
    bool cos_fused = false;
    if constexpr (kCosMode) cos_fused = cos_fused_fits(x1, x2, g, W, n, m, d) && (!kBf16 || bf16_kmajor);
    if constexpr (kCosMode || MODE == kPoly) {
        if (!cos_fused) {
            rc = inner_dot_f32(x1, x2, dtype, batch, n, m, d, w.S, s);
            if (rc) return rc;
        }
    }
    if constexpr (MODE == kDot && !kBf16) {
        // fp32: grad is the weight matrix as stored; no weight pass, zero coefficients
        hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)cdiv(2 * batch * n, 256)), dim3(256), 0, s,
                           reinterpret_cast<uint16_t *>(w.coef1), 2 * batch * n);
        hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)cdiv(2 * batch * m, 256)), dim3(256), 0, s,
                           reinterpret_cast<uint16_t *>(w.coef2), 2 * batch * m);
        rc = check_launch("zero_words_kernel");
        if (rc) return rc;
        return products_f32(reinterpret_cast<const float *>(g), reinterpret_cast<const float *>(x1),
                            reinterpret_cast<const float *>(x2), batch, n, m, d, 1.0f, w,
                            reinterpret_cast<float *>(gx1), reinterpret_cast<float *>(gx2), s);
    }
    if constexpr (!kBf16 && (MODE == kEuclid || MODE == kSqEuclid || MODE == kSigmoid || MODE == kPoly)) {
        // fp32: weights formed inside the grad_x1 product (which also writes W); grad_x2 takes
        // coef2 = the column sums of W from its own operand (zero for the kernel functions)
        const float *gf = reinterpret_cast<const float *>(g);
        const float *av = MODE == kPoly ? w.S : reinterpret_cast<const float *>(res);
        const float *x1f = reinterpret_cast<const float *>(x1), *x2f = reinterpret_cast<const float *>(x2);
        float *Wf = reinterpret_cast<float *>(W);
        float *g1 = reinterpret_cast<float *>(gx1), *g2 = reinterpret_cast<float *>(gx2);
        if (fused_fits(gf, MODE == kSqEuclid ? gf : av, x1f, x2f, Wf, g1, g2, n, m, d) &&
            fused_grid_fills(batch, n, m, d)) {
            const float sign = (MODE == kPoly || MODE == kSigmoid) ? 1.0f : -1.0f;
            const int64_t tiles_n = cdiv(n, tile::kT), tiles_c = cdiv(d, kFCols), total = tiles_n * tiles_c * batch;
            hipLaunchKernelGGL((fused_grad1_kernel<MODE>), dim3((unsigned)total), dim3(256), 0, s, gf, av, x2f, x1f,
                               n, m, d, Wf, g1, tiles_n, tiles_c, total, kp, sign, static_cast<const float *>(nullptr),
                               static_cast<const float *>(nullptr), w.colpart, static_cast<const float *>(nullptr),
                               static_cast<const uint32_t *>(nullptr));
            rc = check_launch("fused_grad1_kernel");
            if (rc) return rc;
            if constexpr (MODE == kEuclid || MODE == kSqEuclid) {
                // coef2 = sum_i W from the kernel's column partials
                hipLaunchKernelGGL(reduce_parts_kernel, dim3((unsigned)cdiv(batch * m, 256)), dim3(256), 0, s,
                                   w.colpart, 4 * tiles_n, m, batch, static_cast<const float *>(nullptr), w.coef2);
                rc = check_launch("reduce_parts_kernel");
                if (rc) return rc;
                return grad_product_f32(Wf, true, x1f, true, batch, m, d, n, sign, w.coef2, x2f, g2, s);
            }
            hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)cdiv(2 * batch * m, 256)), dim3(256), 0, s,
                               reinterpret_cast<uint16_t *>(w.coef2), 2 * batch * m);
            rc = check_launch("zero_words_kernel");
            if (rc) return rc;
            return grad_product_f32(Wf, true, x1f, true, batch, m, d, n, sign, w.coef2, x2f, g2, s);
        }
    }
    if constexpr (!kBf16 && kCosO<MODE>) {
        // fp32 cosine from the forward's output: weights, coef1 and the column partials inside
        // the grad_x1 product; coef2 from the partials; grad_x2 on the tile kernel
        const float *gf = reinterpret_cast<const float *>(g), *of = reinterpret_cast<const float *>(res);
        const float *x1f = reinterpret_cast<const float *>(x1), *x2f = reinterpret_cast<const float *>(x2);
        float *Wf = reinterpret_cast<float *>(W);
        float *g1 = reinterpret_cast<float *>(gx1), *g2 = reinterpret_cast<float *>(gx2);
        if (fused_fits(gf, of, x1f, x2f, Wf, g1, g2, n, m, d) && aligned16(n2) && fused_grid_fills(batch, n, m, d)) {
            const int64_t tiles_n = cdiv(n, tile::kT), tiles_c = cdiv(d, kFCols), total = tiles_n * tiles_c * batch;
            // the column reciprocals and the norm-range flag, then both instances (one returns)
            hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<uint16_t *>(w.slow), 2);
            hipLaunchKernelGGL(cos_norm_prep_kernel, dim3((unsigned)cdiv(batch * (n + m), 256)), dim3(256), 0, s, n1,
                               batch * n, n2, batch * m, w.rn2, w.slow);
            hipLaunchKernelGGL((fused_grad1_kernel<MODE, true>), dim3((unsigned)total), dim3(256), 0, s, gf, of, x2f,
                               x1f, n, m, d, Wf, g1, tiles_n, tiles_c, total, kp, 1.0f, n1, n2, w.colpart, w.rn2,
                               static_cast<const uint32_t *>(w.slow));
            hipLaunchKernelGGL((fused_grad1_kernel<MODE, false>), dim3((unsigned)total), dim3(256), 0, s, gf, of, x2f,
                               x1f, n, m, d, Wf, g1, tiles_n, tiles_c, total, kp, 1.0f, n1, n2, w.colpart, w.rn2,
                               static_cast<const uint32_t *>(w.slow));
            rc = check_launch("fused_grad1_kernel");
            if (rc) return rc;
            hipLaunchKernelGGL(reduce_parts_kernel, dim3((unsigned)cdiv(batch * m, 256)), dim3(256), 0, s,
                               w.colpart, 4 * tiles_n, m, batch, n2, w.coef2);
            rc = check_launch("reduce_parts_kernel");
            if (rc) return rc;
            return grad_product_f32(Wf, true, x1f, true, batch, m, d, n, 1.0f, w.coef2, x2f, g2, s);
        }
    }
    if constexpr (kBf16 && (MODE == kEuclid || MODE == kSqEuclid || MODE == kSigmoid || MODE == kPoly)) {
        // bf16: the same fusion; S (polynomial) stays the fp32 recompute
        if constexpr (MODE != kPoly) {
            const uint16_t *gb = reinterpret_cast<const uint16_t *>(g), *rb = reinterpret_cast<const uint16_t *>(res);
            const uint16_t *x1b = reinterpret_cast<const uint16_t *>(x1), *x2b = reinterpret_cast<const uint16_t *>(x2);
            uint16_t *Wb = reinterpret_cast<uint16_t *>(W);
            uint16_t *g1 = reinterpret_cast<uint16_t *>(gx1), *g2 = reinterpret_cast<uint16_t *>(gx2);
            if (fused_bf16_fits(gb, MODE == kSqEuclid ? gb : rb, x1b, x2b, Wb, g1, g2, n, m, d) &&
                fused_grid_fills(batch, n, m, d)) {
                const float sign = MODE == kSigmoid ? 1.0f : -1.0f;
                const int64_t tiles_n = cdiv(n, tile::kT), tiles_c = cdiv(d, kFCols), total = tiles_n * tiles_c * batch;
                hipLaunchKernelGGL((fused_grad1_bf16_kernel<MODE>), dim3((unsigned)total), dim3(256), 0, s, gb, rb,
                                   x2b, x1b, n, m, d, Wb, g1, tiles_n, tiles_c, total, kp, sign,
                                   static_cast<const float *>(nullptr), static_cast<const float *>(nullptr),
                                   static_cast<const float *>(nullptr), static_cast<const uint32_t *>(nullptr));
                rc = check_launch("fused_grad1_bf16_kernel");
                if (rc) return rc;
                if constexpr (MODE == kEuclid || MODE == kSqEuclid)
                    return grad_product_bf16(Wb, true, x1b, true, batch, m, d, n, sign, nullptr, x2b, g2, s);
                hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)cdiv(2 * batch * m, 256)), dim3(256), 0, s,
                                   reinterpret_cast<uint16_t *>(w.coef2), 2 * batch * m);
                rc = check_launch("zero_words_kernel");
                if (rc) return rc;
                return grad_product_bf16(Wb, true, x1b, true, batch, m, d, n, sign, w.coef2, x2b, g2, s);
            }
        }
    }
    if constexpr (kBf16 && kCosO<MODE>) {
        // bf16 cosine from the forward's output: the fp32 path's fusion on the bf16 kernel
        const uint16_t *gb = reinterpret_cast<const uint16_t *>(g), *ob = reinterpret_cast<const uint16_t *>(res);
        const uint16_t *x1b = reinterpret_cast<const uint16_t *>(x1), *x2b = reinterpret_cast<const uint16_t *>(x2);
        uint16_t *Wb = reinterpret_cast<uint16_t *>(W);
        uint16_t *g1 = reinterpret_cast<uint16_t *>(gx1), *g2 = reinterpret_cast<uint16_t *>(gx2);
        if (fused_bf16_fits(gb, ob, x1b, x2b, Wb, g1, g2, n, m, d) && fused_grid_fills(batch, n, m, d)) {
            const int64_t tiles_n = cdiv(n, tile::kT), tiles_c = cdiv(d, kFCols), total = tiles_n * tiles_c * batch;
            hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<uint16_t *>(w.slow), 2);
            hipLaunchKernelGGL(cos_norm_prep_kernel, dim3((unsigned)cdiv(batch * (n + m), 256)), dim3(256), 0, s, n1,
                               batch * n, n2, batch * m, w.rn2, w.slow);
            hipLaunchKernelGGL((fused_grad1_bf16_kernel<MODE, true>), dim3((unsigned)total), dim3(256), 0, s, gb, ob,
                               x2b, x1b, n, m, d, Wb, g1, tiles_n, tiles_c, total, kp, 1.0f, n1, n2, w.rn2,
                               static_cast<const uint32_t *>(w.slow));
            hipLaunchKernelGGL((fused_grad1_bf16_kernel<MODE, false>), dim3((unsigned)total), dim3(256), 0, s, gb,
                               ob, x2b, x1b, n, m, d, Wb, g1, tiles_n, tiles_c, total, kp, 1.0f, n1, n2, w.rn2,
                               static_cast<const uint32_t *>(w.slow));
            int rc = check_launch("fused_grad1_bf16_kernel");
            if (rc) return rc;
            // P = W^T x1 into gx2 (zero coefficients), then the projection finish
            hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)cdiv(2 * batch * m, 256)), dim3(256), 0, s,
                               reinterpret_cast<uint16_t *>(w.coef2), 2 * batch * m);
            rc = grad_product_bf16(Wb, true, x1b, true, batch, m, d, n, 1.0f, w.coef2, x2b, g2, s);
            if (rc) return rc;
            hipLaunchKernelGGL(cos_proj_finish_kernel, dim3((unsigned)cdiv(batch * m, 4)), dim3(256), 0, s, g2, x2b,
                               n2, batch * m, d);
            return check_launch("cos_proj_finish_kernel");
        }
    }
    int64_t ti = cdiv(n, kPWRows);
    int64_t tj = cdiv(m, kPWCols);
    bool vec_pass = false;
    if constexpr (!kBf16) {
        const void *av = (MODE == kEuclid || MODE == kSigmoid || kCosO<MODE>) ? static_cast<const void *>(res) : w.S;
        vec_pass = m % 4 == 0 && aligned16(g) && aligned16(av) && aligned16(W) && aligned16(w.colpart) &&
                   (n2 == nullptr || aligned16(n2));
    }
    if (cos_fused) {
        if constexpr (kCosMode) {
            ti = 2 * cdiv(n, tile::kT);
            tj = 2 * cdiv(m, tile::kT);
            const int64_t tiles_n = cdiv(n, tile::kT), tiles_m = cdiv(m, tile::kT), total = tiles_n * tiles_m * batch;
            hipLaunchKernelGGL((cos_weights_tile_kernel<T, MODE>), dim3((unsigned)total), dim3(tile::kThreads), 0, s,
                               x1, x2, n, m, d, n1, n2, g, W, w.rowpart, w.colpart, tiles_n, tiles_m, total);
            rc = check_launch("cos_weights_tile_kernel");
        }
    } else if (vec_pass) {
        hipLaunchKernelGGL((pair_weights_vec_kernel<MODE>), dim3((unsigned)tj, (unsigned)ti, (unsigned)batch),
                           dim3(256), 0, s, reinterpret_cast<const float *>(g), reinterpret_cast<const float *>(res),
                           n1, n2, n, m, w.S, w.rowpart, w.colpart, ti, tj, reinterpret_cast<float *>(W), kp);
        rc = check_launch("pair_weights_vec_kernel");
    } else {
        hipLaunchKernelGGL((pair_weights_kernel<T, MODE>), dim3((unsigned)tj, (unsigned)ti, (unsigned)batch),
                           dim3(256), 0, s, g, res, n1, n2, n, m, w.S, w.rowpart, w.colpart, ti, tj, W,
                           kBf16 && !bf16_kmajor ? WT : nullptr, kp);
        rc = check_launch("pair_weights_kernel");
    }
    if (rc) return rc;
    const bool cosine = kCosAny<MODE>;
    const float *div1 = cosine ? n1 : nullptr;
    const float *div2 = cosine ? n2 : nullptr;
    hipLaunchKernelGGL(reduce_parts_kernel, dim3((unsigned)cdiv(batch * n, 256)), dim3(256), 0, s,
                       w.rowpart, tj, n, batch, div1, w.coef1);
    hipLaunchKernelGGL(reduce_parts_kernel, dim3((unsigned)cdiv(batch * m, 256)), dim3(256), 0, s,
                       w.colpart, ti, m, batch, div2, w.coef2);
    rc = check_launch("reduce_parts_kernel");
    if (rc) return rc;
    // kernel functions: W carries the whole gradient (rowpart / colpart, hence coef, are 0)
    const float sign = (cosine || MODE == kPoly || MODE == kSigmoid || MODE == kDot) ? 1.0f : -1.0f;
    if constexpr (kBf16) {
        if (bf16_kmajor) {
            rc = grad_product_bf16(W, false, x2, true, batch, n, d, m, sign, w.coef1, x1, gx1, s);
            if (rc) return rc;
            return grad_product_bf16(W, true, x1, true, batch, m, d, n, sign, w.coef2, x2, gx2, s);
        }
        // both products as A . B^T with k-contiguous operands on the bf16 matrix cores:
        // gx1 = sign * W . (x2^T)^T + coef1 * x1, gx2 = sign * W^T . (x1^T)^T + coef2 * x2
        hipLaunchKernelGGL((transpose_kernel<T>), dim3((unsigned)cdiv(d, 64), (unsigned)cdiv(n, 64), (unsigned)batch),
                           dim3(256), 0, s, x1, n, d, x1t);
        hipLaunchKernelGGL((transpose_kernel<T>), dim3((unsigned)cdiv(d, 64), (unsigned)cdiv(m, 64), (unsigned)batch),
                           dim3(256), 0, s, x2, m, d, x2t);
        rc = check_launch("transpose_kernel");
        if (rc) return rc;
        rc = inner_grad_gemm(W, x2t, dtype, batch, n, d, m, sign, w.coef1, x1, gx1, s);
        if (rc) return rc;
        return inner_grad_gemm(WT, x1t, dtype, batch, m, d, n, sign, w.coef2, x2, gx2, s);
    } else {
        // fp32: the k-major GEMM with split-K fills the GPU better for narrow outputs (d
        // columns) than the NT kernel did (C2 euclidean fwd+bwd 9.1 vs 10.6 ms)
        return products_f32(reinterpret_cast<const float *>(W), reinterpret_cast<const float *>(x1),
                            reinterpret_cast<const float *>(x2), batch, n, m, d, sign, w,
                            reinterpret_cast<float *>(gx1), reinterpret_cast<float *>(gx2), s);
    }
}

// Zero the gradient of the non-empty side when the other has no rows (no pairs, so nothing
// to sum); the empty side's buffer may be a null pointer.  Both dtypes are whole 16-bit words.

int zero_other_side(int dtype, int64_t batch, int64_t n, int64_t m, int64_t d, void *grad_x1,
                    void *grad_x2, hipStream_t s) {
    void *g = n ? grad_x1 : grad_x2;
    const int64_t len = batch * (n ? n : m) * d * (dtype == TPW_F32 ? 2 : 1);
    TPW_REQUIRE(g, "null pointer");
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)cdiv(len, 256)), dim3(256), 0, s,
                       static_cast<uint16_t *>(g), len);
    return check_launch("zero_words_kernel");
}

}  // namespace
}  // namespace tpw

using namespace tpw;

extern "C" size_t tpw_inner_backward_workspace_size(int64_t batch, int64_t n, int64_t m,
                                                    int64_t d) {
    return workspace_bytes(batch, n, m, d);
}

extern "C" int tpw_euclidean_backward(const void *grad, const void *x1, const void *x2,
                                      const void *res, int dtype, int64_t batch, int64_t n,
                                      int64_t m, int64_t d, void *grad_x1, void *grad_x2,
                                      void *workspace, void *stream) {
    TPW_REQUIRE(dtype == TPW_F32 || dtype == TPW_BF16, "unsupported dtype %d", dtype);
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    if (batch == 0 || d == 0 || (n == 0 && m == 0)) return TPW_OK;
    if (n == 0 || m == 0)
        return zero_other_side(dtype, batch, n, m, d, grad_x1, grad_x2, as_stream(stream));
    TPW_REQUIRE(grad && x1 && x2 && res && grad_x1 && grad_x2 && workspace, "null pointer");
    TPW_REQUIRE(cdiv(n, kPWRows) <= kMaxGridYZ && cdiv(m, kGT) <= kMaxGridYZ &&
                    cdiv(n, kGT) <= kMaxGridYZ && batch <= kMaxGridYZ,
                "sizes exceed the launch grid");
    hipStream_t s = as_stream(stream);
    if (dtype == TPW_F32)
        return run_backward<float, kEuclid>(
            static_cast<const float *>(grad), static_cast<const float *>(x1),
            static_cast<const float *>(x2), static_cast<const float *>(res), nullptr, nullptr,
            dtype, batch, n, m, d, static_cast<float *>(grad_x1), static_cast<float *>(grad_x2),
            workspace, s);
    return run_backward<uint16_t, kEuclid>(
        static_cast<const uint16_t *>(grad), static_cast<const uint16_t *>(x1),
        static_cast<const uint16_t *>(x2), static_cast<const uint16_t *>(res), nullptr, nullptr,
        dtype, batch, n, m, d, static_cast<uint16_t *>(grad_x1), static_cast<uint16_t *>(grad_x2),
        workspace, s);
}

extern "C" int tpw_cosine_backward(const void *grad, const void *x1, const void *x2,
                                   const float *norms1, const float *norms2, const void *out, int dtype,
                                   int64_t batch, int64_t n, int64_t m, int64_t d, int similarity,
                                   void *grad_x1, void *grad_x2, void *workspace, void *stream) {
    TPW_REQUIRE(dtype == TPW_F32 || dtype == TPW_BF16, "unsupported dtype %d", dtype);
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    if (batch == 0 || d == 0 || (n == 0 && m == 0)) return TPW_OK;
    if (n == 0 || m == 0)
        return zero_other_side(dtype, batch, n, m, d, grad_x1, grad_x2, as_stream(stream));
    TPW_REQUIRE(grad && x1 && x2 && norms1 && norms2 && grad_x1 && grad_x2 && workspace,
                "null pointer");
    TPW_REQUIRE(cdiv(n, kPWRows) <= kMaxGridYZ && cdiv(m, kGT) <= kMaxGridYZ &&
                    cdiv(n, kGT) <= kMaxGridYZ && batch <= kMaxGridYZ,
                "sizes exceed the launch grid");
    hipStream_t s = as_stream(stream);
    // with the forward's output, the weights come from it (no recomputed S)
    if (dtype == TPW_F32) {
        auto run = out ? (similarity == 2 ? run_backward<float, kCosCorrO>
                          : similarity    ? run_backward<float, kCosSimO>
                                          : run_backward<float, kCosDistO>)
                       : (similarity == 2 ? run_backward<float, kCosCorr>
                          : similarity    ? run_backward<float, kCosSim>
                                          : run_backward<float, kCosDist>);
        return run(static_cast<const float *>(grad), static_cast<const float *>(x1),
                   static_cast<const float *>(x2), static_cast<const float *>(out), norms1, norms2, dtype, batch,
                   n, m, d, static_cast<float *>(grad_x1), static_cast<float *>(grad_x2), workspace, s,
                   KerParams{});
    }
    auto run = out ? (similarity == 2 ? run_backward<uint16_t, kCosCorrO>
                      : similarity    ? run_backward<uint16_t, kCosSimO>
                                      : run_backward<uint16_t, kCosDistO>)
                   : (similarity == 2 ? run_backward<uint16_t, kCosCorr>
                      : similarity    ? run_backward<uint16_t, kCosSim>
                                      : run_backward<uint16_t, kCosDist>);
    return run(static_cast<const uint16_t *>(grad), static_cast<const uint16_t *>(x1),
               static_cast<const uint16_t *>(x2), static_cast<const uint16_t *>(out), norms1, norms2, dtype, batch,
               n, m, d, static_cast<uint16_t *>(grad_x1), static_cast<uint16_t *>(grad_x2), workspace, s,
               KerParams{});
}

extern "C" int tpw_sqeuclidean_backward(const void *grad, const void *x1, const void *x2,
                                        int dtype, int64_t batch, int64_t n, int64_t m, int64_t d,
                                        void *grad_x1, void *grad_x2, void *workspace,
                                        void *stream) {
    TPW_REQUIRE(dtype == TPW_F32 || dtype == TPW_BF16, "unsupported dtype %d", dtype);
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    if (batch == 0 || d == 0 || (n == 0 && m == 0)) return TPW_OK;
    if (n == 0 || m == 0)
        return zero_other_side(dtype, batch, n, m, d, grad_x1, grad_x2, as_stream(stream));
    TPW_REQUIRE(grad && x1 && x2 && grad_x1 && grad_x2 && workspace, "null pointer");
    TPW_REQUIRE(cdiv(n, kPWRows) <= kMaxGridYZ && cdiv(m, kGT) <= kMaxGridYZ &&
                    cdiv(n, kGT) <= kMaxGridYZ && batch <= kMaxGridYZ,
                "sizes exceed the launch grid");
    hipStream_t s = as_stream(stream);
    if (dtype == TPW_F32)
        return run_backward<float, kSqEuclid>(
            static_cast<const float *>(grad), static_cast<const float *>(x1),
            static_cast<const float *>(x2), nullptr, nullptr, nullptr, dtype, batch, n, m, d,
            static_cast<float *>(grad_x1), static_cast<float *>(grad_x2), workspace, s);
    return run_backward<uint16_t, kSqEuclid>(
        static_cast<const uint16_t *>(grad), static_cast<const uint16_t *>(x1),
        static_cast<const uint16_t *>(x2), nullptr, nullptr, nullptr, dtype, batch, n, m, d,
        static_cast<uint16_t *>(grad_x1), static_cast<uint16_t *>(grad_x2), workspace, s);
}

extern "C" int tpw_linear_backward(const void *grad, const void *x1, const void *x2,
                                        int dtype, int64_t batch, int64_t n, int64_t m, int64_t d,
                                        void *grad_x1, void *grad_x2, void *workspace,
                                        void *stream) {
    TPW_REQUIRE(dtype == TPW_F32 || dtype == TPW_BF16, "unsupported dtype %d", dtype);
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    if (batch == 0 || d == 0 || (n == 0 && m == 0)) return TPW_OK;
    if (n == 0 || m == 0)
        return zero_other_side(dtype, batch, n, m, d, grad_x1, grad_x2, as_stream(stream));
    TPW_REQUIRE(grad && x1 && x2 && grad_x1 && grad_x2 && workspace, "null pointer");
    TPW_REQUIRE(cdiv(n, kPWRows) <= kMaxGridYZ && cdiv(m, kGT) <= kMaxGridYZ &&
                    cdiv(n, kGT) <= kMaxGridYZ && batch <= kMaxGridYZ,
                "sizes exceed the launch grid");
    hipStream_t s = as_stream(stream);
    if (dtype == TPW_F32)
        return run_backward<float, kDot>(
            static_cast<const float *>(grad), static_cast<const float *>(x1),
            static_cast<const float *>(x2), nullptr, nullptr, nullptr, dtype, batch, n, m, d,
            static_cast<float *>(grad_x1), static_cast<float *>(grad_x2), workspace, s);
    return run_backward<uint16_t, kDot>(
        static_cast<const uint16_t *>(grad), static_cast<const uint16_t *>(x1),
        static_cast<const uint16_t *>(x2), nullptr, nullptr, nullptr, dtype, batch, n, m, d,
        static_cast<uint16_t *>(grad_x1), static_cast<uint16_t *>(grad_x2), workspace, s);
}

extern "C" int tpw_pairwise_kernel_backward(const void *grad, const void *x1, const void *x2,
                                            const void *out, int dtype, int64_t batch, int64_t n,
                                            int64_t m, int64_t d, int kind, float gamma,
                                            float coef0, int degree, void *grad_x1, void *grad_x2,
                                            void *workspace, void *stream) {
    TPW_REQUIRE(dtype == TPW_F32 || dtype == TPW_BF16, "unsupported dtype %d", dtype);
    TPW_REQUIRE(kind == TPW_KER_POLYNOMIAL || kind == TPW_KER_SIGMOID, "unknown kernel %d", kind);
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    if (batch == 0 || d == 0 || (n == 0 && m == 0)) return TPW_OK;
    if (n == 0 || m == 0)
        return zero_other_side(dtype, batch, n, m, d, grad_x1, grad_x2, as_stream(stream));
    TPW_REQUIRE(grad && x1 && x2 && grad_x1 && grad_x2 && workspace, "null pointer");
    TPW_REQUIRE(kind == TPW_KER_POLYNOMIAL || out, "the sigmoid backward needs the forward output");
    TPW_REQUIRE(cdiv(n, kPWRows) <= kMaxGridYZ && cdiv(m, kGT) <= kMaxGridYZ &&
                    cdiv(n, kGT) <= kMaxGridYZ && batch <= kMaxGridYZ,
                "sizes exceed the launch grid");
    hipStream_t s = as_stream(stream);
    KerParams kp;
    kp.gamma = gamma;
    kp.coef0 = coef0;
    kp.degree = degree;
    if (dtype == TPW_F32) {
        auto run = kind == TPW_KER_POLYNOMIAL ? run_backward<float, kPoly> : run_backward<float, kSigmoid>;
        return run(static_cast<const float *>(grad), static_cast<const float *>(x1),
                   static_cast<const float *>(x2), static_cast<const float *>(out), nullptr, nullptr,
                   dtype, batch, n, m, d, static_cast<float *>(grad_x1), static_cast<float *>(grad_x2),
                   workspace, s, kp);
    }
    auto run = kind == TPW_KER_POLYNOMIAL ? run_backward<uint16_t, kPoly> : run_backward<uint16_t, kSigmoid>;
    return run(static_cast<const uint16_t *>(grad), static_cast<const uint16_t *>(x1),
               static_cast<const uint16_t *>(x2), static_cast<const uint16_t *>(out), nullptr, nullptr,
               dtype, batch, n, m, d, static_cast<uint16_t *>(grad_x1), static_cast<uint16_t *>(grad_x2),
               workspace, s, kp);
}
