// Non-GEMM pairwise reductions on the VALU: Minkowski distances for p = 0, 1, 2, 3, inf and
// general p, and their gradient (at::_cdist_forward / at::_cdist_backward semantics), plus
// the reference's own kernels of the same shape: _ppminkowski (sum of |d|^p, no root),
// _wminkowski (per-feature weights, root), _canberra and _braycurtis.
//
// Forward: 256-thread blocks own a 128 x 128 output tile; thread (ty, tx) owns rows
// 8 ty + r (r < 8) and columns 64 h + 4 tx + c (h < 2, c < 4).  Both operand panels are
// staged in LDS feature-major ([k][row], 4-float pad), so one k step costs a thread four
// 16-byte LDS reads (8 x1 values broadcast over tx, 8 x2 values) for 64 pair-features.
// Per pair-feature the VALU does a subtract and an abs-modified accumulate (p = 1: add,
// p = inf: max), three ops for p = 3 (d * |d| fused into the accumulate), one exp2/log2
// pair more for general p.  Stores are non-temporal float4 rows (256 B per 16 lanes).
// Bray-Curtis runs the p = 1 kernel for sum |a - b| and a second pass for sum |a + b| that
// divides the stored numerator (two accumulators per output would halve the register
// tile; the VALU work is the same).
//
// Backward (grad of x1; x2 by the transposed call): out[i,k] = sum_j F(x1[i,k], x2[j,k],
// per-pair weights of (i, j)).  A block owns 128 rows x 64 features with its x1 values held
// in registers, streams 32 j at a time (x2 panel [j][k] and up to two per-pair weights
// computed while staging into LDS), thread block 8 rows x 4 features.  The j range is
// split over several blocks when the row/feature grid alone would not fill the GPU; the
// per-split partial sums are then added in split order by a second kernel, so the result
// is deterministic (the reference accumulates with atomics on its GPU path).
#include <math.h>

#include <type_traits>

#include "common.hpp"

namespace tpw {
namespace {

enum PKind { kP0 = 0, kP1, kP2, kP3, kPInf, kPLt2, kPGen, kPNInf };

// What a forward launch computes per (i, j) (PK picks |d|^p for the first three).
enum Mode {
    kRoot = 0,  // (sum_k |d|^p)^(1/p)            at::_cdist_forward
    kSum,       // sum_k |d|^p                     _ppminkowski (cpu/ppminkowski_kernel.cpp:13-29)
    kWeighted,  // (sum_k w_k |d|^p)^(1/p)         _wminkowski (cpu/wminkowski_kernel.cpp:13-60)
    kCanberra,  // sum_k |d| / (|a| + |b|), terms with |a| + |b| == 0 skipped (canberra_kernel.cpp:13-30)
    kBrayDen,   // out = out / sum_k |a + b|, out holding sum_k |a - b| (braycurtis_kernel.cpp:13-29)
    kPlusSum,   // sum_k |a + b| (the Bray-Curtis denominator, for the backward)
    kChi2,      // -sum_k (a - b)^2 / (a + b), 0 where a + b == 0 (additive_chi2_kernel.cpp:13-30)
    kJS,        // sum_k rel_entr(a, m) + rel_entr(b, m), m = (a + b) / 2, divided by p
                // (2, or 2 ln base; sqjensenshannon_kernel.cpp:13-45,74)
};

// rel_entr of cpu/rel_entr.h: NaN stays NaN; x log(x / y) for x, y > 0; 0 for x == 0 and
// y >= 0; +inf otherwise.
__device__ __forceinline__ float rel_entr(float x, float y) {
    if (x != x) return x;
    if (x > 0.0f && y > 0.0f) return x * logf(x / y);
    if (x == 0.0f && y >= 0.0f) return 0.0f;
    return INFINITY;
}

constexpr int kThreads = 256;
constexpr int kTile = 128;
constexpr int kBK = 32;
constexpr int kPad = 4;

template <int PK>
__device__ __forceinline__ float lp_step(float acc, float a, float b, float p) {
    const float d = a - b;
    if constexpr (PK == kP1) return acc + fabsf(d);
    else if constexpr (PK == kPInf) return fmaxf(acc, fabsf(d));
    else if constexpr (PK == kPNInf) return fminf(acc, fabsf(d));
    else if constexpr (PK == kP2) return fmaf(d, d, acc);
    else if constexpr (PK == kP3) return fmaf(d * d, fabsf(d), acc);
    else if constexpr (PK == kP0) return acc + (d != 0.0f ? 1.0f : 0.0f);
    else return acc + exp2f(p * __log2f(fabsf(d)));
}

template <int MODE, int PK>
__device__ __forceinline__ float fam_step(float acc, float a, float b, float wk, float p) {
    if constexpr (MODE == kRoot || MODE == kSum) {
        return lp_step<PK>(acc, a, b, p);
    } else if constexpr (MODE == kWeighted) {
        const float d = a - b;
        if constexpr (PK == kP1) return fmaf(wk, fabsf(d), acc);
        else if constexpr (PK == kP2) return fmaf(d * d, wk, acc);
        else if constexpr (PK == kP3) return fmaf(d * d * fabsf(d), wk, acc);
        else if constexpr (PK == kPInf) return fmaxf(acc, fabsf(d) * wk);
        else if constexpr (PK == kPNInf) return fminf(acc, fabsf(d) * wk);
        else return fmaf(exp2f(p * __log2f(fabsf(d))), wk, acc);
    } else if constexpr (MODE == kCanberra) {
        const float den = fabsf(a) + fabsf(b);
        return den != 0.0f ? acc + __fdividef(fabsf(a - b), den) : acc;
    } else if constexpr (MODE == kChi2) {
        const float nom = a + b, d = a - b;
        return nom != 0.0f ? acc - __fdividef(d * d, nom) : acc;
    } else if constexpr (MODE == kJS) {
        const float mid = (a + b) * 0.5f;
        return acc + (rel_entr(a, mid) + rel_entr(b, mid));
    } else {  // kBrayDen, kPlusSum
        return acc + fabsf(a + b);
    }
}

template <int MODE, int PK>
__device__ __forceinline__ float fam_init() {
    if constexpr ((MODE == kWeighted && PK == kPInf)) return -INFINITY;
    else if constexpr (PK == kPNInf && (MODE == kWeighted || MODE == kSum)) return INFINITY;
    else return 0.0f;
}

// max (min) of acc, |d0|, |d1| in one instruction.  fmaxf compiles to v_max_f32 plus a
// canonicalising v_max_f32 of |d| in IEEE mode (3 ops per pair-feature); v_max3_f32 with
// abs input modifiers takes two features per instruction (1.5 ops).  NaN handling is the
// IEEE maxNum of fmaxf.
__device__ __forceinline__ float max3_abs(float acc, float d0, float d1) {
    float r;
    asm("v_max3_f32 %0, %1, |%2|, |%3|" : "=v"(r) : "v"(acc), "v"(d0), "v"(d1));
    return r;
}
__device__ __forceinline__ float min3_abs(float acc, float d0, float d1) {
    float r;
    asm("v_min3_f32 %0, %1, |%2|, |%3|" : "=v"(r) : "v"(acc), "v"(d0), "v"(d1));
    return r;
}

// Four independent accumulations of one row value a against four column values b[c], for the
// p = 1, 2 steps of lp_step, with the same operations and roundings: the four subtractions
// first, then the four accumulates, so that a wave's consecutive VALU instructions are
// independent.  The p = 3 and p = +-inf forward steps stay in the compiler's order: there the
// asm groups made every step wait for all of its LDS reads before the first subtraction, and
// the kernels ran 2-5 % slower than without them.
template <int PK>
__device__ __forceinline__ void lp_step4(float &c0, float &c1, float &c2, float &c3, float a, float b0, float b1,
                                         float b2, float b3) {
    float t0, t1, t2, t3;
    if constexpr (PK == kP1) {
        asm("v_sub_f32 %[t0], %[a], %[b0]\n\tv_sub_f32 %[t1], %[a], %[b1]\n\t"
            "v_sub_f32 %[t2], %[a], %[b2]\n\tv_sub_f32 %[t3], %[a], %[b3]\n\t"
            "v_add_f32_e64 %[c0], %[c0], |%[t0]|\n\tv_add_f32_e64 %[c1], %[c1], |%[t1]|\n\t"
            "v_add_f32_e64 %[c2], %[c2], |%[t2]|\n\tv_add_f32_e64 %[c3], %[c3], |%[t3]|"
            : [t0] "=&v"(t0), [t1] "=&v"(t1), [t2] "=&v"(t2), [t3] "=&v"(t3), [c0] "+v"(c0), [c1] "+v"(c1),
              [c2] "+v"(c2), [c3] "+v"(c3)
            : [a] "v"(a), [b0] "v"(b0), [b1] "v"(b1), [b2] "v"(b2), [b3] "v"(b3));
    } else {
        static_assert(PK == kP2, "lp_step4: p = 1, 2");
        asm("v_sub_f32 %[t0], %[a], %[b0]\n\tv_sub_f32 %[t1], %[a], %[b1]\n\t"
            "v_sub_f32 %[t2], %[a], %[b2]\n\tv_sub_f32 %[t3], %[a], %[b3]\n\t"
            "v_fmac_f32 %[c0], %[t0], %[t0]\n\tv_fmac_f32 %[c1], %[t1], %[t1]\n\t"
            "v_fmac_f32 %[c2], %[t2], %[t2]\n\tv_fmac_f32 %[c3], %[t3], %[t3]"
            : [t0] "=&v"(t0), [t1] "=&v"(t1), [t2] "=&v"(t2), [t3] "=&v"(t3), [c0] "+v"(c0), [c1] "+v"(c1),
              [c2] "+v"(c2), [c3] "+v"(c3)
            : [a] "v"(a), [b0] "v"(b0), [b1] "v"(b1), [b2] "v"(b2), [b3] "v"(b3));
    }
}

template <int PK>
__device__ __forceinline__ float lp_finish(float acc, float inv_p) {
    if constexpr (PK == kP2) return sqrt_rn(acc);
    else if constexpr (PK == kP3) return cbrtf(acc);
    else if constexpr (PK == kPGen || PK == kPLt2) return powf(acc, inv_p);
    else return acc;
}

template <int MODE, int PK>
__device__ __forceinline__ float fam_finish(float acc, float inv_p, float prev) {
    if constexpr (MODE == kRoot || MODE == kWeighted) return lp_finish<PK>(acc, inv_p);
    else if constexpr (MODE == kBrayDen) return prev / acc;
    else if constexpr (MODE == kJS) return acc / inv_p;  // inv_p carries the divisor here
    else return acc;
}

// w: per-feature weights [batch, d] (kWeighted only).  out: read first under kBrayDen.
// OM (output mode) 2, rownum: out = rownum[row] / value (IEEE divide), the signal-to-noise
// ratio's variance over the pair's squared distance.  OM 1, out16: the values are stored rounded
// to bf16 there instead of to out (the cdist of bf16 inputs, computed in fp32 and rounded once).
// Compile-time, so that OM 0 (the fp32 distances) keeps the code it had without them: as runtime
// branches they took the p = 1 kernel from 159 to 192 VGPRs (3 -> 2 waves per SIMD) and put the
// p = 3 kernel's epilogue on the stack (C3 forward 2.03 -> 2.46 ms, manhattan 1.21 -> 1.47 ms);
// the exp of OM 3 as a runtime branch held the p = 3 kernel at 218 VGPRs (2 waves per SIMD,
// 158 and 3 without it: 2.06 -> 1.97 ms).
// OM 3: out = exp(value * post), the kernel functions exp(-gamma * distance) of rbf_kernel /
// laplacian_kernel (one rounding per operation, as mul_ then exp_).
// Blocks per CU: p = +-inf holds two features' operands per step (32 VGPRs) and the compiler
// gives it 204 VGPRs at two blocks; held to three blocks it fits in 168 without scratch, and
// the third wave per SIMD overlaps one block's output stores with the others' steps
// (chebyshev 16384^2 x 128: 1.16 -> 1.06 ms).
template <int PK>
constexpr int kFwdBlocks = (PK == kPInf || PK == kPNInf) ? 3 : 2;

template <int MODE, int PK, bool VEC, int OM = 0>
__global__ __launch_bounds__(kThreads, kFwdBlocks<PK>) void lp_forward_kernel(
    const float *__restrict__ x1, const float *__restrict__ x2, const float *__restrict__ w,
    int64_t n, int64_t m, int64_t d, float p, float inv_p, float *__restrict__ out, float post,
    const float *__restrict__ rownum, uint16_t *__restrict__ out16) {
    __shared__ float As[kBK][kTile + kPad];
    __shared__ float Bs[kBK][kTile + kPad];
    __shared__ float Wk[MODE == kWeighted ? kBK : 1];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int64_t b = blockIdx.z;
    const int64_t row0 = (int64_t)blockIdx.y * kTile, col0 = (int64_t)blockIdx.x * kTile;
    const float *A = x1 + b * n * d;
    const float *B = x2 + b * m * d;

    float acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = fam_init<MODE, PK>();

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
        if constexpr (MODE == kWeighted) {
            if (tid < kBK) Wk[tid] = k0 + tid < d ? w[b * d + k0 + tid] : 0.0f;
        }
        __syncthreads();
        if (k0 + kBK < d) {
            load(A, n, row0, k0 + kBK, pa);
            load(B, m, col0, k0 + kBK, pb);
        }
        const int kmax = d - k0 < kBK ? (int)(d - k0) : kBK;
        int kbeg = 0;
        if constexpr ((PK == kPInf || PK == kPNInf) && (MODE == kRoot || MODE == kSum)) {
            for (; kbeg + 1 < kmax; kbeg += 2) {
                float av[2][8], bv[2][8];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const floatx4 a0 = *reinterpret_cast<const floatx4 *>(&As[kbeg + h][8 * ty]);
                    const floatx4 a1 = *reinterpret_cast<const floatx4 *>(&As[kbeg + h][8 * ty + 4]);
                    const floatx4 b0 = *reinterpret_cast<const floatx4 *>(&Bs[kbeg + h][4 * tx]);
                    const floatx4 b1 = *reinterpret_cast<const floatx4 *>(&Bs[kbeg + h][64 + 4 * tx]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        av[h][e] = a0[e], av[h][4 + e] = a1[e];
                        bv[h][e] = b0[e], bv[h][4 + e] = b1[e];
                    }
                }
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float d0 = av[0][i] - bv[0][j], d1 = av[1][i] - bv[1][j];
                        acc[i][j] = PK == kPInf ? max3_abs(acc[i][j], d0, d1) : min3_abs(acc[i][j], d0, d1);
                    }
            }
        }
        for (int k = kbeg; k < kmax; ++k) {
            const floatx4 a0 = *reinterpret_cast<const floatx4 *>(&As[k][8 * ty]);
            const floatx4 a1 = *reinterpret_cast<const floatx4 *>(&As[k][8 * ty + 4]);
            const floatx4 b0 = *reinterpret_cast<const floatx4 *>(&Bs[k][4 * tx]);
            const floatx4 b1 = *reinterpret_cast<const floatx4 *>(&Bs[k][64 + 4 * tx]);
            const float wk = MODE == kWeighted ? Wk[MODE == kWeighted ? k : 0] : 0.0f;
            const float av[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
            const float bv[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
            if constexpr ((MODE == kRoot || MODE == kSum) && (PK == kP1 || PK == kP2)) {
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int j = 0; j < 8; j += 4)
                        lp_step4<PK>(acc[i][j], acc[i][j + 1], acc[i][j + 2], acc[i][j + 3], av[i], bv[j], bv[j + 1],
                                     bv[j + 2], bv[j + 3]);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc[i][j] = fam_step<MODE, PK>(acc[i][j], av[i], bv[j], wk, p);
            }
        }
        __syncthreads();
    }

    const bool vec_store = VEC && (m % 4 == 0);
    if (!vec_store) {
        // rows of m % 4 != 0 floats (or unaligned outputs): the tile goes through the operand
        // LDS (free after the K loop's last barrier) in four 64 x 64 quarters, and each wave
        // writes whole 64-value row pieces, a dword per lane: 256 contiguous bytes per store
        // instead of 4-byte stores 16 bytes apart
        constexpr int kSt = 66;
        static_assert(64 * kSt <= kBK * (kTile + kPad), "the stage fits in As");
        float *st = &As[0][0];
        const int wave = tid >> 6, lane = tid & 63;
        for (int rh = 0; rh < 2; ++rh)
            for (int h = 0; h < 2; ++h) {
                if ((ty >> 3) == rh) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const int64_t row = row0 + 8 * ty + i;
                        const int64_t col = col0 + 64 * h + 4 * tx;
                        floatx4 prev = {0.0f, 0.0f, 0.0f, 0.0f};
                        if constexpr (MODE == kBrayDen) {
#pragma unroll
                            for (int c = 0; c < 4; ++c)
                                if (row < n && col + c < m) prev[c] = out[(b * n + row) * m + col + c];
                        }
                        floatx4 v;
#pragma unroll
                        for (int c = 0; c < 4; ++c) v[c] = fam_finish<MODE, PK>(acc[i][4 * h + c], inv_p, prev[c]);
                        if constexpr (OM == 3) {
#pragma clang fp contract(off)
#pragma unroll
                            for (int c = 0; c < 4; ++c) v[c] = expf(v[c] * post);
                        }
                        if constexpr (OM == 2) {
                            const float num = row < n ? rownum[b * n + row] : 0.0f;
#pragma unroll
                            for (int c = 0; c < 4; ++c) v[c] = __fdiv_rn(num, v[c]);
                        }
#pragma unroll
                        for (int c = 0; c < 4; ++c) st[(8 * ty + i - 64 * rh) * kSt + 4 * tx + c] = v[c];
                    }
                }
                __syncthreads();
                const int64_t col = col0 + 64 * h + lane;
#pragma unroll 4
                for (int r = 16 * wave; r < 16 * wave + 16; ++r) {
                    const int64_t row = row0 + 64 * rh + r;
                    if (row < n && col < m) {
                        if constexpr (OM == 1) out16[(b * n + row) * m + col] = f32_to_bf16_rne(st[r * kSt + lane]);
                        else store_nt(out + (b * n + row) * m + col, st[r * kSt + lane]);
                    }
                }
                __syncthreads();  // the quarter is written before the next one is staged
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int64_t row = row0 + 8 * ty + i;
        if (row >= n) continue;
        float *orow = out + (b * n + row) * m;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t col = col0 + 64 * h + 4 * tx;
            floatx4 prev = {0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (MODE == kBrayDen) {
                if (vec_store && col + 3 < m) {
                    prev = *reinterpret_cast<const floatx4 *>(orow + col);
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (col + c < m) prev[c] = orow[col + c];
                }
            }
            floatx4 v;
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = fam_finish<MODE, PK>(acc[i][4 * h + c], inv_p, prev[c]);
            if constexpr (OM == 3) {
#pragma clang fp contract(off)
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = expf(v[c] * post);
            }
            if constexpr (OM == 2) {
                const float num = rownum[b * n + row];
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = __fdiv_rn(num, v[c]);
            }
            if constexpr (OM == 1) {
                uint16_t *o16 = out16 + (b * n + row) * m;
                if (vec_store && col + 3 < m) {
                    const uint2 pk = make_uint2((uint32_t)f32_to_bf16_rne(v[0]) | ((uint32_t)f32_to_bf16_rne(v[1]) << 16),
                                                (uint32_t)f32_to_bf16_rne(v[2]) | ((uint32_t)f32_to_bf16_rne(v[3]) << 16));
                    __builtin_nontemporal_store(pk.x, reinterpret_cast<uint32_t *>(o16 + col));
                    __builtin_nontemporal_store(pk.y, reinterpret_cast<uint32_t *>(o16 + col) + 1);
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (col + c < m) o16[col + c] = f32_to_bf16_rne(v[c]);
                }
            } else if (vec_store && col + 3 < m) {
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
constexpr int kBFeat = 64;   // features (k) per block of the narrow kernel (FW = 64)
constexpr int kBFeatWide = 128;  // ... of the wide kernel (FW = 128: 8 x 8 per thread)
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

// sign(d) as ATen's (0 < d) - (d < 0): +-1, and 0 for +-0 and NaN.  copysign(1, d) is one
// v_bfi_b32 and "d < 0 or d > 0" one ordered not-equal compare (v_cmp_lg_f32), so the p = 1
// backward step is 5 VALU ops (sub, bfi, cmp, select, fma) instead of 6.
__device__ __forceinline__ float signf(float d) {
    const float s = __builtin_copysignf(1.0f, d);
    return ((d < 0.0f) | (d > 0.0f)) ? s : 0.0f;
}

// The p = 1 step sign(a - b) * w in three ops (sub, med3, fma) for operands pre-scaled by
// 2^75: for a, b in {0} u [2^-52, 2^52] the scaled values are exact and finite, a' - b' has
// the sign of a - b, and a nonzero difference of such values is a multiple of 2^-75 (at
// least 2^0 after scaling), so clamping it to [-1, 1] gives exactly sign(a - b).  Tiles or
// stages holding any other value (NaN and inf included) take the signf path.
constexpr float kSignScale = 0x1p75f, kSignUnscale = 0x1p-75f;
__device__ __forceinline__ bool sign_scalable(float x) {
    const float ax = fabsf(x);
    return ax == 0.0f || (ax >= 0x1p-52f && ax <= 0x1p52f);
}
__device__ __forceinline__ float sign_scaled(float d_scaled) {
    return __builtin_amdgcn_fmed3f(d_scaled, -1.0f, 1.0f);
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

// Four backward terms of one row, interleaved as lp_step4: acc[c] += w * T(a[c] - b[c]) with
// T(d) = d |d| (p = 3), d (p = 2) or, for operands pre-scaled by 2^75, med3(d, -1, 1) =
// sign(d) (the p = 1 fast path), with grad_term's operations and roundings (the product and
// the accumulate are one fma, as the compiler contracts grad_term's w * T + acc).
template <int PK, bool SIGN = false>
__device__ __forceinline__ void grad_step4(float &c0, float &c1, float &c2, float &c3, float a0, float a1, float a2,
                                           float a3, float b0, float b1, float b2, float b3, float w) {
    float t0, t1, t2, t3;
#define TPW_GRAD4(MID)                                                                                          \
    asm("v_sub_f32 %[t0], %[a0], %[b0]\n\tv_sub_f32 %[t1], %[a1], %[b1]\n\t"                                     \
        "v_sub_f32 %[t2], %[a2], %[b2]\n\tv_sub_f32 %[t3], %[a3], %[b3]\n\t" MID                                  \
        "v_fmac_f32 %[c0], %[w], %[t0]\n\tv_fmac_f32 %[c1], %[w], %[t1]\n\t"                                      \
        "v_fmac_f32 %[c2], %[w], %[t2]\n\tv_fmac_f32 %[c3], %[w], %[t3]"                                           \
        : [t0] "=&v"(t0), [t1] "=&v"(t1), [t2] "=&v"(t2), [t3] "=&v"(t3), [c0] "+v"(c0), [c1] "+v"(c1),            \
          [c2] "+v"(c2), [c3] "+v"(c3)                                                                            \
        : [a0] "v"(a0), [a1] "v"(a1), [a2] "v"(a2), [a3] "v"(a3), [b0] "v"(b0), [b1] "v"(b1), [b2] "v"(b2),       \
          [b3] "v"(b3), [w] "v"(w))
    if constexpr (SIGN) {
        static_assert(PK == kP1, "the sign fast path is p = 1");
        TPW_GRAD4("v_med3_f32 %[t0], %[t0], -1.0, 1.0\n\tv_med3_f32 %[t1], %[t1], -1.0, 1.0\n\t"
                  "v_med3_f32 %[t2], %[t2], -1.0, 1.0\n\tv_med3_f32 %[t3], %[t3], -1.0, 1.0\n\t");
    } else if constexpr (PK == kP3) {
        TPW_GRAD4("v_mul_f32_e64 %[t0], %[t0], |%[t0]|\n\tv_mul_f32_e64 %[t1], %[t1], |%[t1]|\n\t"
                  "v_mul_f32_e64 %[t2], %[t2], |%[t2]|\n\tv_mul_f32_e64 %[t3], %[t3], |%[t3]|\n\t");
    } else {
        static_assert(PK == kP2, "grad_step4: p = 2, 3 and the p = 1 sign fast path");
        TPW_GRAD4("");
    }
#undef TPW_GRAD4
}

// |d|^e for the general-p formulas (pow of the reference kernels).
__device__ __forceinline__ float abs_pow(float d, float e) { return exp2f(e * __log2f(fabsf(d))); }

// The two per-pair weights of the backward, from the upstream grad g and the per-pair
// arrays aux0 / aux1 of each mode:
//   kRoot     aux0 = dist           w1 = torch's _cdist_backward weight, w2 = dist
//   kSum      -                     w1 = g
//   kWeighted aux0 = out = S^(1/p)  w1 = g * S^(1/p - 1) = g * out^(1 - p)
//   kCanberra -                     w1 = g
//   kBrayDen  aux0 = out, aux1 = sum |a + b|:  w1 = g / ss, w2 = w1 * out (= g sd / ss^2)
template <int MODE, int PK>
__device__ __forceinline__ void pair_weights(float g, float a0, float a1, float p, float &w1,
                                             float &w2) {
    w2 = 0.0f;
    if constexpr (MODE == kRoot) {
        w1 = pair_weight<PK>(g, a0, p);
        w2 = a0;
    } else if constexpr (MODE == kWeighted) {
        if constexpr (PK == kP1) w1 = g;
        else if constexpr (PK == kP2) w1 = __fdiv_rn(g, a0);
        else if constexpr (PK == kP3) w1 = __fdiv_rn(g, a0 * a0);
        else w1 = g * powf(a0, 1.0f - p);
    } else if constexpr (MODE == kBrayDen) {
        w1 = __fdiv_rn(g, a1);
        w2 = w1 * a0;
    } else if constexpr (MODE == kJS) {
        w1 = g / p;  // the forward's divisor (sqjensenshannon_kernel.cpp:166)
    } else {
        w1 = g;
    }
}

// Per pair-feature contribution to grad of the first operand (a = own value, b = the other
// operand's), or, under WGRAD, to the weight gradient (before the sum over rows).  The
// formulas are those of the reference kernels: _ppminkowski (ppminkowski_kernel.cpp:125-160),
// _wminkowski (wminkowski_kernel.cpp:140-210), _canberra (canberra_kernel.cpp:85-125),
// _braycurtis (braycurtis_kernel.cpp:108-152).
template <int MODE, int PK, bool WGRAD>
__device__ __forceinline__ float fam_term(float a, float b, float w1, float w2, float wk, float p) {
    const float d = a - b;
    if constexpr (MODE == kRoot) {
        return grad_term<PK>(d, w1, w2, p);
    } else if constexpr (MODE == kSum) {
        if constexpr (PK == kP1) return signf(d) * w1;
        else if constexpr (PK == kP2) return 2.0f * d * w1;
        else if constexpr (PK == kP3) return 3.0f * d * fabsf(d) * w1;
        else return p * abs_pow(d, p - 1.0f) * signf(d) * w1;
    } else if constexpr (MODE == kWeighted && !WGRAD) {
        if constexpr (PK == kP1) return wk * signf(d) * w1;
        else if constexpr (PK == kP2) return wk * d * w1;
        else if constexpr (PK == kP3) return wk * d * fabsf(d) * w1;
        else return wk * abs_pow(d, p - 1.0f) * signf(d) * w1;
    } else if constexpr (MODE == kWeighted) {
        if constexpr (PK == kP1) return fabsf(d) * w1;
        else if constexpr (PK == kP2) return d * d * 0.5f * w1;
        else if constexpr (PK == kP3) return d * d * fabsf(d) * (1.0f / 3.0f) * w1;
        else return abs_pow(d, p) / p * w1;
    } else if constexpr (MODE == kCanberra) {
        const float nom = fabsf(a) + fabsf(b);
        return (signf(d) / nom - signf(a) * fabsf(d) / nom / nom) * w1;
    } else if constexpr (MODE == kChi2) {  // additive_chi2_kernel.cpp:90-125
        const float nom = a + b;
        if (nom == 0.0f) return 0.0f;
        const float q = __fdividef(d, nom);
        return (q * q - 2.0f * q) * w1;
    } else if constexpr (MODE == kJS) {  // sqjensenshannon_kernel.cpp:92-140
        const float sum = a + b, mid = sum * 0.5f;
        if (!(mid > 0.0f)) return 0.0f;
        float t = 0.0f;
        if (a > 0.0f) t += (b + sum * logf(a / mid)) / sum;
        if (b > 0.0f) t -= b / sum;
        return t * w1;
    } else {
        return w1 * signf(d) - w2 * signf(a + b);
    }
}

// Whether the narrow kernel's per-pair weights are computed once into an [n, m] array before
// the gradient kernels (they need a second per-pair operand and arithmetic beyond g itself)
// rather than while staging: staging then reads one array instead of two.  The wide kernel
// (FW = 128) forms them while staging, from g and the distance: at d <= 128 each pair's weight
// is then formed once per direction, and no [n, m] array is written and read back.
template <int MODE, int PK>
constexpr bool kPrecomputed = (MODE == kRoot && (PK == kP2 || PK == kP3 || PK == kPLt2 || PK == kPGen)) ||
                              (MODE == kWeighted && PK != kP1) || MODE == kBrayDen;
// The cases the wide kernel serves (above 64 features): the cdist backward at p = 2, 3 and
// p > 2 in general, and the p = 2 power sum (sqeuclidean, rbf_kernel).  p = inf (a second
// per-pair array) and 0 < p < 2 would spill its registers at this width; p = 1 takes it only
// through run_backward_p1_gated (the sign path alone, chosen by a range scan).
template <int MODE, int PK>
constexpr bool kWide = (MODE == kRoot && (PK == kP2 || PK == kP3 || PK == kPGen)) || (MODE == kSum && PK == kP2);

// VEC: every pointer is 16-byte aligned; four pairs per step with 16-byte accesses, and the
// len % 4 tail by the first threads.
template <int MODE, int PK, bool VEC>
__global__ void pair_weight_kernel(const float *__restrict__ g, const float *__restrict__ aux0,
                                   const float *aux1, int64_t len, float p, float *w1,
                                   float *__restrict__ w2) {
    const int64_t start = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t tail = 0;
    if constexpr (VEC) {
        const int64_t len4 = len >> 2;
        for (int64_t t = start; t < len4; t += stride) {
            const floatx4 gv = reinterpret_cast<const floatx4 *>(g)[t];
            const floatx4 a0 = reinterpret_cast<const floatx4 *>(aux0)[t];
            floatx4 a1 = {0.0f, 0.0f, 0.0f, 0.0f};
            if (aux1) a1 = reinterpret_cast<const floatx4 *>(aux1)[t];
            floatx4 r1, r2;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float u, v;
                pair_weights<MODE, PK>(gv[e], a0[e], a1[e], p, u, v);
                r1[e] = u;
                r2[e] = v;
            }
            reinterpret_cast<floatx4 *>(w1)[t] = r1;  // may alias aux1 (same elements)
            if (w2) reinterpret_cast<floatx4 *>(w2)[t] = r2;
        }
        tail = len4 << 2;
    }
    for (int64_t t = tail + start; t < len; t += stride) {
        float a, b;
        pair_weights<MODE, PK>(g[t], aux0[t], aux1 ? aux1[t] : 0.0f, p, a, b);
        w1[t] = a;  // may alias aux1 (same element)
        if (w2) w2[t] = b;
    }
}

// out[(split, b, i, k)] = sum over this split's j of fam_term.  G(b,i,j) and the per-pair
// arrays are read at [b*n*m + i*gs_i + j*gs_j] (gs = (m, 1) direct, (1, n) transposed).
// Under PRE, aux0 / aux1 hold the precomputed weights w1 / w2 and g is not read.  FW is the
// block's feature width: 64 (thread block 8 rows x 4 features) or 128 (8 x 8, the forward's
// ratio of LDS reads to VALU work: per j step two 16-byte reads of weights and two of x2 for 64
// pair-features).  EXPG: g is the upstream gradient of out = exp(-gamma * value) (rbf_kernel,
// laplacian_kernel) and eo that out, staged as a second per-pair array; the weight is formed
// from (g * eo) * es, es = -gamma, with the two roundings of the exp's and the scalar multiply's
// backward, so no N x M pass forms that gradient first.  gate: when not null, the block runs
// only if *gate == gate_run (two instances of one backward launched together, a flag set by an
// earlier launch choosing which one computes).
template <int MODE, int PK, bool TR, bool WGRAD, bool PRE, int FW = kBFeat, bool EXPG = false>
__global__ __launch_bounds__(kThreads, 2) void lp_backward_kernel(
    const float *__restrict__ g, const float *__restrict__ aux0, const float *__restrict__ aux1,
    const float *__restrict__ x1, const float *__restrict__ x2, const float *__restrict__ w,
    int64_t n, int64_t m, int64_t d, float p, int64_t j_per_split, int64_t batch,
    float *__restrict__ out, const float *__restrict__ eo, float es, const uint32_t *__restrict__ gate,
    uint32_t gate_run) {
    if (gate != nullptr && __builtin_amdgcn_readfirstlane(*gate) != gate_run) return;
    constexpr bool kTwo = (MODE == kRoot && PK == kPInf) || MODE == kBrayDen;
    constexpr int kCW = FW / 16;                // features per thread
    constexpr int kWavesPerRow = FW / 64;       // waves staging one x2 panel row
    constexpr int kPanelQ = kBJ * FW / kThreads;  // x2 panel values per thread and stage
    static_assert(FW == 64 || FW == 128, "feature width");
    __shared__ float Ws[kBJ][kBRows + kPad];
    __shared__ float Ds[kTwo ? kBJ : 1][kBRows + kPad];
    __shared__ float Xs[kBJ][FW + kPad];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    // thread (ty, tx) owns rows 8 ty + r and features 64 (c / 4) + 4 tx + c % 4 of the block
    auto feat_of = [](int t, int c) { return 64 * (c >> 2) + 4 * t + (c & 3); };
    const int64_t split = blockIdx.z / batch, b = blockIdx.z - split * batch;
    const int64_t i0 = (int64_t)blockIdx.y * kBRows, k0 = (int64_t)blockIdx.x * FW;
    const int64_t jbeg = split * j_per_split;
    const int64_t jend = jbeg + j_per_split < m ? jbeg + j_per_split : m;
    const float *G = g + b * n * m;
    const float *A0 = aux0 ? aux0 + b * n * m : nullptr;
    const float *A1 = aux1 ? aux1 + b * n * m : nullptr;
    const float *E = EXPG ? eo + b * n * m : nullptr;
    const float *X1 = x1 + b * n * d;
    const float *X2 = x2 + b * m * d;

    float xv[8][kCW], acc[8][kCW], wkv[kCW];
#pragma unroll
    for (int c = 0; c < kCW; ++c) {
        const int64_t k = k0 + feat_of(tx, c);
        wkv[c] = (MODE == kWeighted && k < d) ? w[b * d + k] : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const int64_t i = i0 + 8 * ty + r;
#pragma unroll
        for (int c = 0; c < kCW; ++c) {
            const int64_t k = k0 + feat_of(tx, c);
            xv[r][c] = (i < n && k < d) ? X1[i * d + k] : 0.0f;
            acc[r][c] = 0.0f;
        }
    }

    // Staging is software-pipelined: the per-pair values and the x2 panel of stage j0 + kBJ
    // are loaded into registers while stage j0 is computed from LDS, and go to LDS after
    // the stage's closing barrier.  Lane (tid) loads weight q of a stage at
    //   direct:     row ii = (tid >> 5) + 8 q, column jj = tid & 31   (coalesced along j)
    //   transposed: row ii = tid & 127,        column jj = (tid >> 7) + 2 q  (along i)
    // and panel value q at row jj = wave / kWavesPerRow + (4 / kWavesPerRow) q, feature
    // kk = 64 (wave % kWavesPerRow) + lane.  The loads are
    // raw buffer loads from wave-uniform bases: a lane past the end of an array reads 0, and
    // lanes past a row's end (j >= m, k >= d) or past jend read values that only reach
    // accumulators of rows, features or stage steps that are never stored or run, so no
    // load needs a bounds branch.
    constexpr bool kReadG = !PRE;                               // upstream grad
    constexpr bool kReadA0 = PRE || (MODE == kRoot && PK != kP1);  // weights, or the distance
    constexpr bool kReadA1 = PRE && kTwo;
    static_assert(!EXPG || (!PRE && !kTwo && !WGRAD), "the exp-scaled gradient: one weight from g");
    // the upstream gradient of one pair, exp-scaled under EXPG
    auto gval = [&](float gv, float ev) {
        if constexpr (EXPG) return __fmul_rn(__fmul_rn(gv, ev), es);
        else return gv;
    };
    // The wide kernel (V4) stages with 16-byte loads instead (its launch requires 16-byte
    // aligned arrays and n, m, d multiples of 4): lane (tid) loads float4 q of a stage at
    //   direct:     row ii = (tid >> 3) + 32 q, columns jj = 4 (tid & 7) + 0..3
    //   transposed: column jj = (tid >> 5) + 8 q, rows ii = 4 (tid & 31) + 0..3
    //   panel:      row jj = (tid >> 5) + 8 q, features kk = 4 (tid & 31) + 0..3
    // from one descriptor per array and stage with loop-invariant lane offsets.
    constexpr bool V4 = FW == kBFeatWide;
    static_assert(!V4 || !kTwo, "the wide kernel stages one per-pair array");
    // The p = 2 power sum on the wide kernel: its terms 2 d g accumulate as d g (the p = 2
    // step of the cdist backward, one fma each) and the sum is doubled once at the end.
    // Doubling is exact, so this differs from summing 2 d g only where a partial sum is
    // subnormal or overflows.
    constexpr bool kHalfSum = V4 && MODE == kSum && PK == kP2;
    // p = 1 on the wide kernel: only the pre-scaled sign path (sign_scaled), launched where every
    // value of x1 and x2 lies in the scalable range (sign_range_kernel); x1 is scaled once, the
    // x2 panel as it is staged.  The narrow kernel's per-tile test and its signf path would not
    // fit the wide kernel's registers.
    constexpr bool kSignOnly = V4 && PK == kP1 && (MODE == kRoot || MODE == kSum) && !WGRAD;
    float rg[kReadG ? 16 : 1], ra0[kReadA0 ? 16 : 1], ra1[kReadA1 ? 16 : 1], re[EXPG ? 16 : 1], rx[kPanelQ];
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lw_i = TR ? (tid & 127) : (tid >> 5), lw_j = TR ? (tid >> 7) : (tid & 31);
    const int lx_j = (tid >> 6) / kWavesPerRow, lx_k = 64 * ((tid >> 6) % kWavesPerRow) + lane;
    // byte offsets within a wave's rows (the launch keeps them below 2^32)
    const uint32_t lw_voff = TR ? (uint32_t)lane * 4u : (uint32_t)(((lane >> 5) * m + (lane & 31)) * 4);
    const uint32_t lx_voff = (uint32_t)lane * 4u;
    const int64_t nm = n * m, md = m * d;

    uint32_t v4_pair_off[V4 ? 4 : 1], v4_panel_off[V4 ? 4 : 1];
    if constexpr (V4) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v4_pair_off[q] = TR ? (uint32_t)((((tid >> 5) + 8 * q) * n + 4 * (tid & 31)) * 4)
                                : (uint32_t)((((tid >> 3) + 32 * q) * m + 4 * (tid & 7)) * 4);
            v4_panel_off[q] = (uint32_t)((((tid >> 5) + 8 * q) * d + 4 * (tid & 31)) * 4);
        }
    }
    // V4: the 16 per-pair values of one array for stage j0, as four float4
    auto load_pairs4 = [&](const float *arr, auto &r, int64_t j0) {
        const int64_t off = TR ? j0 * n + i0 : i0 * m + j0;
        const auto rs = buffer_over(arr + off, nm - off);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const floatx4 v = buffer_load4(rs, v4_pair_off[q]);
#pragma unroll
            for (int e = 0; e < 4; ++e) r[4 * q + e] = v[e];
        }
    };
    // the 16 per-pair values of one array for stage j0
    auto load_pairs = [&](const float *arr, auto &r, int64_t j0) {
        // one descriptor per step keeps the lane offset a single register (per-step lane
        // offsets would be loop-invariant and stay live across the stage loop)
        if constexpr (TR) {  // 64 rows of one column per wave and step
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int64_t off = (j0 + (wv >> 1) + 2 * q) * n + i0 + (wv & 1) * 64;
                r[q] = buffer_load(buffer_over(arr + off, nm - off), lw_voff);
            }
        } else {  // 32 columns of two rows per wave and step
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int64_t off = (i0 + 2 * wv + 8 * q) * m + j0;
                r[q] = buffer_load(buffer_over(arr + off, nm - off), lw_voff);
            }
        }
    };
    auto load = [&](int64_t j0) {
        if constexpr (V4) {
            if constexpr (kReadG) load_pairs4(G, rg, j0);
            if constexpr (kReadA0) load_pairs4(A0, ra0, j0);
            if constexpr (EXPG) load_pairs4(E, re, j0);
            const int64_t off = j0 * d + k0;
            const auto rs = buffer_over(X2 + off, md - off);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const floatx4 v = buffer_load4(rs, v4_panel_off[q]);
#pragma unroll
                for (int e = 0; e < 4; ++e) rx[4 * q + e] = v[e];
            }
            return;
        }
        if constexpr (kReadG) load_pairs(G, rg, j0);
        if constexpr (kReadA0) load_pairs(A0, ra0, j0);
        if constexpr (kReadA1) load_pairs(A1, ra1, j0);
        if constexpr (EXPG) load_pairs(E, re, j0);
#pragma unroll
        for (int q = 0; q < kPanelQ; ++q) {
            const int64_t off = (j0 + wv / kWavesPerRow + (4 / kWavesPerRow) * q) * d + k0 + 64 * (wv % kWavesPerRow);
            rx[q] = buffer_load(buffer_over(X2 + off, md - off), lx_voff);
        }
    };
    auto store = [&](int64_t j0) {
        if constexpr (V4) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float wq[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int ii = TR ? 4 * (tid & 31) + e : (tid >> 3) + 32 * q;
                    const int jj = TR ? (tid >> 5) + 8 * q : 4 * (tid & 7) + e;
                    float w1, w2;
                    pair_weights<MODE, PK>(kReadG ? gval(rg[4 * q + e], re[EXPG ? 4 * q + e : 0]) : 0.0f,
                                           kReadA0 ? ra0[4 * q + e] : 0.0f, 0.0f, p, w1, w2);
                    if constexpr (PRE) w1 = ra0[4 * q + e];
                    wq[e] = (i0 + ii < n && j0 + jj < jend) ? w1 : 0.0f;
                }
                if constexpr (TR) {
                    *reinterpret_cast<floatx4 *>(&Ws[(tid >> 5) + 8 * q][4 * (tid & 31)]) =
                        floatx4{wq[0], wq[1], wq[2], wq[3]};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) Ws[4 * (tid & 7) + e][(tid >> 3) + 32 * q] = wq[e];
                }
                const float sc = kSignOnly ? kSignScale : 1.0f;  // exact in the scalable range
                *reinterpret_cast<floatx4 *>(&Xs[(tid >> 5) + 8 * q][4 * (tid & 31)]) =
                    floatx4{rx[4 * q] * sc, rx[4 * q + 1] * sc, rx[4 * q + 2] * sc, rx[4 * q + 3] * sc};
            }
            return;
        }
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int ii = lw_i + (TR ? 0 : 8 * q), jj = lw_j + (TR ? 2 * q : 0);
            float w1 = 0.0f, w2 = 0.0f;
            if (i0 + ii < n && j0 + jj < jend) {
                if constexpr (PRE) {
                    w1 = ra0[q];
                    if constexpr (kTwo) w2 = ra1[q];
                } else {
                    pair_weights<MODE, PK>(gval(rg[q], re[EXPG ? q : 0]), kReadA0 ? ra0[q] : 0.0f, 0.0f, p, w1, w2);
                }
            }
            Ws[jj][ii] = w1;
            if constexpr (kTwo) Ds[jj][ii] = w2;
        }
#pragma unroll
        for (int q = 0; q < kPanelQ; ++q) Xs[lx_j + (4 / kWavesPerRow) * q][lx_k] = rx[q];
    };

    // x2 values of panel row jj at the thread's features feat_of(tcol, c) (one or two 16-byte
    // LDS reads, 16 bytes apart across the lanes)
    auto load_panel = [&](float (&x)[kCW], int jj, int tcol) {
#pragma unroll
        for (int h = 0; h < kCW / 4; ++h) {
            const floatx4 v = *reinterpret_cast<const floatx4 *>(&Xs[jj][64 * h + 4 * tcol]);
#pragma unroll
            for (int e = 0; e < 4; ++e) x[4 * h + e] = v[e];
        }
    };

    // p = 1 sign fast path (sign_scaled): flags[2] marks a tile of x1 outside the scalable
    // range, flags[s & 1] a panel of stage s.  A wave that finds such a value stores 1 (the
    // stores race benignly); thread 0 clears the next stage's word, which no thread reads
    // again before that stage's barrier.
    constexpr bool kSignFast = PK == kP1 && (MODE == kRoot || MODE == kSum) && !WGRAD;
    __shared__ int flags[3];
    bool tile_fast = false, xv_scaled = false;  // xv holds x1 * 2^75 while xv_scaled
    if constexpr (kSignOnly) {
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int c = 0; c < kCW; ++c) xv[r][c] *= kSignScale;
    } else if constexpr (kSignFast) {
        bool ok = true;
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int c = 0; c < kCW; ++c) ok = ok && sign_scalable(xv[r][c]);
        if (tid == 0) flags[0] = flags[2] = 0;
        __syncthreads();
        if (__any(!ok) && lane == 0) flags[2] = 1;
    }

    if (jbeg < jend) load(jbeg);
    int stage = 0;
    for (int64_t j0 = jbeg; j0 < jend; j0 += kBJ, ++stage) {
        store(j0);
        if constexpr (kSignFast && !kSignOnly) {
            bool ok = true;
#pragma unroll
            for (int q = 0; q < kPanelQ; ++q) ok = ok && sign_scalable(rx[q]);
            if (__any(!ok) && lane == 0) flags[stage & 1] = 1;
            if (tid == 0) flags[(stage + 1) & 1] = 0;
        }
        __syncthreads();
        if (j0 + kBJ < jend) load(j0 + kBJ);
        const int jmax = jend - j0 < kBJ ? (int)(jend - j0) : kBJ;
        if constexpr (kSignOnly) {
            for (int jj = 0; jj < jmax; ++jj) {
                const floatx4 w0 = *reinterpret_cast<const floatx4 *>(&Ws[jj][8 * ty]);
                const floatx4 w1 = *reinterpret_cast<const floatx4 *>(&Ws[jj][8 * ty + 4]);
                float x[kCW];
                load_panel(x, jj, tx);
                const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
#pragma unroll
                for (int r = 0; r < 8; ++r)
#pragma unroll
                    for (int c = 0; c < kCW; c += 4)
                        grad_step4<kP1, true>(acc[r][c], acc[r][c + 1], acc[r][c + 2], acc[r][c + 3], xv[r][c],
                                              xv[r][c + 1], xv[r][c + 2], xv[r][c + 3], x[c], x[c + 1], x[c + 2],
                                              x[c + 3], wv[r]);
            }
            __syncthreads();
            continue;
        } else if constexpr (kSignFast) {
            if (stage == 0) tile_fast = flags[2] == 0;
            const bool fast = tile_fast && flags[stage & 1] == 0;
            if (fast != xv_scaled) {  // exact both ways: the tile is in the scalable range
                const float f = fast ? kSignScale : kSignUnscale;
#pragma unroll
                for (int r = 0; r < 8; ++r)
#pragma unroll
                    for (int c = 0; c < kCW; ++c) xv[r][c] *= f;
                xv_scaled = fast;
            }
            if (fast) {
                for (int jj = 0; jj < jmax; ++jj) {
                    const floatx4 w0 = *reinterpret_cast<const floatx4 *>(&Ws[jj][8 * ty]);
                    const floatx4 w1 = *reinterpret_cast<const floatx4 *>(&Ws[jj][8 * ty + 4]);
                    float x[kCW];
                    load_panel(x, jj, tx);
                    const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
                    float xs[kCW];
#pragma unroll
                    for (int c = 0; c < kCW; ++c) xs[c] = x[c] * kSignScale;
#pragma unroll
                    for (int r = 0; r < 8; ++r)
#pragma unroll
                        for (int c = 0; c < kCW; c += 4)
                            grad_step4<kP1, true>(acc[r][c], acc[r][c + 1], acc[r][c + 2], acc[r][c + 3], xv[r][c],
                                                  xv[r][c + 1], xv[r][c + 2], xv[r][c + 3], xs[c], xs[c + 1],
                                                  xs[c + 2], xs[c + 3], wv[r]);
                }
                __syncthreads();
                continue;
            }
        }
        for (int jj = 0; jj < jmax; ++jj) {
            const floatx4 w0 = *reinterpret_cast<const floatx4 *>(&Ws[jj][8 * ty]);
            const floatx4 w1 = *reinterpret_cast<const floatx4 *>(&Ws[jj][8 * ty + 4]);
            float x[kCW];
            load_panel(x, jj, tx);
            const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
            float dv[8];
            if constexpr (kTwo) {
                const floatx4 d0 = *reinterpret_cast<const floatx4 *>(&Ds[jj][8 * ty]);
                const floatx4 d1 = *reinterpret_cast<const floatx4 *>(&Ds[jj][8 * ty + 4]);
                dv[0] = d0[0]; dv[1] = d0[1]; dv[2] = d0[2]; dv[3] = d0[3];
                dv[4] = d1[0]; dv[5] = d1[1]; dv[6] = d1[2]; dv[7] = d1[3];
            } else {
#pragma unroll
                for (int r = 0; r < 8; ++r) dv[r] = 0.0f;
            }
            if constexpr ((MODE == kRoot && (PK == kP2 || PK == kP3)) || kHalfSum) {
#pragma unroll
                for (int r = 0; r < 8; ++r)
#pragma unroll
                    for (int c = 0; c < kCW; c += 4)
                        grad_step4<PK>(acc[r][c], acc[r][c + 1], acc[r][c + 2], acc[r][c + 3], xv[r][c], xv[r][c + 1],
                                       xv[r][c + 2], xv[r][c + 3], x[c], x[c + 1], x[c + 2], x[c + 3], wv[r]);
            } else {
#pragma unroll
                for (int r = 0; r < 8; ++r)
#pragma unroll
                    for (int c = 0; c < kCW; ++c)
                        acc[r][c] += fam_term<MODE, PK, WGRAD>(xv[r][c], x[c], wv[r], dv[r], wkv[c], p);
            }
        }
        __syncthreads();
    }

    float *o = out + (split * batch + b) * n * d;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const int64_t i = i0 + 8 * ty + r;
        if (i >= n) continue;
#pragma unroll
        for (int c = 0; c < kCW; ++c) {
            const int64_t k = k0 + feat_of(tx, c);
            if (k < d) o[i * d + k] = kHalfSum ? 2.0f * acc[r][c] : acc[r][c];
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

// *flag = 1 where some value of a [la] or b [lb] lies outside sign_scalable's range (the caller
// clears the flag first; every writer stores the same 1).
__global__ void sign_range_kernel(const float *__restrict__ a, int64_t la, const float *__restrict__ b, int64_t lb,
                                  uint32_t *__restrict__ flag) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    bool bad = false;
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < la + lb; t += stride)
        bad = bad || !sign_scalable(t < la ? a[t] : b[t - la]);
    if (__any(bad) && (threadIdx.x & 63) == 0) *flag = 1u;
}

// Column sums of t [batch, n, d] over n, in a fixed order: blocks of 64 columns x 256 rows
// write partial sums [batch, chunks, d]; column_finish_kernel adds the chunks in order.
constexpr int kColRows = 256;
__global__ void column_partial_kernel(const float *__restrict__ t, int64_t n, int64_t d,
                                      float *__restrict__ part) {
    __shared__ float red[4][64];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int64_t k = (int64_t)blockIdx.x * 64 + tx, chunk = blockIdx.y, b = blockIdx.z;
    const int64_t r0 = chunk * kColRows;
    float s = 0.0f;
    if (k < d)
        for (int64_t r = r0 + ty; r < r0 + kColRows && r < n; r += 4) s += t[(b * n + r) * d + k];
    red[ty][tx] = s;
    __syncthreads();
    if (ty == 0 && k < d)
        part[(b * gridDim.y + chunk) * d + k] = ((red[0][tx] + red[1][tx]) + red[2][tx]) + red[3][tx];
}
__global__ void column_finish_kernel(const float *__restrict__ part, int64_t chunks, int64_t d,
                                     int64_t batch, float *__restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= batch * d) return;
    const int64_t b = t / d, k = t - b * d;
    float s = 0.0f;
    for (int64_t c = 0; c < chunks; ++c) s += part[(b * chunks + c) * d + k];
    out[t] = s;
}

// g'[t] = (g[t] * o[t]) * es: the gradient of out = exp(-gamma * dist) with respect to dist,
// es = -gamma, one rounding per product as the backward of exp_ and then of mul_(-gamma).
// VEC: 16-byte aligned arrays, four per step, the len % 4 tail by the first threads.
template <bool VEC>
__global__ void exp_grad_kernel(const float *__restrict__ g, const float *__restrict__ o, float es, int64_t len,
                                float *__restrict__ out) {
    const int64_t start = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t tail = 0;
    if constexpr (VEC) {
        const int64_t len4 = len >> 2;
        for (int64_t t = start; t < len4; t += stride) {
            const floatx4 gv = reinterpret_cast<const floatx4 *>(g)[t];
            const floatx4 ov = reinterpret_cast<const floatx4 *>(o)[t];
            floatx4 r;
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = __fmul_rn(__fmul_rn(gv[e], ov[e]), es);
            reinterpret_cast<floatx4 *>(out)[t] = r;
        }
        tail = len4 << 2;
    }
    for (int64_t t = tail + start; t < len; t += stride) out[t] = __fmul_rn(__fmul_rn(g[t], o[t]), es);
}

__global__ void fill_kernel(float *__restrict__ p, int64_t len, float v) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < len) p[t] = v;
}

int pkind_of(double p) {
    if (p == 0.0) return kP0;
    if (p == 1.0) return kP1;
    if (p == 2.0) return kP2;
    if (p == 3.0) return kP3;
    if (isinf(p)) return p > 0 ? kPInf : kPNInf;
    if (p > 0.0 && p < 2.0) return kPLt2;
    return kPGen;
}

template <int MODE, int PK>
int launch_forward(const float *x1, const float *x2, const float *w, int64_t batch, int64_t n,
                   int64_t m, int64_t d, double p, float *out, hipStream_t s, bool exp_post = false,
                   float post = 0.0f, const float *rownum = nullptr, uint16_t *out16 = nullptr) {
    dim3 grid((unsigned)cdiv(m, kTile), (unsigned)cdiv(n, kTile), (unsigned)batch);
    const bool vec = (d % 4 == 0) && aligned16(x1) && aligned16(x2) && aligned16(out) && aligned16(out16);
    const float pf = (float)p, inv_p = (float)(1.0 / p);
    const LaunchEvents ev = launch_events("lp_forward_kernel");
    auto launch = [&](auto om) {
        constexpr int OM = decltype(om)::value;
        if (vec)
            hipExtLaunchKernelGGL((lp_forward_kernel<MODE, PK, true, OM>), grid, dim3(kThreads), 0, s, ev.start,
                                  ev.stop, 0, x1, x2, w, n, m, d, pf, inv_p, out, post, rownum, out16);
        else
            hipExtLaunchKernelGGL((lp_forward_kernel<MODE, PK, false, OM>), grid, dim3(kThreads), 0, s, ev.start,
                                  ev.stop, 0, x1, x2, w, n, m, d, pf, inv_p, out, post, rownum, out16);
    };
    // the bf16 output exists for the cdist metrics (kRoot), the row-numerator divide for the
    // signal-to-noise ratio (kSum, p = 2), the exp for the laplacian (kRoot, p = 1) and rbf
    // (kSum, p = 2) kernels: only those instantiations carry them
    if (exp_post) {
        if constexpr ((MODE == kRoot && PK == kP1) || (MODE == kSum && PK == kP2))
            launch(std::integral_constant<int, 3>{});
        else TPW_REQUIRE(false, "the exp epilogue is for the laplacian and rbf kernels");
    } else if (out16) {
        if constexpr (MODE == kRoot) launch(std::integral_constant<int, 1>{});
        else TPW_REQUIRE(false, "bf16 output is for the cdist metrics");
    } else if (rownum) {
        if constexpr (MODE == kSum && PK == kP2) launch(std::integral_constant<int, 2>{});
        else TPW_REQUIRE(false, "the row-numerator divide is for the signal-to-noise ratio");
    } else {
        launch(std::integral_constant<int, 0>{});
    }
    return check_launch("lp_forward_kernel");
}

template <int MODE>
int dispatch_forward(int pk, const float *x1, const float *x2, const float *w, int64_t batch,
                     int64_t n, int64_t m, int64_t d, double p, float *out, hipStream_t s,
                     uint16_t *out16 = nullptr) {
    switch (pk) {
        case kP0: return launch_forward<MODE, kP0>(x1, x2, w, batch, n, m, d, p, out, s, false, 0.0f, nullptr, out16);
        case kP1: return launch_forward<MODE, kP1>(x1, x2, w, batch, n, m, d, p, out, s, false, 0.0f, nullptr, out16);
        case kP2: return launch_forward<MODE, kP2>(x1, x2, w, batch, n, m, d, p, out, s, false, 0.0f, nullptr, out16);
        case kP3: return launch_forward<MODE, kP3>(x1, x2, w, batch, n, m, d, p, out, s, false, 0.0f, nullptr, out16);
        case kPInf: return launch_forward<MODE, kPInf>(x1, x2, w, batch, n, m, d, p, out, s, false, 0.0f, nullptr, out16);
        case kPNInf:
            return launch_forward<MODE, kPNInf>(x1, x2, w, batch, n, m, d, p, out, s, false, 0.0f, nullptr, out16);
        case kPLt2: return launch_forward<MODE, kPLt2>(x1, x2, w, batch, n, m, d, p, out, s, false, 0.0f, nullptr, out16);
        default: return launch_forward<MODE, kPGen>(x1, x2, w, batch, n, m, d, p, out, s, false, 0.0f, nullptr, out16);
    }
}

int fill(float *p, int64_t len, float v, hipStream_t s) {
    if (len == 0) return TPW_OK;  // an empty buffer may be a null pointer
    TPW_REQUIRE(p, "null pointer");
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)cdiv(len, 256)), dim3(256), 0, s, p, len, v);
    return check_launch("fill_kernel");
}

// Blocks of the backward grid per CU that may be resident at once: the kernels use more
// than 128 VGPRs (at most 4 waves per SIMD, i.e. 4 blocks of 4 waves per CU).
constexpr int kMaxBlocksPerCU = 4;

int device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return 256;
    return cus;
}

// Number of j splits for `slots` resident blocks: the (row block, feature block, batch)
// grid alone fills base blocks; splitting j multiplies that, and a whole number of
// resident rounds avoids a partly filled last round.  More slots never give fewer splits,
// so the workspace is sized with the largest slot count.
int64_t lp_backward_splits(int64_t slots, int64_t batch, int64_t n, int64_t m, int64_t d, int64_t fw) {
    const int64_t base = cdiv(n, kBRows) * cdiv(d, fw) * batch;
    if (base == 0) return 1;  // no output rows (empty n, d or batch): nothing to split
    int64_t splits = base >= slots ? 1 : slots / base;
    const int64_t max_by_m = cdiv(m, 512);
    if (splits > max_by_m) splits = max_by_m;
    if (splits > 16) splits = 16;
    if (splits < 1) splits = 1;
    while (splits > 1 && splits * batch > kMaxGridYZ) --splits;
    return splits;
}
int64_t max_slots() { return (int64_t)device_cus() * kMaxBlocksPerCU; }

// grad [batch, n, d] of the first operand (x2's gradient: pass x2 as x1, n <-> m, TR).
template <int MODE, int PK, bool TR, bool WGRAD, bool PRE, int FW, bool EXPG = false>
int launch_backward(const float *g, const float *aux0, const float *aux1, const float *x1,
                    const float *x2, const float *w, int64_t batch, int64_t n, int64_t m, int64_t d,
                    double p, float *grad, float *part, hipStream_t s, const float *eo = nullptr,
                    float es = 0.0f, const uint32_t *gate = nullptr, uint32_t gate_run = 0,
                    int64_t *shared_splits = nullptr, bool finish = true) {
    // the direct layout's staging lanes span two rows of m: their byte offsets are 32-bit
    TPW_REQUIRE(TR || 4 * m + 128 < ((int64_t)1 << 32),
                "backward: %lld columns exceed the kernel's 32-bit staging offsets", (long long)m);
    auto kern = lp_backward_kernel<MODE, PK, TR, WGRAD, PRE, FW, EXPG>;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kThreads, 0) != hipSuccess || per_cu <= 0)
        per_cu = 2;
    if (per_cu > kMaxBlocksPerCU) per_cu = kMaxBlocksPerCU;
    // gated instances of one backward share the first one's split count (and so the partials'
    // layout and the one sum_splits pass after the last)
    int64_t splits = shared_splits && *shared_splits > 0
                         ? *shared_splits
                         : lp_backward_splits((int64_t)device_cus() * per_cu, batch, n, m, d, FW);
    if (shared_splits) *shared_splits = splits;
    const int64_t jps = cdiv(cdiv(m, splits), kBJ) * kBJ;
    dim3 grid((unsigned)cdiv(d, FW), (unsigned)cdiv(n, kBRows), (unsigned)(splits * batch));
    float *dst = splits > 1 ? part : grad;
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, s, g, aux0, aux1, x1, x2, w, n, m, d, (float)p,
                       jps, batch, dst, eo, es, gate, gate_run);
    int rc = check_launch("lp_backward_kernel");
    if (rc != TPW_OK || splits == 1 || !finish) return rc;
    const int64_t len = batch * n * d;
    hipLaunchKernelGGL(sum_splits_kernel, dim3((unsigned)cdiv(len, 256)), dim3(256), 0, s, part,
                       splits, len, grad);
    return check_launch("sum_splits_kernel");
}

// Per-pair weights into w1 (and w2), for the kPrecomputed cases.
template <int MODE, int PK>
int launch_pair_weights(const float *g, const float *aux0, const float *aux1, int64_t len,
                        double p, float *w1, float *w2, hipStream_t s) {
    const bool vec = aligned16(g) && aligned16(aux0) && aligned16(aux1) && aligned16(w1) && aligned16(w2);
    const int64_t items = vec ? cdiv(len, 4) : len;
    const unsigned grid = (unsigned)(cdiv(items, 256) < 16384 ? cdiv(items, 256) : 16384);
    if (vec)
        hipLaunchKernelGGL((pair_weight_kernel<MODE, PK, true>), dim3(grid), dim3(256), 0, s, g, aux0, aux1,
                           len, (float)p, w1, w2);
    else
        hipLaunchKernelGGL((pair_weight_kernel<MODE, PK, false>), dim3(grid), dim3(256), 0, s, g, aux0,
                           aux1, len, (float)p, w1, w2);
    return check_launch("pair_weight_kernel");
}

// The gradient of the first operand and/or (TWO) of the second, and/or (WG) the row
// partials of the weight gradient, sharing one weight precomputation.  wbuf1 / wbuf2
// receive the precomputed weights ([batch, n, m] each) where the case uses them.
struct BwdJob {
    const float *g, *aux0, *aux1, *x1, *x2, *w;
    int64_t batch, n, m, d;
    double p;
    float *gx1, *gx2, *rows, *part, *wbuf1, *wbuf2;
    bool x1_transposed;  // single-direction call for x2's gradient (x1/x2 already swapped)
    const float *eo = nullptr;  // exp-scaled gradient (EXPG): the exp kernel's output, and -gamma
    float es = 0.0f;
    uint32_t *flag = nullptr;  // a workspace word for the p = 1 range flag (nullptr: no wide p = 1)
};

template <int MODE, int PK, int FW, bool PRE, bool EXPG = false>
int run_backward_fw(const BwdJob &j, hipStream_t s) {
    // staging reads the per-pair arrays only where the weights need them
    constexpr bool kAux = PRE || (MODE == kRoot && PK != kP1);
    const float *a0 = kAux ? j.aux0 : nullptr, *a1 = kAux ? j.aux1 : nullptr;
    if constexpr (PRE) {
        constexpr bool two = MODE == kBrayDen;
        const int rc = launch_pair_weights<MODE, PK>(j.g, j.aux0, j.aux1, j.batch * j.n * j.m, j.p,
                                                     j.wbuf1, two ? j.wbuf2 : nullptr, s);
        if (rc != TPW_OK) return rc;
        a0 = j.wbuf1;
        a1 = two ? j.wbuf2 : nullptr;
    }
    int rc = TPW_OK;
    if (j.gx1) {
        if (j.x1_transposed)  // n, m are already those of the operand whose grad is wanted
            rc = launch_backward<MODE, PK, true, false, PRE, FW, EXPG>(j.g, a0, a1, j.x1, j.x2, j.w, j.batch, j.n,
                                                                    j.m, j.d, j.p, j.gx1, j.part, s, j.eo, j.es);
        else
            rc = launch_backward<MODE, PK, false, false, PRE, FW, EXPG>(j.g, a0, a1, j.x1, j.x2, j.w, j.batch, j.n,
                                                                     j.m, j.d, j.p, j.gx1, j.part, s, j.eo, j.es);
    }
    if (rc == TPW_OK && j.gx2)
        rc = launch_backward<MODE, PK, true, false, PRE, FW, EXPG>(j.g, a0, a1, j.x2, j.x1, j.w, j.batch, j.m, j.n,
                                                                j.d, j.p, j.gx2, j.part, s, j.eo, j.es);
    if constexpr (MODE == kWeighted) {
        if (rc == TPW_OK && j.rows)
            rc = launch_backward<MODE, PK, false, true, PRE, FW>(j.g, a0, a1, j.x1, j.x2, j.w, j.batch, j.n,
                                                              j.m, j.d, j.p, j.rows, j.part, s);
    }
    return rc;
}

// p = 1 (the root or the power sum) above 64 features: sign_range_kernel flags x1 and x2 values
// outside the pre-scaled sign path's range, then the wide kernel (sign path only; runs when the
// flag is clear) and the narrow one (per-tile test and signf path; runs when it is set) are both
// launched with the wide kernel's split count, and one sum_splits pass follows.
template <int MODE, bool EXPG = false>
int run_backward_p1_gated(const BwdJob &j, hipStream_t s) {
    int rc = fill(reinterpret_cast<float *>(j.flag), 1, 0.0f, s);
    if (rc != TPW_OK) return rc;
    const int64_t l1 = j.batch * j.n * j.d, l2 = j.batch * j.m * j.d;
    const int64_t blocks = cdiv(l1 + l2, 256 * 8);
    hipLaunchKernelGGL(sign_range_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s, j.x1,
                       l1, j.x2, l2, j.flag);
    rc = check_launch("sign_range_kernel");
    if (rc != TPW_OK) return rc;
    auto both = [&](auto tr, const float *xa, const float *xb, int64_t na, int64_t nb, float *grad) {
        constexpr bool TR = decltype(tr)::value;
        int64_t sp = 0;
        int r = launch_backward<MODE, kP1, TR, false, false, kBFeatWide, EXPG>(
            j.g, nullptr, nullptr, xa, xb, j.w, j.batch, na, nb, j.d, j.p, grad, j.part, s, j.eo, j.es, j.flag, 0u,
            &sp, false);
        if (r != TPW_OK) return r;
        return launch_backward<MODE, kP1, TR, false, false, kBFeat, EXPG>(j.g, nullptr, nullptr, xa, xb, j.w, j.batch,
                                                                           na, nb, j.d, j.p, grad, j.part, s, j.eo,
                                                                           j.es, j.flag, 1u, &sp, true);
    };
    if (j.gx1) {
        rc = j.x1_transposed ? both(std::true_type{}, j.x1, j.x2, j.n, j.m, j.gx1)
                             : both(std::false_type{}, j.x1, j.x2, j.n, j.m, j.gx1);
        if (rc != TPW_OK) return rc;
    }
    if (j.gx2) rc = both(std::true_type{}, j.x2, j.x1, j.m, j.n, j.gx2);
    return rc;
}

// The wide kernel above 64 features where it serves the case and its 16-byte staging fits
// (aligned arrays, n, m and d multiples of 4); else the narrow one.
// Whether run_backward takes run_backward_p1_gated (p = 1: the wide kernel's shapes, and a flag word).
bool p1_gated_fits(const BwdJob &j) {
    return j.flag && j.d > kBFeat && j.n % 4 == 0 && j.m % 4 == 0 && j.d % 4 == 0 && aligned16(j.g) &&
           aligned16(j.x1) && aligned16(j.x2) && aligned16(j.eo);
}

template <int MODE, int PK, bool EXPG = false>
int run_backward(const BwdJob &j, hipStream_t s) {
    if constexpr (PK == kP1 && (MODE == kRoot || MODE == kSum)) {
        if (p1_gated_fits(j)) return run_backward_p1_gated<MODE, EXPG>(j, s);
    }
    if constexpr (kWide<MODE, PK>) {
        const bool fits = j.d > kBFeat && j.n % 4 == 0 && j.m % 4 == 0 && j.d % 4 == 0 && aligned16(j.g) &&
                          aligned16(j.aux0) && aligned16(j.x1) && aligned16(j.x2) && aligned16(j.eo);
        if (fits) return run_backward_fw<MODE, PK, kBFeatWide, false, EXPG>(j, s);
    }
    static_assert(!EXPG || !kPrecomputed<MODE, PK>, "the exp-scaled gradient is formed while staging");
    return run_backward_fw<MODE, PK, kBFeat, kPrecomputed<MODE, PK>, EXPG>(j, s);
}

template <int MODE>
int dispatch_backward(int pk, const BwdJob &j, hipStream_t s) {
    switch (pk) {
        case kP1: return run_backward<MODE, kP1>(j, s);
        case kP2: return run_backward<MODE, kP2>(j, s);
        case kP3: return run_backward<MODE, kP3>(j, s);
        case kPInf:
            if constexpr (MODE == kRoot) return run_backward<MODE, kPInf>(j, s);
            break;
        case kPLt2: return run_backward<MODE, kPLt2>(j, s);
        case kPGen: return run_backward<MODE, kPGen>(j, s);
        default: break;
    }
    set_error("backward for p = %g is not supported by this kernel", j.p);
    return TPW_ERR_INVALID;
}

// Workspace of the backward: [split partials | weight gradient rows | column partials |
// pair buffer 1 | pair buffer 2].  Pair buffers hold the precomputed weights (and, for
// Bray-Curtis, the denominator that buffer 1 is computed from in place).
struct Workspace {
    size_t part, rows, cols, pair1, pair2, flag, total;
    // the range flag's word (the last 256 bytes)
    uint32_t *flag_word(void *ws) const {
        return reinterpret_cast<uint32_t *>(static_cast<char *>(ws) + part + rows + cols + pair1 + pair2);
    }
};
inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }
Workspace workspace_layout(int metric, int64_t batch, int64_t n, int64_t m, int64_t d) {
    const int64_t slots = max_slots();
    // the wide kernel's grid has fewer feature blocks, so it may take more splits
    int64_t s1 = lp_backward_splits(slots, batch, n, m, d, kBFeatWide);
    int64_t s2 = lp_backward_splits(slots, batch, m, n, d, kBFeatWide);
    const int64_t s1n = lp_backward_splits(slots, batch, n, m, d, kBFeat);
    const int64_t s2n = lp_backward_splits(slots, batch, m, n, d, kBFeat);
    s1 = s1 > s1n ? s1 : s1n;
    s2 = s2 > s2n ? s2 : s2n;
    Workspace w{};
    const int64_t part1 = s1 > 1 ? s1 * batch * n * d : 0, part2 = s2 > 1 ? s2 * batch * m * d : 0;
    w.part = align256(sizeof(float) * (size_t)(part1 > part2 ? part1 : part2));
    const size_t pair = align256(sizeof(float) * (size_t)(batch * n * m));
    if (metric == TPW_FAM_WMINKOWSKI) {
        w.rows = align256(sizeof(float) * (size_t)(batch * n * d));
        w.cols = align256(sizeof(float) * (size_t)(batch * cdiv(n, kColRows) * d));
    }
    if (metric == TPW_FAM_WMINKOWSKI || metric == TPW_FAM_BRAYCURTIS || metric < 0) w.pair1 = pair;
    if (metric == TPW_FAM_BRAYCURTIS) w.pair2 = pair;
    // the p = 1 range flag: the Minkowski (cdist) backward, laplacian_kernel's and the p-power sum's
    if (metric < 0 || metric == TPW_FAM_PPMINKOWSKI) w.flag = 256;
    w.total = w.part + w.rows + w.cols + w.pair1 + w.pair2 + w.flag;
    return w;
}
constexpr int kLpMetric = -1;  // the Minkowski (cdist) backward in workspace_layout

#define TPW_FAM_CHECKS()                                                                     \
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");                   \
    TPW_REQUIRE(cdiv(n, kTile) <= kMaxGridYZ && cdiv(m, kTile) <= kMaxGridYZ && batch <= kMaxGridYZ, \
                "too many rows or batches")

}  // namespace
}  // namespace tpw

using namespace tpw;

extern "C" int tpw_lp_distances(const float *x1, const float *x2, int64_t batch, int64_t n,
                                int64_t m, int64_t d, double p, float *out, void *stream) {
    TPW_FAM_CHECKS();
    TPW_REQUIRE(p >= 0.0, "p must be non-negative, got %g", p);
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    return dispatch_forward<kRoot>(pkind_of(p), x1, x2, nullptr, batch, n, m, d, p, out,
                                   as_stream(stream));
}

extern "C" int tpw_lp_distances_bf16(const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m,
                                     int64_t d, double p, uint16_t *out, void *stream) {
    TPW_FAM_CHECKS();
    TPW_REQUIRE(p >= 0.0, "p must be non-negative, got %g", p);
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    return dispatch_forward<kRoot>(pkind_of(p), x1, x2, nullptr, batch, n, m, d, p, nullptr, as_stream(stream),
                                   out);
}

extern "C" int tpw_snr_centered(const float *a, const float *b, const float *v1, int64_t batch, int64_t n,
                                int64_t m, int64_t d, float *out, void *stream) {
    TPW_FAM_CHECKS();
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(a && b && v1 && out, "null pointer");
    return launch_forward<kSum, kP2>(a, b, nullptr, batch, n, m, d, 2.0, out, as_stream(stream), false, 0.0f, v1);
}

extern "C" size_t tpw_lp_backward_workspace_size(int64_t batch, int64_t n, int64_t m, int64_t d) {
    return workspace_layout(kLpMetric, batch, n, m, d).total;
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
    if (p == 0.0 || m == 0)  // zero gradient, as _cdist_backward returns for p == 0
        return fill(grad_x1, batch * n * d, 0.0f, s);
    TPW_REQUIRE(grad && x1 && x2 && dist, "null pointer");
    const Workspace lay = workspace_layout(kLpMetric, batch, n, m, d);
    TPW_REQUIRE(workspace, "workspace of %zu bytes required", lay.total);
    char *ws = static_cast<char *>(workspace);
    BwdJob j{grad, dist, nullptr, x1, x2, nullptr, batch, n, m, d, p, grad_x1, nullptr, nullptr,
             reinterpret_cast<float *>(ws), reinterpret_cast<float *>(ws + lay.part + lay.rows + lay.cols),
             nullptr, transposed != 0};
    j.flag = lay.flag_word(ws);
    return dispatch_backward<kRoot>(pkind_of(p), j, s);
}

extern "C" int tpw_lp_distances_backward2(const float *grad, const float *x1, const float *x2,
                                          const float *dist, int64_t batch, int64_t n, int64_t m,
                                          int64_t d, double p, float *grad_x1, float *grad_x2,
                                          void *workspace, void *stream) {
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    TPW_REQUIRE(p >= 0.0, "p must be non-negative, got %g", p);
    TPW_REQUIRE(cdiv(n, kBRows) <= kMaxGridYZ && cdiv(m, kBRows) <= kMaxGridYZ, "too many rows");
    if (batch == 0 || d == 0 || (n == 0 && m == 0)) return TPW_OK;
    hipStream_t s = as_stream(stream);
    if (p == 0.0 || n == 0 || m == 0) {
        const int rc = fill(grad_x1, batch * n * d, 0.0f, s);
        return rc != TPW_OK ? rc : fill(grad_x2, batch * m * d, 0.0f, s);
    }
    TPW_REQUIRE(grad && x1 && x2 && dist && grad_x1 && grad_x2, "null pointer");
    const Workspace lay = workspace_layout(kLpMetric, batch, n, m, d);
    TPW_REQUIRE(workspace, "workspace of %zu bytes required", lay.total);
    char *ws = static_cast<char *>(workspace);
    BwdJob j{grad, dist, nullptr, x1, x2, nullptr, batch, n, m, d, p, grad_x1, grad_x2, nullptr,
             reinterpret_cast<float *>(ws), reinterpret_cast<float *>(ws + lay.part + lay.rows + lay.cols),
             nullptr, false};
    j.flag = lay.flag_word(ws);
    return dispatch_backward<kRoot>(pkind_of(p), j, s);
}

// ----------------------------------------------------------------- reference kernel family
extern "C" int tpw_ppminkowski(const float *x1, const float *x2, int64_t batch, int64_t n,
                               int64_t m, int64_t d, double p, float *out, void *stream) {
    TPW_FAM_CHECKS();
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    hipStream_t s = as_stream(stream);
    if (p == 0.0) return fill(out, batch * n * m, (float)d, s);  // ppminkowski_kernel.cpp:90-91
    return dispatch_forward<kSum>(pkind_of(p), x1, x2, nullptr, batch, n, m, d, p, out, s);
}

extern "C" int tpw_wminkowski(const float *x1, const float *x2, const float *w, int64_t batch,
                              int64_t n, int64_t m, int64_t d, double p, float *out, void *stream) {
    TPW_FAM_CHECKS();
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && w && out, "null pointer");
    hipStream_t s = as_stream(stream);
    if (p == 0.0) return fill(out, batch * n * m, (float)d, s);  // wminkowski_kernel.cpp:101-102
    return dispatch_forward<kWeighted>(pkind_of(p), x1, x2, w, batch, n, m, d, p, out, s);
}

extern "C" int tpw_canberra(const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m,
                            int64_t d, float *out, void *stream) {
    TPW_FAM_CHECKS();
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    return launch_forward<kCanberra, kP1>(x1, x2, nullptr, batch, n, m, d, 1.0, out, as_stream(stream));
}

extern "C" int tpw_braycurtis(const float *x1, const float *x2, int64_t batch, int64_t n, int64_t m,
                              int64_t d, float *out, void *stream) {
    TPW_FAM_CHECKS();
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    hipStream_t s = as_stream(stream);
    const int rc = launch_forward<kRoot, kP1>(x1, x2, nullptr, batch, n, m, d, 1.0, out, s);
    if (rc != TPW_OK) return rc;
    return launch_forward<kBrayDen, kP1>(x1, x2, nullptr, batch, n, m, d, 1.0, out, s);
}

extern "C" size_t tpw_family_backward_workspace_size(int metric, int64_t batch, int64_t n,
                                                     int64_t m, int64_t d) {
    return workspace_layout(metric, batch, n, m, d).total;
}

#define TPW_FAM_BWD_PROLOGUE(METRIC)                                                          \
    TPW_FAM_CHECKS();                                                                        \
    if (batch == 0 || d == 0 || (n == 0 && m == 0)) return TPW_OK;                           \
    const Workspace lay = workspace_layout(METRIC, batch, n, m, d);                          \
    TPW_REQUIRE(lay.total == 0 || workspace, "workspace of %zu bytes required", lay.total); \
    char *ws = static_cast<char *>(workspace);                                               \
    float *part = reinterpret_cast<float *>(ws);                                             \
    float *rows = reinterpret_cast<float *>(ws + lay.part);                                  \
    float *cols = reinterpret_cast<float *>(ws + lay.part + lay.rows);                       \
    float *pair1 = reinterpret_cast<float *>(ws + lay.part + lay.rows + lay.cols);           \
    float *pair2 = reinterpret_cast<float *>(ws + lay.part + lay.rows + lay.cols + lay.pair1); \
    (void)rows, (void)cols, (void)pair1, (void)pair2;                                        \
    hipStream_t s = as_stream(stream)

extern "C" int tpw_ppminkowski_backward(const float *grad, const float *x1, const float *x2,
                                        int64_t batch, int64_t n, int64_t m, int64_t d, double p,
                                        float *grad_x1, float *grad_x2, void *workspace,
                                        void *stream) {
    TPW_FAM_BWD_PROLOGUE(TPW_FAM_PPMINKOWSKI);
    if (p == 0.0 || n == 0 || m == 0) {  // zero gradients (ppminkowski_kernel.cpp:236)
        int rc = fill(grad_x1, batch * n * d, 0.0f, s);
        return rc != TPW_OK ? rc : fill(grad_x2, batch * m * d, 0.0f, s);
    }
    TPW_REQUIRE(grad && x1 && x2 && grad_x1 && grad_x2, "null pointer");
    if (isinf(p))  // the first arg-extremum's sign (ppminkowski_kernel.cpp:171-208)
        return lp_inf_backward(grad, x1, x2, nullptr, batch, n, m, d, p < 0, grad_x1, grad_x2, nullptr, s);
    BwdJob j{grad, nullptr, nullptr, x1, x2, nullptr, batch, n, m, d, p, grad_x1, grad_x2, nullptr,
             part, nullptr, nullptr, false};
    j.flag = lay.flag_word(ws);
    return dispatch_backward<kSum>(pkind_of(p), j, s);
}

extern "C" int tpw_wminkowski_backward(const float *grad, const float *x1, const float *x2,
                                       const float *w, const float *out, int64_t batch, int64_t n,
                                       int64_t m, int64_t d, double p, float *grad_x1,
                                       float *grad_x2, float *grad_w, void *workspace,
                                       void *stream) {
    TPW_FAM_BWD_PROLOGUE(TPW_FAM_WMINKOWSKI);
    if (p == 0.0 || n == 0 || m == 0) {  // zero gradients (wminkowski_kernel.cpp:296)
        int rc = fill(grad_x1, batch * n * d, 0.0f, s);
        if (rc == TPW_OK) rc = fill(grad_x2, batch * m * d, 0.0f, s);
        return rc != TPW_OK ? rc : fill(grad_w, batch * d, 0.0f, s);
    }
    TPW_REQUIRE(grad && x1 && x2 && w && out && grad_x1 && grad_x2 && grad_w, "null pointer");
    int rc;
    if (isinf(p)) {  // the first weighted arg-extremum (wminkowski_kernel.cpp:214-265)
        rc = lp_inf_backward(grad, x1, x2, w, batch, n, m, d, p < 0, grad_x1, grad_x2, rows, s);
    } else {
        BwdJob j{grad, out, nullptr, x1, x2, w, batch, n, m, d, p, grad_x1, grad_x2, rows, part, pair1,
                 nullptr, false};
        rc = dispatch_backward<kWeighted>(pkind_of(p), j, s);
    }
    if (rc != TPW_OK) return rc;
    const int64_t chunks = cdiv(n, kColRows);
    hipLaunchKernelGGL(column_partial_kernel, dim3((unsigned)cdiv(d, 64), (unsigned)chunks, (unsigned)batch),
                       dim3(256), 0, s, rows, n, d, cols);
    rc = check_launch("column_partial_kernel");
    if (rc != TPW_OK) return rc;
    hipLaunchKernelGGL(column_finish_kernel, dim3((unsigned)cdiv(batch * d, 256)), dim3(256), 0, s,
                       cols, chunks, d, batch, grad_w);
    return check_launch("column_finish_kernel");
}

extern "C" int tpw_canberra_backward(const float *grad, const float *x1, const float *x2,
                                     int64_t batch, int64_t n, int64_t m, int64_t d,
                                     float *grad_x1, float *grad_x2, void *workspace,
                                     void *stream) {
    TPW_FAM_BWD_PROLOGUE(TPW_FAM_CANBERRA);
    if (n == 0 || m == 0) {
        int rc = fill(grad_x1, batch * n * d, 0.0f, s);
        return rc != TPW_OK ? rc : fill(grad_x2, batch * m * d, 0.0f, s);
    }
    TPW_REQUIRE(grad && x1 && x2 && grad_x1 && grad_x2, "null pointer");
    BwdJob j{grad, nullptr, nullptr, x1, x2, nullptr, batch, n, m, d, 1.0, grad_x1, grad_x2, nullptr,
             part, nullptr, nullptr, false};
    return dispatch_backward<kCanberra>(kP1, j, s);
}

extern "C" int tpw_braycurtis_backward(const float *grad, const float *x1, const float *x2,
                                       const float *out, int64_t batch, int64_t n, int64_t m,
                                       int64_t d, float *grad_x1, float *grad_x2, void *workspace,
                                       void *stream) {
    TPW_FAM_BWD_PROLOGUE(TPW_FAM_BRAYCURTIS);
    if (n == 0 || m == 0) {
        int rc = fill(grad_x1, batch * n * d, 0.0f, s);
        return rc != TPW_OK ? rc : fill(grad_x2, batch * m * d, 0.0f, s);
    }
    TPW_REQUIRE(grad && x1 && x2 && out && grad_x1 && grad_x2, "null pointer");
    // ss = sum_k |a + b| per pair into pair buffer 1, recomputed as the reference's backward
    // does; the weights then overwrite it in place (w1) and fill pair buffer 2 (w2)
    int rc = launch_forward<kPlusSum, kP1>(x1, x2, nullptr, batch, n, m, d, 1.0, pair1, s);
    if (rc != TPW_OK) return rc;
    BwdJob j{grad, out, pair1, x1, x2, nullptr, batch, n, m, d, 1.0, grad_x1, grad_x2, nullptr, part,
             pair1, pair2, false};
    return dispatch_backward<kBrayDen>(kP1, j, s);
}

extern "C" int tpw_additive_chi2(const float *x1, const float *x2, int64_t batch, int64_t n,
                                 int64_t m, int64_t d, float *out, void *stream) {
    TPW_FAM_CHECKS();
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    return launch_forward<kChi2, kP1>(x1, x2, nullptr, batch, n, m, d, 1.0, out, as_stream(stream));
}

extern "C" int tpw_sqjensenshannon(const float *x1, const float *x2, int64_t batch, int64_t n,
                                   int64_t m, int64_t d, double divisor, float *out, void *stream) {
    TPW_FAM_CHECKS();
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    // launch_forward passes inv_p = 1 / p; the JS epilogue divides by inv_p, so p = 1 / divisor
    return launch_forward<kJS, kP1>(x1, x2, nullptr, batch, n, m, d, 1.0 / divisor, out, as_stream(stream));
}

extern "C" int tpw_additive_chi2_backward(const float *grad, const float *x1, const float *x2,
                                          int64_t batch, int64_t n, int64_t m, int64_t d,
                                          float *grad_x1, float *grad_x2, void *workspace,
                                          void *stream) {
    TPW_FAM_BWD_PROLOGUE(TPW_FAM_CHI2);
    if (n == 0 || m == 0) {
        int rc = fill(grad_x1, batch * n * d, 0.0f, s);
        return rc != TPW_OK ? rc : fill(grad_x2, batch * m * d, 0.0f, s);
    }
    TPW_REQUIRE(grad && x1 && x2 && grad_x1 && grad_x2, "null pointer");
    BwdJob j{grad, nullptr, nullptr, x1, x2, nullptr, batch, n, m, d, 1.0, grad_x1, grad_x2, nullptr,
             part, nullptr, nullptr, false};
    return dispatch_backward<kChi2>(kP1, j, s);
}

extern "C" int tpw_sqjensenshannon_backward(const float *grad, const float *x1, const float *x2,
                                            int64_t batch, int64_t n, int64_t m, int64_t d,
                                            double divisor, float *grad_x1, float *grad_x2,
                                            void *workspace, void *stream) {
    TPW_FAM_BWD_PROLOGUE(TPW_FAM_JS);
    if (n == 0 || m == 0) {
        int rc = fill(grad_x1, batch * n * d, 0.0f, s);
        return rc != TPW_OK ? rc : fill(grad_x2, batch * m * d, 0.0f, s);
    }
    TPW_REQUIRE(grad && x1 && x2 && grad_x1 && grad_x2, "null pointer");
    BwdJob j{grad, nullptr, nullptr, x1, x2, nullptr, batch, n, m, d, divisor, grad_x1, grad_x2,
             nullptr, part, nullptr, nullptr, false};
    return dispatch_backward<kJS>(kP1, j, s);
}

extern "C" int tpw_pairwise_exp_kernel(const float *x1, const float *x2, int64_t batch, int64_t n,
                                       int64_t m, int64_t d, int kind, float gamma, float *out,
                                       void *stream) {
    TPW_FAM_CHECKS();
    TPW_REQUIRE(kind == TPW_KER_RBF || kind == TPW_KER_LAPLACIAN, "unknown kernel %d", kind);
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    hipStream_t s = as_stream(stream);
    // mul_(-gamma) multiplies by the scalar rounded to float; d == 0 gives exp(0) = 1
    const float post = -gamma;
    if (kind == TPW_KER_RBF)  // sqeuclidean = _ppminkowski p = 2: sum of squares, no root
        return launch_forward<kSum, kP2>(x1, x2, nullptr, batch, n, m, d, 2.0, out, s, true, post);
    return launch_forward<kRoot, kP1>(x1, x2, nullptr, batch, n, m, d, 1.0, out, s, true, post);
}

extern "C" size_t tpw_pairwise_exp_kernel_backward_workspace_size(int kind, int64_t batch, int64_t n, int64_t m,
                                                                 int64_t d) {
    return workspace_layout(kind == TPW_KER_RBF ? TPW_FAM_PPMINKOWSKI : kLpMetric, batch, n, m, d).total;
}

extern "C" int tpw_pairwise_exp_kernel_backward(const float *grad, const float *out, const float *x1,
                                                const float *x2, int64_t batch, int64_t n, int64_t m, int64_t d,
                                                int kind, float gamma, float *grad_x1, float *grad_x2,
                                                void *workspace, void *stream) {
    TPW_REQUIRE(kind == TPW_KER_RBF || kind == TPW_KER_LAPLACIAN, "unknown kernel %d", kind);
    const int metric = kind == TPW_KER_RBF ? TPW_FAM_PPMINKOWSKI : kLpMetric;
    TPW_FAM_BWD_PROLOGUE(metric);
    if (n == 0 || m == 0) {
        int rc = fill(grad_x1, batch * n * d, 0.0f, s);
        return rc != TPW_OK ? rc : fill(grad_x2, batch * m * d, 0.0f, s);
    }
    TPW_REQUIRE(grad && out && x1 && x2 && grad_x1 && grad_x2, "null pointer");
    // each pair's gradient of the distance is (grad * out) * (-gamma), the backward of exp_ and
    // then of mul_(-gamma); then the sqeuclidean (_ppminkowski p = 2) or cdist p = 1 backward
    if (kind == TPW_KER_RBF) {
        // formed while the backward kernel stages its pairs: no N x M array is written
        BwdJob j{grad, nullptr, nullptr, x1, x2, nullptr, batch, n, m, d, 2.0, grad_x1, grad_x2, nullptr, part,
                 nullptr, nullptr, false, out, -gamma};
        return run_backward<kSum, kP2, true>(j, s);
    }
    // p = 1: on the wide kernel's shapes (run_backward_p1_gated) the gradient is formed while the
    // kernels stage their pairs (the narrow fallback instance too, at two waves per SIMD: it runs
    // only for values outside the sign path's range); elsewhere a second per-pair array would
    // take the narrow kernel from three waves per SIMD to two (156 -> 174 VGPRs), so one
    // elementwise pass writes the gradients into the workspace first
    {
        BwdJob j{grad, nullptr, nullptr, x1, x2, nullptr, batch, n, m, d, 1.0, grad_x1, grad_x2, nullptr, part,
                 nullptr, nullptr, false, out, -gamma};
        j.flag = lay.flag_word(ws);
        if (p1_gated_fits(j)) return run_backward<kRoot, kP1, true>(j, s);
    }
    const int64_t len = batch * n * m;
    const bool vec = aligned16(grad) && aligned16(out) && aligned16(pair1);
    const unsigned grid = (unsigned)(cdiv(vec ? cdiv(len, 4) : len, 256) < 16384 ? cdiv(vec ? cdiv(len, 4) : len, 256)
                                                                                  : 16384);
    if (vec)
        hipLaunchKernelGGL(exp_grad_kernel<true>, dim3(grid), dim3(256), 0, s, grad, out, -gamma, len, pair1);
    else
        hipLaunchKernelGGL(exp_grad_kernel<false>, dim3(grid), dim3(256), 0, s, grad, out, -gamma, len, pair1);
    const int rc = check_launch("exp_grad_kernel");
    if (rc != TPW_OK) return rc;
    BwdJob j{pair1, nullptr, nullptr, x1, x2, nullptr, batch, n, m, d, 1.0, grad_x1, grad_x2, nullptr, part,
             nullptr, nullptr, false};
    j.flag = lay.flag_word(ws);
    return run_backward<kRoot, kP1>(j, s);
}
