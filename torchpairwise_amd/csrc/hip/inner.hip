// Inner-product family on the CDNA4 matrix cores: out = epilogue(x1 . x2^T, aux1, aux2).
//
// Block = 256 threads (4 waves, 2 x 2), output tile 128 x 128, wave tile 64 x 64 = 2 x 2
// blocks of 32 x 32.  Each K chunk is 128 bytes of every operand row (32 fp32 or 64 bf16
// features), staged in LDS with a 16-byte pad per row (144-byte stride, conflict-free
// 16-byte reads for 16 consecutive rows).  The k index inside a chunk is permuted so that
// every lane feeds the MFMA from one contiguous 64-byte run of its row: lane (i + 32 h)
// supplies features [h*KC/2, (h+1)*KC/2) of row i, in the order the MFMA k slots consume
// them; A and B use the same permutation, so the sum over k is unchanged.
//   fp32: v_mfma_f32_32x32x2_f32, 16 per chunk and 32 x 32 block
//   bf16: v_mfma_f32_32x32x16_bf16 (gfx950), 4 per chunk and block, fp32 accumulation
// The epilogue (norms, sqrt, guarded divide, clip) is applied to the accumulators in
// registers and the result is written once with non-temporal stores.
// Operand staging, two paths:
//   direct (every chunk full: d a multiple of the chunk, 16-byte rows): the chunk goes from
//     global memory straight into LDS with global_load_lds_dwordx4, no registers in between;
//     each wave covers 9 x 64 of the 2304 16-byte slots of the padded A|B panels (a pad slot
//     loads a duplicate piece that is never read; rows past the edge load the last row,
//     whose outputs are not stored).  120 VGPRs: 4 waves per SIMD, 4 blocks per CU;
//   register prefetch (any d): the next chunk's global loads are issued into registers
//     before the current chunk's MFMAs, and stored to LDS after them (zero padding past d).
// Tiles are assigned XCD-contiguously (consecutive workgroup ids go round-robin over the
// 8 XCDs, so id % 8 selects the XCD) and in groups of 8 tile rows, so that the blocks
// resident on one XCD share A and B panels in that XCD's L2.
#include "common.hpp"
#include "tile_mfma.hpp"

namespace tpw {
namespace {

constexpr int kThreads = 256;
constexpr int kTile = 128;
constexpr int kRowVec = 8;              // uint4 per 128-byte chunk row
constexpr int kLdsStride = kRowVec + 1; // in uint4 (144 bytes)
constexpr int kStageStride = 68;         // floats per staged output row (64 + 4 pad)
static_assert(4 * 32 * kStageStride * 4 <= 2 * kTile * kLdsStride * 16, "staging fits the panels");

template <typename T>
struct Elem;
template <>
struct Elem<float> {
    static constexpr int kPer16 = 4;
    static constexpr int kChunk = 32;
    __device__ static float load(const float *p) { return *p; }
};
template <>
struct Elem<uint16_t> {  // bf16 bits
    static constexpr int kPer16 = 8;
    static constexpr int kChunk = 64;
};

// Gradient products of the backward (not a public epilogue code): out = sign * s +
// aux1[row] * X[row, col], X having the output's type and shape.
constexpr int kEpiGrad = 100;
// The kernel functions of tpw_pairwise_kernel: (s gamma + coef0)^degree and
// tanh(s gamma + coef0).
constexpr int kEpiPoly = 101;
constexpr int kEpiSigmoid = 102;
// kEpiGrad with coef[row] = the sum over K of A's row (tile kernel only).
constexpr int kEpiGradA = 103;
// radius_neighbors_mask (euclidean): the euclidean epilogue's value, as the distance op stores it
// (kEpiRadiusB: rounded to bf16), compared with kp.eps: 1 when d <= eps (NaN: 0), as bool bytes.
constexpr int kEpiRadius = 104;
constexpr int kEpiRadiusB = 105;
// k_neighbors_mask (euclidean): per output row, the C smallest (distance, column) keys among the
// tile's 128 columns, written as candidates instead of the distances (topk_tile_epilogue).
// EPI = kEpiTopK + 2 log2(C / 2) for C = 2, 4, 8, 16, + 1 when the distance is first rounded to
// bf16, as the bf16 distance op stores it.
constexpr int kEpiTopK = 106;
// The polynomial kernel for degree 0 .. 3 (products, no powf): the same values as kEpiPoly, on
// the tile kernel, whose four blocks per CU the general degree's powf would spill.
constexpr int kEpiPolySmall = 120;
// Output stores: non-temporal for fp32 and bf16 (matrix-core or data-path bound: plain stores
// cost 1-4 %), plain for the radius mask's bool bytes (0.553 -> 0.540 ms at 16384^2).
template <typename OutT>
constexpr bool kStoreNT = sizeof(OutT) > 1;
template <int EPI>
constexpr bool kTopK = EPI >= kEpiTopK && EPI < kEpiTopK + 8;
template <int EPI>
constexpr int kTopKC = 2 << ((EPI - kEpiTopK) >> 1);
template <int EPI>
constexpr bool kTopKB = ((EPI - kEpiTopK) & 1) != 0;

// Row / column norms read by the epilogue (aux1 also carries the gradient coefficients).
template <int EPI>
constexpr bool kAux1 = EPI == TPW_EPI_EUCLIDEAN || EPI == TPW_EPI_SQEUCLIDEAN ||
                       EPI == TPW_EPI_COSINE_SIM || EPI == TPW_EPI_COSINE_DIST ||
                       EPI == TPW_EPI_CORRELATION || EPI == kEpiGrad || EPI == kEpiRadius ||
                       EPI == kEpiRadiusB || kTopK<EPI>;
template <int EPI>
constexpr bool kAux2 = kAux1<EPI> && EPI != kEpiGrad;

// x^k for k = 0 .. 3 as ipow below computes it (products).
__device__ __forceinline__ float ipow_small(float x, int k) {
#pragma clang fp contract(off)
    if (k == 2) return x * x;
    if (k == 3) return x * x * x;
    if (k == 1) return x;
    return 1.0f;
}

// x^k for an integral k as ATen's pow with a scalar exponent computes it on the GPU: k = 2, 3
// as products, otherwise the float power function.
__device__ __forceinline__ float ipow(float x, int k) {
#pragma clang fp contract(off)
    if (k == 2) return x * x;
    if (k == 3) return x * x * x;
    if (k == 1) return x;
    if (k == 0) return 1.0f;
    return powf(x, (float)k);
}

template <int EPI>
__device__ __forceinline__ float epilogue(float s, float a1, float a2, const KerParams &kp) {
#pragma clang fp contract(off)
    if constexpr (EPI == kEpiPoly || EPI == kEpiPolySmall || EPI == kEpiSigmoid) {
        // the reference's matmul(...).mul_(gamma).add_(coef0), then pow_ / tanh_
        const float base = s * kp.gamma + kp.coef0;
        if constexpr (EPI == kEpiPolySmall) return ipow_small(base, kp.degree);
        return EPI == kEpiPoly ? ipow(base, kp.degree) : tanhf(base);
    } else if constexpr (EPI == TPW_EPI_DOT || EPI == kEpiGrad) {
        return s;
    } else if constexpr (EPI == kEpiRadius || EPI == kEpiRadiusB) {
        float v = epilogue<TPW_EPI_EUCLIDEAN>(s, a1, a2, kp);
        if constexpr (EPI == kEpiRadiusB) v = bf16_to_f32(f32_to_bf16_rne(v));
        return v <= kp.eps ? 1.0f : 0.0f;
    } else if constexpr (EPI == TPW_EPI_EUCLIDEAN || EPI == TPW_EPI_SQEUCLIDEAN) {
        // (a1 + a2) - 2 s with one rounding: 2 s is exact, so the fma is bit-identical
        float v = __builtin_fmaf(-2.0f, s, a1 + a2);
        v = v > 0.0f ? v : 0.0f;
        // v_sqrt_f32 (1 ulp): the |a|^2 + |b|^2 - 2ab form already carries more error
        if constexpr (EPI == TPW_EPI_EUCLIDEAN) v = __builtin_amdgcn_sqrtf(v);
        return v;
    } else {
        float den = a1 * a2;
        float q = den != 0.0f ? __fdiv_rn(s, den) : s;
        if constexpr (EPI == TPW_EPI_COSINE_SIM) return q;
        float v = 1.0f - q;
        if constexpr (EPI == TPW_EPI_CORRELATION) return v;
        return fminf(fmaxf(v, 0.0f), 2.0f);
    }
}

// bf16 cosine-family outputs: where every norm of a tile lies in [2^-60, 2^60] (so each n1 n2 is
// a normal nonzero float and the quotient branch above applies), q = s r1 r2 from the rows' and
// columns' reciprocals r = RN(1 / norm) instead of an IEEE divide per element: within 2 ulp of
// the quotient before the output's bf16 rounding (2^-9).  Tiles with another norm (zero
// included) keep epilogue<>.
template <int EPI, typename OutT>
constexpr bool kCosRcp = sizeof(OutT) == 2 && (EPI == TPW_EPI_COSINE_SIM || EPI == TPW_EPI_COSINE_DIST ||
                                               EPI == TPW_EPI_CORRELATION);

template <int EPI>
__device__ __forceinline__ float cos_epilogue_rcp(float s, float r1, float r2) {
#pragma clang fp contract(off)
    const float q = s * (r1 * r2);
    if constexpr (EPI == TPW_EPI_COSINE_SIM) return q;
    const float v = 1.0f - q;
    if constexpr (EPI == TPW_EPI_CORRELATION) return v;
    return fminf(fmaxf(v, 0.0f), 2.0f);
}

// The tile's 256 norms (rows, then columns; thread t owns entry t) replaced by their reciprocals
// when all of them lie in [2^-60, 2^60]; whether they were (the same in every thread).
__device__ __forceinline__ bool cos_norms_to_rcp(float *s_aux, int tid) {
    const float v = s_aux[tid];
    if (!__syncthreads_and(v >= 0x1p-60f && v <= 0x1p60f)) return false;
    s_aux[tid] = __fdiv_rn(1.0f, v);
    __syncthreads();
    return true;
}

// Selection order of the neighbour masks: ascending distance (distances are >= 0 or -0; -0 ==
// +0, NaN after +inf), then ascending column.  Columns past the edge take the largest key.
__device__ __forceinline__ uint64_t topk_key(float v, uint32_t col) {
    const uint32_t bits = v != v ? 0xffffffffu : (__float_as_uint(v) & 0x7fffffffu);
    return ((uint64_t)bits << 32) | col;
}
__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int mask) {
    const uint32_t lo = __shfl_xor((uint32_t)v, mask, 64), hi = __shfl_xor((uint32_t)(v >> 32), mask, 64);
    return ((uint64_t)hi << 32) | lo;
}
// x into the ascending list L, the largest falling off (a compare-exchange chain).
template <int C>
__device__ __forceinline__ void topk_insert(uint64_t (&L)[C], uint64_t x) {
#pragma unroll
    for (int i = 0; i < C; ++i) {
        const bool lt = x < L[i];
        const uint64_t lo = lt ? x : L[i];
        x = lt ? L[i] : x;
        L[i] = lo;
    }
}
// L := the C smallest of the ascending lists L and R, ascending: the element-wise minimum of L
// and reversed R is bitonic, and a bitonic merge network sorts it.
template <int C>
__device__ __forceinline__ void topk_merge(uint64_t (&L)[C], const uint64_t (&R)[C]) {
#pragma unroll
    for (int i = 0; i < C; ++i) {
        const uint64_t r = R[C - 1 - i];
        L[i] = r < L[i] ? r : L[i];
    }
#pragma unroll
    for (int j = C / 2; j > 0; j >>= 1)
#pragma unroll
        for (int i = 0; i < C; ++i)
            if ((i & j) == 0) {
                const uint64_t a = L[i], c = L[i + j];
                L[i] = a < c ? a : c;
                L[i + j] = a < c ? c : a;
            }
}

__device__ __forceinline__ void store_out(float *p, float v) { store_nt(p, v); }
__device__ __forceinline__ void store_out(uint16_t *p, float v) {
    __builtin_nontemporal_store(f32_to_bf16_rne(v), p);
}
__device__ __forceinline__ void store_out(uint8_t *p, float v) { *p = v != 0.0f ? 1 : 0; }

// Loads one 16-byte piece (row r, piece c of chunk kc) of a [rows, d] operand.
template <typename T, bool VEC>
__device__ __forceinline__ uint4 load_piece(const T *__restrict__ x, int64_t rows, int64_t d,
                                            int64_t r, int64_t kbase) {
    uint4 v = {0u, 0u, 0u, 0u};
    if (r >= rows) return v;
    constexpr int E = Elem<T>::kPer16;
    if constexpr (VEC) {
        if (kbase < d) v = *reinterpret_cast<const uint4 *>(x + r * d + kbase);
    } else {
        const T *p = x + r * d;
        if constexpr (E == 4) {
            uint32_t e[4];
#pragma unroll
            for (int t = 0; t < 4; ++t)
                e[t] = (kbase + t < d) ? __float_as_uint(p[kbase + t]) : 0u;
            v = make_uint4(e[0], e[1], e[2], e[3]);
        } else {
            uint32_t e[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                uint32_t lo = (kbase + 2 * t < d) ? (uint32_t)p[kbase + 2 * t] : 0u;
                uint32_t hi = (kbase + 2 * t + 1 < d) ? (uint32_t)p[kbase + 2 * t + 1] : 0u;
                e[t] = lo | (hi << 16);
            }
            v = make_uint4(e[0], e[1], e[2], e[3]);
        }
    }
    return v;
}

// One 16-byte k-piece of the chunk: a[mi] / b[ni] hold the lane's 4 fp32 (or 8 bf16) features
// of its A row / B column for this piece.
__device__ __forceinline__ void mfma_piece(floatx16 (&acc)[2][2], const uint4 (&a)[2],
                                           const uint4 (&b)[2], float) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const uint32_t av = e == 0 ? a[mi].x : e == 1 ? a[mi].y : e == 2 ? a[mi].z : a[mi].w;
                const uint32_t bv = e == 0 ? b[ni].x : e == 1 ? b[ni].y : e == 2 ? b[ni].z : b[ni].w;
                acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                    __uint_as_float(av), __uint_as_float(bv), acc[mi][ni], 0, 0, 0);
            }
        }
    }
}

__device__ __forceinline__ void mfma_piece(floatx16 (&acc)[2][2], const uint4 (&a)[2],
                                           const uint4 (&b)[2], uint16_t) {
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8, a[mi]), __builtin_bit_cast(bf16x8, b[ni]), acc[mi][ni],
                0, 0, 0);
        }
    }
}

typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;
constexpr int kSlotsPerWave = 9;  // 2 panels x 128 rows x 9 slots / 4 waves / 64 lanes

template <typename T, typename OutT, int EPI, bool VEC, bool DIRECT>
__global__ __launch_bounds__(kThreads, 2) void pairwise_inner_kernel(
    const T *__restrict__ x1, const T *__restrict__ x2, int64_t n, int64_t m, int64_t d,
    const float *__restrict__ aux1, const float *__restrict__ aux2, OutT *__restrict__ out,
    int64_t tiles_n, int64_t tiles_m, int64_t total, const OutT *__restrict__ X, float sign,
    KerParams kp) {
    // operand panels (As, Bs); after the K loop the same bytes stage the fp32 output
    __shared__ uint4 smem[2 * kTile * kLdsStride];
    uint4 *As = smem;
    uint4 *Bs = smem + kTile * kLdsStride;
    // norms of the tile's rows ([0]) and columns ([1]); published by the first barrier of the
    // K loop (or the one for d == 0)
    __shared__ __align__(16) float s_aux[2][kTile];
    constexpr int E = Elem<T>::kPer16;
    constexpr int KC = Elem<T>::kChunk;

    int64_t b, tr, tc;
    xcd_tile_of(blockIdx.x, tiles_n, tiles_m, total, b, tr, tc);
    const int64_t row0 = tr * kTile, col0 = tc * kTile;
    const T *A = x1 + b * n * d;
    const T *B = x2 + b * m * d;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
    const int l32 = lane & 31, h = lane >> 5;

    if constexpr (kAux1<EPI>) {
        const int i = tid & (kTile - 1);
        if (tid < kTile) s_aux[0][i] = row0 + i < n ? aux1[b * n + row0 + i] : 0.0f;
        else if (kAux2<EPI>) s_aux[1][i] = col0 + i < m ? aux2[b * m + col0 + i] : 0.0f;
    }

    floatx16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.0f;

    const int64_t nchunks = (d + KC - 1) / KC;
    if (nchunks == 0) __syncthreads();
    uint4 pa[DIRECT ? 1 : 4], pb[DIRECT ? 1 : 4];
    int32_t off[DIRECT ? kSlotsPerWave : 1];
    if constexpr (DIRECT) {
        // element offsets (from the panel's batch base) of this lane's slot in each of its 9
        // wave loads: slot s -> panel s / 1152, row (s % 1152) / 9, piece (s % 1152) % 9
#pragma unroll
        for (int j = 0; j < kSlotsPerWave; ++j) {
            const int sl = (wave * kSlotsPerWave + j) * 64 + lane;
            const int panel = sl >= kTile * kLdsStride;
            const int s2 = sl - panel * kTile * kLdsStride;
            const int r = s2 / kLdsStride, c0 = s2 - r * kLdsStride;
            const int c = c0 == kRowVec ? kRowVec - 1 : c0;
            const int64_t lim = panel ? m : n;
            int64_t row = (panel ? col0 : row0) + r;
            row = row < lim ? row : lim - 1;
            off[j] = (int32_t)(row * d + c * E);
        }
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int idx = tid + kThreads * q;
            const int r = idx >> 3, c = idx & 7;
            pa[q] = load_piece<T, VEC>(A, n, d, row0 + r, (int64_t)c * E);
            pb[q] = load_piece<T, VEC>(B, m, d, col0 + r, (int64_t)c * E);
        }
    }

    for (int64_t kc = 0; kc < nchunks; ++kc) {
        if constexpr (DIRECT) {
            const int64_t kb = kc * KC;
#pragma unroll
            for (int j = 0; j < kSlotsPerWave; ++j) {
                const int first = (wave * kSlotsPerWave + j) * 64;  // wave-uniform LDS slot
                const T *src = (first >= kTile * kLdsStride ? B : A) + kb + off[j];
                __builtin_amdgcn_global_load_lds((global_void *)src, (lds_void *)(smem + first), 16, 0, 0);
            }
            __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's slots have landed
            __syncthreads();
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int idx = tid + kThreads * q;
                const int r = idx >> 3, c = idx & 7;
                As[r * kLdsStride + c] = pa[q];
                Bs[r * kLdsStride + c] = pb[q];
            }
            __syncthreads();
            if (kc + 1 < nchunks) {
                const int64_t kb = (kc + 1) * KC;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int idx = tid + kThreads * q;
                    const int r = idx >> 3, c = idx & 7;
                    pa[q] = load_piece<T, VEC>(A, n, d, row0 + r, kb + (int64_t)c * E);
                    pb[q] = load_piece<T, VEC>(B, m, d, col0 + r, kb + (int64_t)c * E);
                }
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint4 a[2], bv[2];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) a[mi] = As[(wr + mi * 32 + l32) * kLdsStride + h * 4 + q];
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) bv[ni] = Bs[(wc + ni * 32 + l32) * kLdsStride + h * 4 + q];
            mfma_piece(acc, a, bv, T{});
        }
        __syncthreads();
    }

    bool rcp = false;  // bf16 cosine family: s_aux holds reciprocals
    if constexpr (kCosRcp<EPI, OutT>) rcp = cos_norms_to_rcp(&s_aux[0][0], tid);
    // the output value of accumulator s
    auto value = [&](float s, float a1, float a2) {
        if constexpr (kCosRcp<EPI, OutT>)
            if (rcp) return cos_epilogue_rcp<EPI>(s, a1, a2);
        return epilogue<EPI>(s, a1, a2, kp);
    };
    // Accumulator layout of the 32 x 32 MFMA: register r of lane l holds
    // row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
    const bool full = row0 + kTile <= n && col0 + kTile <= m;
    float a2v[2];
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
        a2v[ni] = kAux2<EPI> ? s_aux[1][wc + ni * 32 + l32] : 0.0f;
    // bf16 rows are written 8 values (16 bytes) per lane: needs m % 8 == 0 for alignment
    const bool staged = full && (sizeof(OutT) == 4 || (sizeof(OutT) == 2 && m % 8 == 0));
    {
        if (staged) {
            // full tile: each wave stages a 32 x 64 half of its tile in fp32 in its own LDS
            // slice (the operand panels are free after the K loop's last barrier) and writes
            // it back in row segments: fp32 as float4 (16 lanes per 256-byte segment), bf16
            // as 8 rounded values per lane (8 lanes per 128-byte segment).
            float *stage = reinterpret_cast<float *>(smem) + wave * (32 * kStageStride);
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) {
                // the norms of the lane's 16 rows: 4 groups of 4 consecutive rows
                floatx4 a1q[4];
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    a1q[g] = kAux1<EPI> ? *reinterpret_cast<const floatx4 *>(&s_aux[0][wr + mi * 32 + 8 * g + 4 * h])
                                        : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int rr = 8 * (r >> 2) + 4 * h + (r & 3);
                        const float a1 = a1q[r >> 2][r & 3];
                        stage[rr * kStageStride + ni * 32 + l32] =
                            EPI == kEpiGrad ? sign * acc[mi][ni][r] : value(acc[mi][ni][r], a1, a2v[ni]);
                    }
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes landed
                __builtin_amdgcn_wave_barrier();
                const int64_t ooff = (b * n + row0 + wr + mi * 32) * m + col0 + wc;
                OutT *orow = out + ooff;
                if constexpr (sizeof(OutT) == 4) {
#pragma unroll
                    for (int it = 0; it < 8; ++it) {
                        const int rr = it * 4 + (lane >> 4), cc = (lane & 15) * 4;
                        floatx4 v = *reinterpret_cast<const floatx4 *>(&stage[rr * kStageStride + cc]);
                        if constexpr (EPI == kEpiGrad) {
                            const float c = s_aux[0][wr + mi * 32 + rr];
                            const floatx4 xv = *reinterpret_cast<const floatx4 *>(
                                reinterpret_cast<const float *>(X) + ooff + (int64_t)rr * m + cc);
                            v += c * xv;
                        }
                        store_nt4(reinterpret_cast<float *>(orow) + (int64_t)rr * m + cc, v);
                    }
                } else {
#pragma unroll
                    for (int it = 0; it < 4; ++it) {
                        const int rr = it * 8 + (lane >> 3), cc = (lane & 7) * 8;
                        floatx4 v0 = *reinterpret_cast<const floatx4 *>(&stage[rr * kStageStride + cc]);
                        floatx4 v1 = *reinterpret_cast<const floatx4 *>(&stage[rr * kStageStride + cc + 4]);
                        if constexpr (EPI == kEpiGrad) {
                            const float c = s_aux[0][wr + mi * 32 + rr];
                            const uint4 xq = *reinterpret_cast<const uint4 *>(X + ooff + (int64_t)rr * m + cc);
                            const uint32_t xw[4] = {xq.x, xq.y, xq.z, xq.w};
#pragma unroll
                            for (int e = 0; e < 2; ++e) {
                                v0[2 * e] += c * __uint_as_float(xw[e] << 16);
                                v0[2 * e + 1] += c * __uint_as_float(xw[e] & 0xffff0000u);
                                v1[2 * e] += c * __uint_as_float(xw[2 + e] << 16);
                                v1[2 * e + 1] += c * __uint_as_float(xw[2 + e] & 0xffff0000u);
                            }
                        }
                        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                        u32x4 q;
                        q[0] = f32x2_to_bf16x2_rne(v0[0], v0[1]);
                        q[1] = f32x2_to_bf16x2_rne(v0[2], v0[3]);
                        q[2] = f32x2_to_bf16x2_rne(v1[0], v1[1]);
                        q[3] = f32x2_to_bf16x2_rne(v1[2], v1[3]);
                        __builtin_nontemporal_store(q, reinterpret_cast<u32x4 *>(orow + (int64_t)rr * m + cc));
                    }
                }
                __builtin_amdgcn_s_waitcnt(0xc07f);  // reads done before the slice is rewritten
                __builtin_amdgcn_wave_barrier();
            }
            return;
        }
    }
    OutT *obase = out + (b * n + row0 + wr + 4 * h) * m + col0 + wc + l32;
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
        const bool col_ok = col0 + wc + ni * 32 + l32 < m;
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rr = mi * 32 + 8 * (r >> 2) + (r & 3);  // row in the wave tile, less 4 h
                const float a1 = kAux1<EPI> ? s_aux[0][wr + 4 * h + rr] : 0.0f;
                if (full || (row0 + wr + 4 * h + rr < n && col_ok)) {
                    float v = value(acc[mi][ni][r], a1, a2v[ni]);
                    if constexpr (EPI == kEpiGrad) v = sign * v + a1 * to_f32(X[(obase - out) + rr * m + ni * 32]);
                    store_out(obase + rr * m + ni * 32, v);
                }
            }
        }
    }
}

// The tile kernel of tile_mfma.hpp for inputs whose K chunks are all full (d * sizeof(T) a
// multiple of 128 bytes, 16-byte aligned rows) and outputs whose rows split into whole 16-byte
// units: one 32 KiB operand buffer (4 blocks per CU), the chunk loaded by DMA while no wave
// reads it, transposed products, and the epilogue applied while the tile is staged for
// row-segment stores.  AK / BK: x1 / x2 stored k-major, [d, n] / [d, m] (the backward's products
// read W^T, x1 and x2 that way, without a transposed copy); bf16 k-major pieces come from two
// transposing LDS reads each.
// RG: bf16 output rows of m % 8 != 0 values (store_tile's ragged mode), a separate
// instantiation so that the aligned kernels' code is unchanged by it.
template <typename T, typename OutT, int EPI, int NB = 1, bool AK = false, bool BK = false, bool RG = false>
__global__ __launch_bounds__(tile::kThreads, NB == 1 ? 4 : 2) void inner_tile_kernel(
    const T *__restrict__ x1, const T *__restrict__ x2, int64_t n, int64_t m, int64_t d,
    const float *__restrict__ aux1, const float *__restrict__ aux2, OutT *__restrict__ out,
    int64_t tiles_n, int64_t tiles_m, int64_t total, KerParams kp, const OutT *__restrict__ X, float sign) {
    using namespace tile;
    __shared__ uint4 smem[NB * kBuf];
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
    // the tile's norms by DMA as well (a compiler-visible load would leave its register
    // "pending" for the compiler, which then waits for every store in flight before reusing it)
    if constexpr (kAux1<EPI>)
        dma_tile_rows(aux1 + b * n, kAux2<EPI> ? aux2 + b * m : nullptr, kAux2<EPI>, wave, lane, row0, col0, n, m,
                      s_aux);
    constexpr int ES = (int)sizeof(T);
    uint32_t off[kSlots];
    dma_offsets_k<AK, BK, ES>(off, wave, lane, row0, col0, n, m, row_bytes, n * ES, m * ES);
    // bytes from one K chunk to the next: 128 along a row, 128 / ES K rows of a k-major operand
    const int64_t a_step = AK ? 128 * n : 128, b_step = BK ? 128 * m : 128;
    const int grp = ((lane >> 4) & 1) * 16;  // first row of the lane's 16-lane group (bf16 k-major)
    dma_chunk2(A, B, off, wave, 0, 0, smem);

    floatx16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.0f;
    // kEpiGradA: this lane's share of its A rows' sums (its half of every chunk, in K order)
    float rsum[2] = {0.0f, 0.0f};

    const int nchunks = (int)(row_bytes / 128);
    for (int kc = 0; kc < nchunks; ++kc) {
        if (NB == 1 && kc > 0) {
            barrier_lds();  // every wave is done with chunk kc - 1
            dma_chunk2(A, B, off, wave, kc * a_step, kc * b_step, smem);
        }
        barrier_all();  // chunk kc (and, the first time, the norms) has landed
        // two buffers: chunk kc + 1 goes to the buffer chunk kc - 1 used, which every wave is
        // done with (the barrier above), while chunk kc is multiplied
        if (NB == 2 && kc + 1 < nchunks)
            dma_chunk2(A, B, off, wave, (kc + 1) * a_step, (kc + 1) * b_step, smem + ((kc + 1) & 1) * kBuf);
        const uint4 *As = smem + (NB == 2 ? (kc & 1) * kBuf : 0), *Bs = As + kPanel;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int c = h * 4 + q;
            uint4 a[2], bv[2];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
                a[mi] = !AK       ? piece(As, wr + mi * 32 + l32, c)
                        : ES == 4 ? kpiece(As, wr + mi * 32 + l32, h, q)
                                  : kpiece_bf16<256>(As, wr + mi * 32 + grp, lane, h, q);
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
                bv[ni] = !BK      ? piece(Bs, wc + ni * 32 + l32, c)
                         : ES == 4 ? kpiece(Bs, wc + ni * 32 + l32, h, q)
                                   : kpiece_bf16<256>(Bs, wc + ni * 32 + grp, lane, h, q);
            mfma_piece_t(acc, a, bv, T{});
            if constexpr (EPI == kEpiGradA) {
                // after the products that read the same registers (no wait of its own); the
                // piece's K values in order (bf16: low half of each word first)
#pragma unroll
                for (int mi = 0; mi < 2; ++mi) {
                    const uint32_t w4[4] = {a[mi].x, a[mi].y, a[mi].z, a[mi].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if constexpr (ES == 4) {
                            rsum[mi] += __uint_as_float(w4[e]);
                        } else {
                            rsum[mi] += __uint_as_float(w4[e] << 16);
                            rsum[mi] += __uint_as_float(w4[e] & 0xffff0000u);
                        }
                    }
                }
            }
        }
    }
    barrier_lds();  // the operand buffer becomes the output stage
    bool rcp = false;  // bf16 cosine family: s_aux holds reciprocals
    if constexpr (kCosRcp<EPI, OutT>) rcp = cos_norms_to_rcp(s_aux, tid);

    float a1v[2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
        a1v[mi] = EPI == kEpiGradA ? rsum[mi] + __shfl_xor(rsum[mi], 32, 64)  // both K halves
                  : kAux1<EPI>     ? s_aux[wr + mi * 32 + l32]
                                   : 0.0f;
    if constexpr (kTopK<EPI>) {
        // k-neighbour candidates: per row block mi, each lane keeps the C smallest keys of its 32
        // columns, merges with the lane holding the row's other 32 columns of this wave (lane ^
        // 32), and lanes 0-31 leave the list in LDS; then one thread per tile row merges the two
        // waves' lists and writes the tile's C candidates of that row, out[row][tc][0 .. C - 1].
        constexpr int C = kTopKC<EPI>;
        uint64_t *st = reinterpret_cast<uint64_t *>(smem);  // [2 waves][128 rows][C]: <= 32 KiB
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
            uint64_t L[C];
#pragma unroll
            for (int i = 0; i < C; ++i) L[i] = ~0ull;
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const floatx4 a2 = *reinterpret_cast<const floatx4 *>(&s_aux[kT + wc + ni * 32 + 8 * g + 4 * h]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float v = epilogue<TPW_EPI_EUCLIDEAN>(acc[mi][ni][4 * g + e], a1v[mi], a2[e], kp);
                        if constexpr (kTopKB<EPI>) v = bf16_to_f32(f32_to_bf16_rne(v));
                        const int64_t col = col0 + wc + ni * 32 + 8 * g + 4 * h + e;
                        topk_insert<C>(L, col < m ? topk_key(v, (uint32_t)col) : ~0ull);
                    }
                }
            uint64_t R[C];
#pragma unroll
            for (int i = 0; i < C; ++i) R[i] = shfl_xor64(L[i], 32);
            topk_merge<C>(L, R);
            if (h == 0) {
#pragma unroll
                for (int i = 0; i < C; ++i) st[((wc >> 6) * kT + wr + mi * 32 + l32) * C + i] = L[i];
            }
        }
        barrier_lds();
        if (tid < kT) {
            uint64_t L[C], R[C];
#pragma unroll
            for (int i = 0; i < C; ++i) {
                L[i] = st[tid * C + i];
                R[i] = st[(kT + tid) * C + i];
            }
            topk_merge<C>(L, R);
            const int64_t row = row0 + tid;
            if (row < n) {
                uint4 *dst = reinterpret_cast<uint4 *>(reinterpret_cast<uint64_t *>(out) + ((b * n + row) * tiles_m + tc) * C);
#pragma unroll
                for (int i = 0; i < C; i += 2)
                    dst[i / 2] = make_uint4((uint32_t)L[i], (uint32_t)(L[i] >> 32), (uint32_t)L[i + 1],
                                            (uint32_t)(L[i + 1] >> 32));
            }
        }
        return;
    } else {
    store_tile<OutT, kStoreNT<OutT>>(
        smem,
        [&](int mi, int ni, int g) {
            floatx4 o;
            if constexpr (EPI == kEpiGrad || EPI == kEpiGradA) {
                // sign * s + coef[row] * X[row][col .. col + 3] (rows and columns past the edge
                // read nothing and are not stored)
                const int64_t row = row0 + wr + mi * 32 + l32, col = col0 + wc + ni * 32 + 8 * g + 4 * h;
                floatx4 xv = {0.0f, 0.0f, 0.0f, 0.0f};
                if (row < n && col < m) {
                    const OutT *xp = X + (b * n + row) * m + col;
                    if constexpr (sizeof(OutT) == 4) {
                        xv = *reinterpret_cast<const floatx4 *>(xp);
                    } else {
                        const uint2 q = *reinterpret_cast<const uint2 *>(xp);
                        xv = floatx4{__uint_as_float(q.x << 16), __uint_as_float(q.x & 0xffff0000u),
                                     __uint_as_float(q.y << 16), __uint_as_float(q.y & 0xffff0000u)};
                    }
                }
#pragma unroll
                // one rounding for the coefficient product, one for the sum (as an explicit fma: the
                // compiler contracted the sum either way within one kernel)
                for (int e = 0; e < 4; ++e) o[e] = __builtin_fmaf(sign, acc[mi][ni][4 * g + e], a1v[mi] * xv[e]);
            } else {
                const floatx4 a2 = kAux2<EPI> ? *reinterpret_cast<const floatx4 *>(&s_aux[kT + wc + ni * 32 + 8 * g + 4 * h])
                                              : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (kCosRcp<EPI, OutT>) {
                    if (rcp) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) o[e] = cos_epilogue_rcp<EPI>(acc[mi][ni][4 * g + e], a1v[mi], a2[e]);
                        return o;
                    }
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = epilogue<EPI>(acc[mi][ni][4 * g + e], a1v[mi], a2[e], kp);
            }
            return o;
        },
        out, b, row0, col0, n, m, RG);
    }
}

// Row norms: one wave per row, lanes stride over the features.
template <typename T>
__global__ void row_norms_kernel(const T *__restrict__ x, int64_t rows, int64_t d, int squared,
                                 float *__restrict__ out) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const T *p = x + row * d;
    float s = 0.0f;
    for (int64_t k = lane; k < d; k += 64) {
        float v;
        if constexpr (sizeof(T) == 4) v = p[k];
        else v = bf16_to_f32(p[k]);
        s += v * v;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) out[row] = squared ? s : sqrt_rn(s);
}

// Row norms with 16-byte loads (rows of whole 16-byte vectors, 16-byte aligned): G lanes per
// row (a power of two, G >= the row's vector count up to 64), 64 / G rows per wave; each lane
// sums the squares of its vectors, then a butterfly over the G lanes.
template <typename T, int G>
__global__ __launch_bounds__(256) void row_norms_vec_kernel(const T *__restrict__ x, int64_t rows, int64_t d,
                                                            int squared, float *__restrict__ out) {
    constexpr int PER = 16 / (int)sizeof(T);
    const int lane = threadIdx.x & 63;
    const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * (64 / G) + lane / G;
    const int gl = lane % G;
    float s = 0.0f;
    if (row < rows) {
        const uint4 *p = reinterpret_cast<const uint4 *>(x + row * d);
        const int64_t nv = d / PER;
        for (int64_t k = gl; k < nv; k += G) {
            const uint4 v = p[k];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if constexpr (sizeof(T) == 4) {
                    const float f = __uint_as_float(w[e]);
                    s += f * f;
                } else {
                    const float lo = __uint_as_float(w[e] << 16), hi = __uint_as_float(w[e] & 0xffff0000u);
                    s += lo * lo;
                    s += hi * hi;
                }
            }
        }
    }
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (row < rows && gl == 0) out[row] = squared ? s : sqrt_rn(s);
}

template <typename T>
int launch_row_norms(const T *x, int64_t rows, int64_t d, int squared, float *norms, hipStream_t s) {
    const int64_t nv = d * (int64_t)sizeof(T) / 16;
    if ((d * (int64_t)sizeof(T)) % 16 != 0 || !aligned16(x) || nv == 0) {
        hipLaunchKernelGGL(row_norms_kernel<T>, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, x, rows, d, squared,
                           norms);
        return check_launch("row_norms_kernel");
    }
    // the smallest power of two >= nv (at most 64) lanes per row
    int g = 1;
    while (g < 64 && g < nv) g *= 2;
    const int64_t rows_per_block = 4 * (64 / g);
    const dim3 grid((unsigned)cdiv(rows, rows_per_block));
    switch (g) {
        case 1: hipLaunchKernelGGL((row_norms_vec_kernel<T, 1>), grid, dim3(256), 0, s, x, rows, d, squared, norms); break;
        case 2: hipLaunchKernelGGL((row_norms_vec_kernel<T, 2>), grid, dim3(256), 0, s, x, rows, d, squared, norms); break;
        case 4: hipLaunchKernelGGL((row_norms_vec_kernel<T, 4>), grid, dim3(256), 0, s, x, rows, d, squared, norms); break;
        case 8: hipLaunchKernelGGL((row_norms_vec_kernel<T, 8>), grid, dim3(256), 0, s, x, rows, d, squared, norms); break;
        case 16: hipLaunchKernelGGL((row_norms_vec_kernel<T, 16>), grid, dim3(256), 0, s, x, rows, d, squared, norms); break;
        case 32: hipLaunchKernelGGL((row_norms_vec_kernel<T, 32>), grid, dim3(256), 0, s, x, rows, d, squared, norms); break;
        default: hipLaunchKernelGGL((row_norms_vec_kernel<T, 64>), grid, dim3(256), 0, s, x, rows, d, squared, norms); break;
    }
    return check_launch("row_norms_vec_kernel");
}

template <typename T, int EPI, typename OutT = T>
int launch_inner(const T *x1, const T *x2, int64_t batch, int64_t n, int64_t m, int64_t d,
                 const float *aux1, const float *aux2, OutT *out, hipStream_t s,
                 const OutT *X = nullptr, float sign = 1.0f, KerParams kp = {}) {
    const int64_t tiles_n = cdiv(n, kTile), tiles_m = cdiv(m, kTile);
    const int64_t total = tiles_n * tiles_m * batch;
    const bool vec = ((d * (int64_t)sizeof(T)) % 16 == 0) && aligned16(x1) && aligned16(x2);
    // direct LDS loads: every chunk full, and the per-lane element offsets fit in int32
    const bool direct = vec && d % Elem<T>::kChunk == 0 && d > 0 && (n > m ? n : m) * d < ((int64_t)1 << 31);
    if constexpr (EPI != kEpiPoly) {
        // the tile kernel: byte offsets below 2^32, whole 16-byte units per output row (and, for
        // the gradient products, 16-byte aligned X rows).  bf16 outputs of the distance
        // epilogues also take ragged rows (store_tile's unit + head / tail stores).  Ragged fp32
        // rows stay on the staged kernel: the tile store's dword rows cost the matrix-core-bound
        // products more (16384 x 16383 x 128 euclidean 0.676 -> 0.716 ms)
        constexpr bool kRaggedOk = sizeof(OutT) == 2 && EPI != kEpiGrad && EPI != kEpiGradA;
        if (direct && (n > m ? n : m) * d * (int64_t)sizeof(T) < ((int64_t)1 << 32) && aligned16(out) &&
            (m % (16 / (int64_t)sizeof(OutT)) == 0 || kRaggedOk) && (EPI != kEpiGrad || aligned16(X))) {
            const LaunchEvents ev = launch_events("inner_tile_kernel");
            // long K (16 chunks or more): two operand buffers, the next chunk's DMA in flight
            // while the current one is multiplied, at two blocks per CU
            if constexpr (kRaggedOk) {
                if (m % (16 / (int64_t)sizeof(OutT)) != 0) {
                    if (d * (int64_t)sizeof(T) >= 16 * 128)
                        hipExtLaunchKernelGGL((inner_tile_kernel<T, OutT, EPI, 2, false, false, true>), dim3((unsigned)total),
                                           dim3(tile::kThreads), 0, s, ev.start, ev.stop, 0, x1, x2, n, m, d, aux1, aux2, out, tiles_n,
                                           tiles_m, total, kp, X, sign);
                    else
                        hipExtLaunchKernelGGL((inner_tile_kernel<T, OutT, EPI, 1, false, false, true>), dim3((unsigned)total),
                                           dim3(tile::kThreads), 0, s, ev.start, ev.stop, 0, x1, x2, n, m, d, aux1, aux2, out, tiles_n,
                                           tiles_m, total, kp, X, sign);
                    return check_launch("inner_tile_kernel");
                }
            }
            if (d * (int64_t)sizeof(T) >= 16 * 128)
                hipExtLaunchKernelGGL((inner_tile_kernel<T, OutT, EPI, 2>), dim3((unsigned)total), dim3(tile::kThreads), 0,
                                   s, ev.start, ev.stop, 0, x1, x2, n, m, d, aux1, aux2, out, tiles_n, tiles_m, total, kp, X, sign);
            else
                hipExtLaunchKernelGGL((inner_tile_kernel<T, OutT, EPI, 1>), dim3((unsigned)total), dim3(tile::kThreads), 0,
                                   s, ev.start, ev.stop, 0, x1, x2, n, m, d, aux1, aux2, out, tiles_n, tiles_m, total, kp, X, sign);
            return check_launch("inner_tile_kernel");
        }
    }
    const LaunchEvents ev = launch_events("pairwise_inner_kernel");
    auto kernel = direct ? pairwise_inner_kernel<T, OutT, EPI, true, true>
                  : vec  ? pairwise_inner_kernel<T, OutT, EPI, true, false>
                         : pairwise_inner_kernel<T, OutT, EPI, false, false>;
    hipExtLaunchKernelGGL(kernel, dim3((unsigned)total), dim3(kThreads), 0, s, ev.start, ev.stop, 0, x1, x2, n, m, d, aux1,
                       aux2, out, tiles_n, tiles_m, total, X, sign, kp);
    return check_launch("pairwise_inner_kernel");
}

// Each row's `count` smallest of its tiles' candidate keys (cand [n][tiles_m][C], ascending per
// tile) -> its bool mask row (mask [n, m], m a multiple of 16): one wave per row; every lane
// keeps the C smallest of its share, a butterfly of merges gives every lane the row's C
// smallest, and the lanes write the row in 16-byte units with 1 at the first `count` columns.
template <int C>
__global__ __launch_bounds__(256) void topk_select_kernel(const uint64_t *__restrict__ cand, int64_t n,
                                                          int64_t tiles_m, int64_t m, int count,
                                                          uint8_t *__restrict__ mask) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= n) return;  // the whole wave
    const uint64_t *c = cand + row * tiles_m * C;
    const int64_t total = tiles_m * C;
    uint64_t L[C], R[C];
#pragma unroll
    for (int i = 0; i < C; ++i) L[i] = ~0ull;
    for (int64_t i = lane; i < total; i += 64) topk_insert<C>(L, c[i]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
        for (int i = 0; i < C; ++i) R[i] = shfl_xor64(L[i], off);
        topk_merge<C>(L, R);
    }
    uint32_t sel[C];
#pragma unroll
    for (int i = 0; i < C; ++i) sel[i] = i < count ? (uint32_t)L[i] : 0xffffffffu;
    uint8_t *mrow = mask + row * m;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    for (int64_t u = lane; u < m / 16; u += 64) {
        uint32_t w0 = 0, w1 = 0, w2 = 0, w3 = 0;
#pragma unroll
        for (int i = 0; i < C; ++i) {
            const uint32_t col = sel[i];
            if ((int64_t)(col >> 4) == u) {
                const uint32_t byte = col & 15, bit = 1u << (8 * (byte & 3));
                w0 |= (byte >> 2) == 0 ? bit : 0u;
                w1 |= (byte >> 2) == 1 ? bit : 0u;
                w2 |= (byte >> 2) == 2 ? bit : 0u;
                w3 |= (byte >> 2) == 3 ? bit : 0u;
            }
        }
        const u32x4 v = {w0, w1, w2, w3};
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(mrow + 16 * u));
    }
}

int topk_width(int64_t count) { return count <= 2 ? 2 : count <= 4 ? 4 : count <= 8 ? 8 : 16; }

bool knn_fits(int dtype, int64_t n, int64_t m, int64_t d, int64_t count) {
    const int64_t es = dtype == TPW_F32 ? 4 : 2;
    const int64_t big = n > m ? n : m;
    return (dtype == TPW_F32 || dtype == TPW_BF16) && count >= 1 && count <= 16 && count <= m && m % 16 == 0 &&
           d > 0 && (d * es) % 128 == 0 && big * d < ((int64_t)1 << 31) && big * d * es < ((int64_t)1 << 32) &&
           cdiv(n, kTile) * cdiv(m, kTile) <= 0x7fffffffLL;
}

template <typename T, int EPI>
int launch_topk(const T *x1, const T *x2, int64_t n, int64_t m, int64_t d, const float *aux1, const float *aux2,
                int count, uint64_t *cand, uint8_t *mask, hipStream_t s) {
    constexpr int C = kTopKC<EPI>;
    const int64_t tiles_n = cdiv(n, kTile), tiles_m = cdiv(m, kTile), total = tiles_n * tiles_m;
    // C >= 8: the lists need the two-blocks-per-CU register budget (at four they spill)
    if (C >= 8 || d * (int64_t)sizeof(T) >= 16 * 128) {
        hipLaunchKernelGGL((inner_tile_kernel<T, uint64_t, EPI, 2>), dim3((unsigned)total), dim3(tile::kThreads), 0,
                           s, x1, x2, n, m, d, aux1, aux2, cand, tiles_n, tiles_m, total, KerParams{}, nullptr, 1.0f);
    } else if constexpr (C < 8) {
        hipLaunchKernelGGL((inner_tile_kernel<T, uint64_t, EPI, 1>), dim3((unsigned)total), dim3(tile::kThreads), 0,
                           s, x1, x2, n, m, d, aux1, aux2, cand, tiles_n, tiles_m, total, KerParams{}, nullptr, 1.0f);
    }
    int rc = check_launch("inner_tile_kernel");
    if (rc != TPW_OK) return rc;
    hipLaunchKernelGGL(topk_select_kernel<C>, dim3((unsigned)cdiv(n, 4)), dim3(256), 0, s, cand, n, tiles_m, m, count,
                       mask);
    return check_launch("topk_select_kernel");
}

template <typename T, bool BF>
int dispatch_topk(const T *x1, const T *x2, int64_t n, int64_t m, int64_t d, const float *aux1, const float *aux2,
                  int count, uint64_t *cand, uint8_t *mask, hipStream_t s) {
    switch (topk_width(count)) {
        case 2: return launch_topk<T, kEpiTopK + BF>(x1, x2, n, m, d, aux1, aux2, count, cand, mask, s);
        case 4: return launch_topk<T, kEpiTopK + 2 + BF>(x1, x2, n, m, d, aux1, aux2, count, cand, mask, s);
        case 8: return launch_topk<T, kEpiTopK + 4 + BF>(x1, x2, n, m, d, aux1, aux2, count, cand, mask, s);
        default: return launch_topk<T, kEpiTopK + 6 + BF>(x1, x2, n, m, d, aux1, aux2, count, cand, mask, s);
    }
}

template <typename T>
int dispatch_epi(const T *x1, const T *x2, int64_t batch, int64_t n, int64_t m, int64_t d,
                 const float *aux1, const float *aux2, int epi, T *out, hipStream_t s) {
    switch (epi) {
        case TPW_EPI_DOT: return launch_inner<T, TPW_EPI_DOT>(x1, x2, batch, n, m, d, aux1, aux2, out, s);
        case TPW_EPI_EUCLIDEAN: return launch_inner<T, TPW_EPI_EUCLIDEAN>(x1, x2, batch, n, m, d, aux1, aux2, out, s);
        case TPW_EPI_SQEUCLIDEAN: return launch_inner<T, TPW_EPI_SQEUCLIDEAN>(x1, x2, batch, n, m, d, aux1, aux2, out, s);
        case TPW_EPI_COSINE_SIM: return launch_inner<T, TPW_EPI_COSINE_SIM>(x1, x2, batch, n, m, d, aux1, aux2, out, s);
        case TPW_EPI_CORRELATION: return launch_inner<T, TPW_EPI_CORRELATION>(x1, x2, batch, n, m, d, aux1, aux2, out, s);
        default: return launch_inner<T, TPW_EPI_COSINE_DIST>(x1, x2, batch, n, m, d, aux1, aux2, out, s);
    }
}

}  // namespace

// S = x1 . x2^T in fp32 whatever the input type (used by the cosine backward).
int inner_dot_f32(const void *x1, const void *x2, int dtype, int64_t batch, int64_t n, int64_t m,
                  int64_t d, float *out, hipStream_t s) {
    if (dtype == TPW_F32)
        return launch_inner<float, TPW_EPI_DOT, float>(static_cast<const float *>(x1),
                                                       static_cast<const float *>(x2), batch, n, m,
                                                       d, nullptr, nullptr, out, s);
    return launch_inner<uint16_t, TPW_EPI_DOT, float>(static_cast<const uint16_t *>(x1),
                                                      static_cast<const uint16_t *>(x2), batch, n,
                                                      m, d, nullptr, nullptr, out, s);
}

// out[b] = sign * (A[b] . B[b]^T) + coef[b*M + row] * X[b][row][col] on the matrix cores
// (A [batch, M, K], B [batch, N, K], X and out [batch, M, N], all of type dtype).
int inner_grad_gemm(const void *A, const void *B, int dtype, int64_t batch, int64_t M, int64_t N,
                    int64_t K, float sign, const float *coef, const void *X, void *out, hipStream_t s) {
    if (dtype == TPW_F32)
        return launch_inner<float, kEpiGrad, float>(
            static_cast<const float *>(A), static_cast<const float *>(B), batch, M, N, K, coef, nullptr,
            static_cast<float *>(out), s, static_cast<const float *>(X), sign);
    return launch_inner<uint16_t, kEpiGrad, uint16_t>(
        static_cast<const uint16_t *>(A), static_cast<const uint16_t *>(B), batch, M, N, K, coef, nullptr,
        static_cast<uint16_t *>(out), s, static_cast<const uint16_t *>(X), sign);
}

// The gradient products' shapes for the tile kernel: whole K chunks; k-contiguous rows below
// 2^32 bytes per batch; k-major operands of whole 16-byte pieces; output rows of whole 16-byte
// units; 16-byte aligned arrays.
template <typename T>
bool grad_fits(const T *A, bool a_kmajor, const T *B, bool b_kmajor, int64_t M, int64_t N, int64_t K, const T *X,
               const T *out) {
    constexpr int64_t ES = (int64_t)sizeof(T), EPP = 16 / ES;
    auto fits = [&](const T *p, bool kmajor, int64_t rows) {
        if (!aligned16(p) || rows <= 0) return false;
        return kmajor ? rows % EPP == 0 && rows * 128 < ((int64_t)1 << 32) : rows * K * ES < ((int64_t)1 << 32);
    };
    return K > 0 && K % Elem<T>::kChunk == 0 && N % EPP == 0 && fits(A, a_kmajor, M) && fits(B, b_kmajor, N) &&
           aligned16(X) && aligned16(out);
}

template <typename T, int EPI, bool AK, bool BK>
int launch_grad_product(const T *A, const T *B, int64_t batch, int64_t M, int64_t N, int64_t K, float sign,
                        const float *coef, const T *X, T *out, hipStream_t s) {
    const int64_t tiles_n = cdiv(M, kTile), tiles_m = cdiv(N, kTile), total = tiles_n * tiles_m * batch;
    const LaunchEvents ev = launch_events("inner_tile_kernel");
    if (K * (int64_t)sizeof(T) >= 16 * 128)
        hipExtLaunchKernelGGL((inner_tile_kernel<T, T, EPI, 2, AK, BK>), dim3((unsigned)total), dim3(tile::kThreads), 0,
                           s, ev.start, ev.stop, 0, A, B, M, N, K, coef, nullptr, out, tiles_n, tiles_m, total, KerParams{}, X, sign);
    else
        hipExtLaunchKernelGGL((inner_tile_kernel<T, T, EPI, 1, AK, BK>), dim3((unsigned)total), dim3(tile::kThreads), 0,
                           s, ev.start, ev.stop, 0, A, B, M, N, K, coef, nullptr, out, tiles_n, tiles_m, total, KerParams{}, X, sign);
    return check_launch("inner_tile_kernel");
}

// Compute units of the current device (256 when the query fails), per device.
static int64_t cu_count() {
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

// The bf16 gradient product of launch_grad_product (out = sign * A'B + coef[row] * X, kEpiGrad,
// or with coef the row sums of A, kEpiGradA) for both operands k-major (A: [K, M], B: [K, N])
// on 128 x 256 output tiles, 2 x 2 waves of 64 x 128.  Each wave feeds eight 32x32x16 products
// per 16-K step from six transposed 16-byte pieces (the 128 x 128 tile kernel's waves: four
// products from four pieces), and a 64-row K chunk moves 48 KiB into LDS for 128 x 256 outputs
// (the tile kernel 64 KiB).  The products, their order (chunks, then the four 16-K steps), the
// row sums of A (in K order) and the epilogue's fma are the tile kernel's, so the outputs are
// the same bit for bit.  M % 128 == 0, N % 256 == 0, K % 64 == 0.  C2 bf16 backward: euclidean
// 1.11 -> 1.07 ms, cosine 1.185 -> 1.135 ms (same box).
template <int EPI>
__global__ __launch_bounds__(tile::kThreads, 2) void grad_wide_bf16_kernel(
    const uint16_t *__restrict__ A, const uint16_t *__restrict__ B, int64_t M, int64_t N, int64_t K,
    const float *__restrict__ coef, const uint16_t *__restrict__ X, uint16_t *__restrict__ out, int64_t tiles_n,
    int64_t tiles_c, int64_t total, float sign) {
    using namespace tile;
    constexpr int kAP = 1024, kBP = 2048, kBufW = kAP + kBP;  // uint4 per A / B panel, per buffer
    __shared__ uint4 smem[kBufW];  // 48 KiB: two blocks per CU
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 128;  // 2 x 2 waves of 64 x 128
    const int l32 = lane & 31, h = lane >> 5;
    const int grp = ((lane >> 4) & 1) * 16;
    int64_t b, tr, tc;
    xcd_tile_of(blockIdx.x, tiles_n, tiles_c, total, b, tr, tc);
    const int64_t row0 = tr * kT, col0 = tc * 256;
    const uint8_t *Ab = reinterpret_cast<const uint8_t *>(A + b * K * M);
    const uint8_t *Bb = reinterpret_cast<const uint8_t *>(B + b * K * N);
    // 12 DMA slots per lane and chunk: slot s = (12 wave + j) 64 + lane, A's 1024 first (K row
    // s / 16, position s % 16), then B's 2048 (K row s' / 32, position s' % 32); the piece at
    // position p of K row kr is logical piece p ^ 4 (kr & 3), the layout kpiece_bf16 reads; a
    // wave's 64 slots of one j lie in one panel
    uint32_t off[12];
#pragma unroll
    for (int j = 0; j < 12; ++j) {
        const int s = (wave * 12 + j) * 64 + lane;
        if (s < kAP) {
            const int kr = s >> 4, lp = (s & 15) ^ (4 * (kr & 3));
            off[j] = (uint32_t)(kr * M * 2 + (row0 + 8 * lp) * 2);
        } else {
            const int t = s - kAP, kr = t >> 5, lp = (t & 31) ^ (4 * (kr & 3));
            off[j] = (uint32_t)(kr * N * 2 + (col0 + 8 * lp) * 2);
        }
    }
    auto dma = [&](int kc, uint4 *buf) {
#pragma unroll
        for (int j = 0; j < 12; ++j) {
            const int first = (wave * 12 + j) * 64;
            const uint8_t *base = first < kAP ? Ab + (int64_t)kc * 64 * M * 2 : Bb + (int64_t)kc * 64 * N * 2;
            dma16(base, off[j], lds_addr(buf + first));
        }
    };
    floatx16 acc[2][4];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.0f;
    float rsum[2] = {0.0f, 0.0f};
    const int nchunks = (int)(K / 64);
    dma(0, smem);
    for (int kc = 0; kc < nchunks; ++kc) {
        if (kc > 0) {
            barrier_lds();  // every wave is done with chunk kc - 1
            dma(kc, smem);
        }
        barrier_all();  // chunk kc has landed
        const uint4 *As = smem, *Bs = As + kAP;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint4 a[2], bv[4];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) a[mi] = kpiece_bf16<256>(As, wr + mi * 32 + grp, lane, h, q);
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) bv[ni] = kpiece_bf16<512>(Bs, wc + ni * 32 + grp, lane, h, q);
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 4; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, bv[ni]), __builtin_bit_cast(bf16x8, a[mi]), acc[mi][ni], 0, 0, 0);
            if constexpr (EPI == kEpiGradA) {
#pragma unroll
                for (int mi = 0; mi < 2; ++mi) {
                    const uint32_t w4[4] = {a[mi].x, a[mi].y, a[mi].z, a[mi].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        rsum[mi] += __uint_as_float(w4[e] << 16);
                        rsum[mi] += __uint_as_float(w4[e] & 0xffff0000u);
                    }
                }
            }
        }
    }
    barrier_lds();  // the buffer becomes the output stage
    uint4 *sl = smem + wave * 512;  // 8 KiB per wave
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
        const int64_t row = row0 + wr + mi * 32 + l32;
        const float a1v = EPI == kEpiGradA ? rsum[mi] + __shfl_xor(rsum[mi], 32, 64) : coef[b * M + row];
        store_wave_rows_bf16<4>(
            sl,
            [&](int ni, int gq) {
                const int64_t col = col0 + wc + ni * 32 + 8 * gq + 4 * h;
                const uint2 qv = *reinterpret_cast<const uint2 *>(X + (b * M + row) * N + col);
                const floatx4 xv = {__uint_as_float(qv.x << 16), __uint_as_float(qv.x & 0xffff0000u),
                                    __uint_as_float(qv.y << 16), __uint_as_float(qv.y & 0xffff0000u)};
                floatx4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = __builtin_fmaf(sign, acc[mi][ni][4 * gq + e], a1v * xv[e]);
                return o;
            },
            out, b, row0 + wr + mi * 32, col0 + wc, M, N);
    }
}

bool grad_product_f32_fits(const float *A, bool a_kmajor, const float *B, bool b_kmajor, int64_t M, int64_t N,
                           int64_t K, const float *X, const float *out) {
    return grad_fits(A, a_kmajor, B, b_kmajor, M, N, K, X, out);
}

int grad_product_f32(const float *A, bool a_kmajor, const float *B, bool b_kmajor, int64_t batch, int64_t M,
                     int64_t N, int64_t K, float sign, const float *coef, const float *X, float *out,
                     hipStream_t s) {
    TPW_REQUIRE(grad_fits(A, a_kmajor, B, b_kmajor, M, N, K, X, out), "unsupported product shape");
    TPW_REQUIRE(b_kmajor, "k-contiguous B: inner_grad_gemm");
    if (coef == nullptr)
        return a_kmajor ? launch_grad_product<float, kEpiGradA, true, true>(A, B, batch, M, N, K, sign, coef, X, out, s)
                        : launch_grad_product<float, kEpiGradA, false, true>(A, B, batch, M, N, K, sign, coef, X, out, s);
    return a_kmajor ? launch_grad_product<float, kEpiGrad, true, true>(A, B, batch, M, N, K, sign, coef, X, out, s)
                    : launch_grad_product<float, kEpiGrad, false, true>(A, B, batch, M, N, K, sign, coef, X, out, s);
}

bool grad_product_bf16_fits(const uint16_t *A, bool a_kmajor, const uint16_t *B, bool b_kmajor, int64_t M,
                            int64_t N, int64_t K, const uint16_t *X, const uint16_t *out) {
    return grad_fits(A, a_kmajor, B, b_kmajor, M, N, K, X, out);
}

int grad_product_bf16(const uint16_t *A, bool a_kmajor, const uint16_t *B, bool b_kmajor, int64_t batch, int64_t M,
                      int64_t N, int64_t K, float sign, const float *coef, const uint16_t *X, uint16_t *out,
                      hipStream_t s) {
    TPW_REQUIRE(grad_fits(A, a_kmajor, B, b_kmajor, M, N, K, X, out), "unsupported product shape");
    TPW_REQUIRE(b_kmajor, "k-contiguous B: inner_grad_gemm");
    // 128 x 256 tiles where they fill every CU with two blocks (else the 128 x 128 kernel's
    // grid is the larger one); offsets within a batch below 2^32 bytes
    const int64_t wide_tiles = (M / 128) * (N / 256) * batch;
    if (a_kmajor && M % 128 == 0 && N % 256 == 0 && K % 64 == 0 && K * M * 2 < ((int64_t)1 << 32) &&
        K * N * 2 < ((int64_t)1 << 32) && wide_tiles >= 2 * cu_count()) {
        const LaunchEvents ev = launch_events("grad_wide_bf16_kernel");
        if (coef == nullptr)
            hipExtLaunchKernelGGL((grad_wide_bf16_kernel<kEpiGradA>), dim3((unsigned)wide_tiles), dim3(tile::kThreads), 0,
                                  s, ev.start, ev.stop, 0, A, B, M, N, K, coef, X, out, M / 128, N / 256, wide_tiles, sign);
        else
            hipExtLaunchKernelGGL((grad_wide_bf16_kernel<kEpiGrad>), dim3((unsigned)wide_tiles), dim3(tile::kThreads), 0,
                                  s, ev.start, ev.stop, 0, A, B, M, N, K, coef, X, out, M / 128, N / 256, wide_tiles, sign);
        return check_launch("grad_wide_bf16_kernel");
    }
    if (coef == nullptr)
        return a_kmajor
                   ? launch_grad_product<uint16_t, kEpiGradA, true, true>(A, B, batch, M, N, K, sign, coef, X, out, s)
                   : launch_grad_product<uint16_t, kEpiGradA, false, true>(A, B, batch, M, N, K, sign, coef, X, out, s);
    return a_kmajor
               ? launch_grad_product<uint16_t, kEpiGrad, true, true>(A, B, batch, M, N, K, sign, coef, X, out, s)
               : launch_grad_product<uint16_t, kEpiGrad, false, true>(A, B, batch, M, N, K, sign, coef, X, out, s);
}

}  // namespace tpw

using namespace tpw;

extern "C" int tpw_row_norms(const void *x, int dtype, int64_t rows, int64_t d, int squared,
                             float *norms, void *stream) {
    TPW_REQUIRE(dtype == TPW_F32 || dtype == TPW_BF16, "unsupported dtype %d", dtype);
    TPW_REQUIRE(rows >= 0 && d >= 0, "invalid sizes");
    if (rows == 0) return TPW_OK;
    TPW_REQUIRE(x && norms, "null pointer");
    hipStream_t s = as_stream(stream);
    if (dtype == TPW_F32) return launch_row_norms(static_cast<const float *>(x), rows, d, squared, norms, s);
    return launch_row_norms(static_cast<const uint16_t *>(x), rows, d, squared, norms, s);
}

extern "C" int tpw_pairwise_inner(const void *x1, const void *x2, int dtype, int64_t batch,
                                  int64_t n, int64_t m, int64_t d, const float *aux1,
                                  const float *aux2, int epilogue, void *out, void *stream) {
    TPW_REQUIRE(dtype == TPW_F32 || dtype == TPW_BF16, "unsupported dtype %d", dtype);
    TPW_REQUIRE(epilogue >= TPW_EPI_DOT && epilogue <= TPW_EPI_CORRELATION, "unknown epilogue %d",
                epilogue);
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    TPW_REQUIRE(epilogue == TPW_EPI_DOT || (aux1 && aux2), "norms required for epilogue %d",
                epilogue);
    const int64_t total = cdiv(n, kTile) * cdiv(m, kTile) * batch;
    TPW_REQUIRE(total <= 0x7fffffffLL, "output too large for one launch");
    hipStream_t s = as_stream(stream);
    if (dtype == TPW_F32)
        return dispatch_epi<float>(static_cast<const float *>(x1), static_cast<const float *>(x2),
                                   batch, n, m, d, aux1, aux2, epilogue, static_cast<float *>(out), s);
    return dispatch_epi<uint16_t>(static_cast<const uint16_t *>(x1),
                                  static_cast<const uint16_t *>(x2), batch, n, m, d, aux1, aux2,
                                  epilogue, static_cast<uint16_t *>(out), s);
}

extern "C" int tpw_radius_mask_euclidean(const void *x1, const void *x2, int dtype, int64_t batch, int64_t n,
                                         int64_t m, int64_t d, const float *aux1, const float *aux2, float eps,
                                         uint8_t *out, void *stream) {
    TPW_REQUIRE(dtype == TPW_F32 || dtype == TPW_BF16, "unsupported dtype %d", dtype);
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && aux1 && aux2 && out, "null pointer");
    TPW_REQUIRE(cdiv(n, kTile) * cdiv(m, kTile) * batch <= (int64_t)0x7fffffff, "output too large for one launch");
    hipStream_t s = as_stream(stream);
    KerParams kp;
    kp.eps = eps;
    if (dtype == TPW_F32)
        return launch_inner<float, kEpiRadius, uint8_t>(static_cast<const float *>(x1), static_cast<const float *>(x2),
                                                         batch, n, m, d, aux1, aux2, out, s, nullptr, 1.0f, kp);
    return launch_inner<uint16_t, kEpiRadiusB, uint8_t>(static_cast<const uint16_t *>(x1),
                                                         static_cast<const uint16_t *>(x2), batch, n, m, d, aux1,
                                                         aux2, out, s, nullptr, 1.0f, kp);
}

extern "C" int tpw_knn_mask_euclidean_supported(int dtype, int64_t n, int64_t m, int64_t d, int64_t count) {
    return n >= 0 && knn_fits(dtype, n, m, d, count) ? 1 : 0;
}

extern "C" size_t tpw_knn_mask_workspace_size(int64_t n, int64_t m, int64_t count) {
    return (size_t)(n * cdiv(m, kTile) * topk_width(count)) * sizeof(uint64_t) + 256;
}

extern "C" int tpw_knn_mask_euclidean(const void *x1, const void *x2, int dtype, int64_t n, int64_t m, int64_t d,
                                      const float *aux1, const float *aux2, int64_t count, uint8_t *mask,
                                      void *workspace, void *stream) {
    TPW_REQUIRE(n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    if (n == 0) return TPW_OK;
    TPW_REQUIRE(knn_fits(dtype, n, m, d, count),
                "unsupported case (dtype %d, n %lld, m %lld, d %lld, count %lld): see "
                "tpw_knn_mask_euclidean_supported", dtype, (long long)n, (long long)m, (long long)d, (long long)count);
    TPW_REQUIRE(x1 && x2 && aux1 && aux2 && mask && workspace, "null pointer");
    TPW_REQUIRE(aligned16(x1) && aligned16(x2) && aligned16(mask) && aligned16(workspace), "16-byte alignment required");
    hipStream_t s = as_stream(stream);
    uint64_t *cand = static_cast<uint64_t *>(workspace);
    if (dtype == TPW_F32)
        return dispatch_topk<float, false>(static_cast<const float *>(x1), static_cast<const float *>(x2), n, m, d,
                                           aux1, aux2, (int)count, cand, mask, s);
    return dispatch_topk<uint16_t, true>(static_cast<const uint16_t *>(x1), static_cast<const uint16_t *>(x2), n, m,
                                         d, aux1, aux2, (int)count, cand, mask, s);
}

extern "C" int tpw_pairwise_kernel(const void *x1, const void *x2, int dtype, int64_t batch,
                                   int64_t n, int64_t m, int64_t d, int kind, float gamma,
                                   float coef0, int degree, void *out, void *stream) {
    TPW_REQUIRE(dtype == TPW_F32 || dtype == TPW_BF16, "unsupported dtype %d", dtype);
    TPW_REQUIRE(kind == TPW_KER_POLYNOMIAL || kind == TPW_KER_SIGMOID, "unknown kernel %d", kind);
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    TPW_REQUIRE(cdiv(n, kTile) * cdiv(m, kTile) * batch <= 0x7fffffffLL, "output too large for one launch");
    hipStream_t s = as_stream(stream);
    KerParams kp;
    kp.gamma = gamma;
    kp.coef0 = coef0;
    kp.degree = degree;
    if (dtype == TPW_F32) {
        auto a = static_cast<const float *>(x1), b = static_cast<const float *>(x2);
        auto o = static_cast<float *>(out);
        if (kind == TPW_KER_POLYNOMIAL && degree >= 0 && degree <= 3)
            return launch_inner<float, kEpiPolySmall, float>(a, b, batch, n, m, d, nullptr, nullptr, o, s, nullptr,
                                                             1.0f, kp);
        return kind == TPW_KER_POLYNOMIAL
                   ? launch_inner<float, kEpiPoly, float>(a, b, batch, n, m, d, nullptr, nullptr, o, s, nullptr, 1.0f, kp)
                   : launch_inner<float, kEpiSigmoid, float>(a, b, batch, n, m, d, nullptr, nullptr, o, s, nullptr, 1.0f, kp);
    }
    auto a = static_cast<const uint16_t *>(x1), b = static_cast<const uint16_t *>(x2);
    auto o = static_cast<uint16_t *>(out);
    if (kind == TPW_KER_POLYNOMIAL && degree >= 0 && degree <= 3)
        return launch_inner<uint16_t, kEpiPolySmall, uint16_t>(a, b, batch, n, m, d, nullptr, nullptr, o, s, nullptr,
                                                               1.0f, kp);
    return kind == TPW_KER_POLYNOMIAL
               ? launch_inner<uint16_t, kEpiPoly, uint16_t>(a, b, batch, n, m, d, nullptr, nullptr, o, s, nullptr, 1.0f, kp)
               : launch_inner<uint16_t, kEpiSigmoid, uint16_t>(a, b, batch, n, m, d, nullptr, nullptr, o, s, nullptr, 1.0f, kp);
}
