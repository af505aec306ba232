// Bit-packed boolean pairwise reductions (hamming, jaccard, pw{and,or,xor,eq,ne}_{sum,mean}).
//
// Layout in HBM: each row of d bools is packed once into W = tpw_packed_words(d) uint32
// words (zero padding), so a 16384 x 128 bool operand becomes 16384 x 4 words (256 KiB)
// and stays resident in L2.  The reduction kernel then computes a 128 x 128 output tile
// per 256-thread block: both word panels are staged in LDS, every thread owns an 8 x 8
// register block and does one bitwise op plus one v_bcnt_u32_b32 (popcount-accumulate)
// per word pair.  The float32 output (the only large stream) is written with
// non-temporal 16-byte stores, 256 contiguous bytes per 16 lanes.
#include "common.hpp"
#include "tile_mfma.hpp"

namespace tpw {
namespace {

constexpr int kTile = 128;        // output rows and columns per block
constexpr int kChunkVec = 4;      // uint4 (4 words) per row and LDS chunk -> 16 words
constexpr int kThreads = 256;
constexpr uint32_t kFloatExactLimit = 1u << 24;  // float accumulator of ones saturates here

// 4 bool bytes (each 0 or 1) -> 4 bits, byte t -> bit t.  The multiplier places byte t's
// bit at position 21 + t; all 16 partial products land on distinct bits (no carries).
__device__ __forceinline__ uint32_t nibble(uint32_t v) {
    return (((v & 0x01010101u) * 0x00204081u) >> 21) & 0xFu;
}

__global__ void pack_bool_kernel(const uint8_t *__restrict__ x, int64_t rows, int64_t d,
                                 int64_t W, uint32_t *__restrict__ words, bool vec) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * W) return;
    int64_t r = t / W, w = t - r * W;
    int64_t k0 = w * 32;
    uint32_t word = 0;
    if (k0 < d) {
        const uint8_t *p = x + r * d + k0;
        int64_t cnt = d - k0 < 32 ? d - k0 : 32;
        if (vec && cnt == 32) {
            uint4 lo = *reinterpret_cast<const uint4 *>(p);
            uint4 hi = *reinterpret_cast<const uint4 *>(p + 16);
            word = nibble(lo.x) | nibble(lo.y) << 4 | nibble(lo.z) << 8 | nibble(lo.w) << 12 |
                   nibble(hi.x) << 16 | nibble(hi.y) << 20 | nibble(hi.z) << 24 |
                   nibble(hi.w) << 28;
        } else {
            for (int i = 0; i < cnt; ++i) word |= (uint32_t)(p[i] != 0) << i;
        }
    }
    words[t] = word;
}

__global__ void row_popcount_kernel(const uint32_t *__restrict__ words, int64_t rows,
                                    int64_t W, int32_t *__restrict__ pops) {
    int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const uint4 *p = reinterpret_cast<const uint4 *>(words + r * W);
    uint32_t c = 0;
    for (int64_t q = 0; q < W / 4; ++q) {
        uint4 v = p[q];
        c += __builtin_popcount(v.x) + __builtin_popcount(v.y) + __builtin_popcount(v.z) +
             __builtin_popcount(v.w);
    }
    pops[r] = (int32_t)c;
}

enum Epi { kSum = 0, kMean = 1, kJaccard = 2, kCountMetric = 16 };  // + TPW_BMET_*

__device__ __forceinline__ float sat_count(uint32_t c) {
    return (float)(c < kFloatExactLimit ? c : kFloatExactLimit);
}

// Bitwise select of a (where the lane's c is set) or b: a conditional around a divide compiles
// to an exec-masked branch per output, whose scalar bookkeeping costs more than the divide.
__device__ __forceinline__ float select_bits(bool c, float a, float b) {
    const uint32_t m = 0u - (uint32_t)c;
    return __uint_as_float((__float_as_uint(a) & m) | (__float_as_uint(b) & ~m));
}

// Output value from the tile's count (of OP) and, for jaccard and the count metrics, the two
// rows' popcounts.  The count metrics reproduce the reference's float32 composites over the
// separate pw*_sum passes (pairwise_metrics.cpp:224-243,339-399): every count is what a
// float accumulator of ones holds (exact below 2^24, then 2^24), and the float operations
// run in the composites' order, one rounding each, without contraction.  Counts are uint32
// (d < 2^31, so pa + pb < 2^32): 64-bit counts would double the epilogue's registers over
// the 64 outputs a thread owns and lower the occupancy of the whole kernel.
template <int OP, int EPI>
__device__ __forceinline__ float finish(uint32_t cnt, uint32_t pa, uint32_t pb, uint32_t d,
                                        double inv_d, float df, float inv_df) {
#pragma clang fp contract(off)
    if constexpr (EPI == kSum) {
        if constexpr (OP == TPW_BIT_EQ) cnt = d - cnt;
        return sat_count(cnt);
    } else if constexpr (EPI == kMean) {
        if constexpr (OP == TPW_BIT_EQ) cnt = d - cnt;
        // fl32(cnt / d) exactly: the double product is within 2^-52 of cnt/d, which is never
        // within 2^-48 of a float rounding midpoint for cnt <= d < 2^24, so the final rounding
        // is the correct one.
        if (inv_d > 0.0) return (float)((double)cnt * inv_d);
        return __fdiv_rn(sat_count(cnt), df);
    } else if constexpr (EPI == kJaccard) {
        const uint32_t sum = pa + pb;
        const float xf = sat_count(sum - 2u * cnt), of = sat_count(sum - cnt);
        return select_bits(of != 0.0f, __fdiv_rn(xf, of), 0.0f);
    } else {
        constexpr int MET = EPI - kCountMetric;
        const uint32_t n11 = cnt, x = pa + pb - 2u * n11;  // and, xor counts
        const float A = sat_count(n11), S = sat_count(x);
        if constexpr (MET == TPW_BMET_HAMMING) {  // pwne_mean
            if (inv_d > 0.0) return (float)((double)x * inv_d);
            return __fdiv_rn(S, df);
        } else if constexpr (MET == TPW_BMET_JACCARD) {  // prf_div(xor, or, "zero")
            const float O = sat_count(pa + pb - n11);
            return select_bits(O != 0.0f, __fdiv_rn(S, O), 0.0f);
        } else if constexpr (MET == TPW_BMET_DICE) {  // R / (2 and + R), R = xor
            return __fdiv_rn(S, 2.0f * A + S);
        } else if constexpr (MET == TPW_BMET_KULCZYNSKI1) {  // and / xor
            return __fdiv_rn(A, S);
        } else if constexpr (MET == TPW_BMET_KULSINSKI) {  // (xor - and + d) / (xor + d)
            const float num = (S - A) + df, den = S + df;
            return __fdiv_rn(num, den);
        } else if constexpr (MET == TPW_BMET_ROGERSTANIMOTO || MET == TPW_BMET_SOKALMICHENER) {
            const float R = 2.0f * S, E = sat_count(d - x);  // R / (eq + R)
            return __fdiv_rn(R, E + R);
        } else if constexpr (MET == TPW_BMET_RUSSELLRAO) {
            // (d - and) / d with ATen's GPU tensor / CPU-scalar divide: a multiply by the
            // float reciprocal computed on the host (inv_df = fl(1 / fl(d)))
            return (df - A) * inv_df;
        } else if constexpr (MET == TPW_BMET_SOKALSNEATH) {  // R / (and + R), R = 2 xor
            const float R = 2.0f * S;
            return __fdiv_rn(R, A + R);
        } else {  // yule: prf_div(2 hR, and * nor + hR, "zero"), hR = (a & ~b) * (~a & b)
            const float n10 = sat_count(pa - n11), n01 = sat_count(pb - n11);
            const float n00 = sat_count(d - (pa + pb - n11));
            const float hR = n10 * n01;
            const float num = 2.0f * hR;
            const float prod = A * n00;
            const float den = prod + hR;
            return select_bits(den != 0.0f, __fdiv_rn(num, den), 0.0f);
        }
    }
}

// Rows of at most kSmallRowLimit features: every count, popcount and composite numerator or
// denominator is an integer of at most 2^21, held exactly by a float, and the quotients of two
// such integers are correctly rounded by a short sequence instead of the general IEEE divide.
//
// div_count_r(x, o, y) for integers 0 <= x <= 2^22, 1 <= o <= 2^21 and y = (1/o)(1 + e1),
// |e1| <= u + 6u^2 (u = 2^-24): q0 = RN(x y) is within (x/o)(2u + 7u^2) of x/o; the residual
// r = x - o q0 is exact (a multiple of ulp(q0) below 4 o ulp(q0) < 2^24 ulp(q0)), so the pre-
// rounding value of fma(r, y, q0) is x/o + (x/o - q0) e1, within (x/o) 2.0001 u^2 of x/o.  For
// x/o in [2^e, 2^(e+1)) (e <= 21) the rounding midpoints are odd multiples of 2^(e-24) (and
// 2^e - 2^(e-25) below the binade), and |x/o - M 2^(e-24)| = |x 2^(24-e) - M o| / (o 2^(24-e))
// is at least 2^(e-24) / o unless zero; it is never zero (x/o = M 2^-j with M odd of 25 bits
// would make the odd part of o divide x, and x/o a 24-bit integer times a power of two).
// (x/o) 2.0001 u^2 < 2^(e+1) o 2.0001 u^2 <= 2^(e-24) / o holds for o <= 2^22 / 1.0001, so
// the final rounding is that of x/o itself: the result is the correctly rounded quotient,
// bit-identical to __fdiv_rn.  div_count makes y from the hardware reciprocal (within 1 ulp:
// |e0| <= 2u) and one Newton step, y = RN(y0 + y0 (1 - o y0)), whose error before rounding
// is below 6 u^2.
constexpr int64_t kSmallRowLimit = (int64_t)1 << 20;

__device__ __forceinline__ float div_count_r(float x, float o, float y) {
    const float q0 = x * y;
    const float r = __builtin_fmaf(-o, q0, x);
    return __builtin_fmaf(r, y, q0);
}

__device__ __forceinline__ float div_count(float x, float o) {
    const float y0 = __builtin_amdgcn_rcpf(o);
    const float y = __builtin_fmaf(__builtin_fmaf(-o, y0, 1.0f), y0, y0);
    return div_count_r(x, o, y);
}

// x / o as __fdiv_rn gives it, o = 0 included (x / 0 = +inf, 0 / 0 = NaN): both values formed,
// one selected.
__device__ __forceinline__ float div_count_z(float x, float o) {
    return select_bits(o == 0.0f, x * __builtin_inff(), div_count(x, o));
}

// finish<> for rows of at most kSmallRowLimit features, on float counts: c is the AND count
// (the fp32 MFMA accumulator, exact), pa and pb the two rows' popcounts, df = d and
// inv_df = RN(1 / d).  Every value is the one finish<> returns for the same counts, bit for
// bit: the integer steps are exact in float here, and the quotients are correctly rounded.
template <int OP, int EPI>
__device__ __forceinline__ float finish_small(float c, float pa, float pb, float df, float inv_df) {
#pragma clang fp contract(off)
    const float S = __builtin_fmaf(-2.0f, c, pa) + pb;  // xor count
    if constexpr (EPI == kSum || EPI == kMean) {
        float k;
        if constexpr (OP == TPW_BIT_AND) k = c;
        else if constexpr (OP == TPW_BIT_OR) k = (pa - c) + pb;
        else if constexpr (OP == TPW_BIT_EQ) k = __builtin_fmaf(2.0f, c, df - pa) - pb;
        else k = S;  // XOR, NE
        if constexpr (EPI == kSum) return k;
        else return div_count_r(k, df, inv_df);
    } else if constexpr (EPI == kJaccard) {
        return div_count(S, __builtin_fmaxf(S + c, 1.0f));  // or = 0 only with xor = 0: 0
    } else {
        constexpr int MET = EPI - kCountMetric;
        const float A = c;
        if constexpr (MET == TPW_BMET_HAMMING) {
            return div_count_r(S, df, inv_df);
        } else if constexpr (MET == TPW_BMET_JACCARD) {
            return div_count(S, __builtin_fmaxf(S + A, 1.0f));
        } else if constexpr (MET == TPW_BMET_DICE) {
            // 2A + S = 0 only with S = 0, and div_count(0, 0) is NaN as 0 / 0 is (the
            // reciprocal of 0 is inf, and 0 inf poisons the Newton step): no zero test
            return div_count(S, 2.0f * A + S);
        } else if constexpr (MET == TPW_BMET_KULCZYNSKI1) {
            return div_count_z(A, S);
        } else if constexpr (MET == TPW_BMET_KULSINSKI) {
            return div_count((S - A) + df, S + df);
        } else if constexpr (MET == TPW_BMET_ROGERSTANIMOTO || MET == TPW_BMET_SOKALMICHENER) {
            const float R = 2.0f * S;
            return div_count(R, (df - S) + R);
        } else if constexpr (MET == TPW_BMET_RUSSELLRAO) {
            return (df - A) * inv_df;
        } else if constexpr (MET == TPW_BMET_SOKALSNEATH) {
            const float R = 2.0f * S;
            return div_count(R, A + R);  // A + R = 0 only with R = 0: 0 / 0, as for dice
        } else {  // yule
            const float n10 = pa - A, n01 = pb - A;
            const float n00 = df - ((pa + pb) - A);
            const float hR = n10 * n01;
            const float num = 2.0f * hR;
            const float prod = A * n00;
            const float den = prod + hR;
            // d <= 2048: n10 + n01 + A + n00 = d bounds n10 n01 and A n00 by d^2 / 4 = 2^20, so
            // every product and sum is an exact integer (the fma's too), num <= 2^21 and
            // den <= 2^20, inside div_count's range.  den = 0 needs both of its terms 0, so
            // hR = 0 and num = 0: dividing by max(den, 1) gives that case its 0 without a
            // select.  Longer rows: products past 2^24 round, and the general divide.
            if (df <= 2048.0f) return div_count(num, __builtin_fmaxf(__builtin_fmaf(A, n00, hR), 1.0f));
            return select_bits(den != 0.0f, __fdiv_rn(num, den), 0.0f);
        }
    }
}

template <int OP>
__device__ __forceinline__ uint32_t bitop(uint32_t a, uint32_t b) {
    if constexpr (OP == TPW_BIT_AND) return a & b;
    else if constexpr (OP == TPW_BIT_OR) return a | b;
    else return a ^ b;  // XOR, NE, and EQ (counted as d - ne)
}

template <int OP>
__device__ __forceinline__ uint32_t popacc(uint32_t acc, uint4 a, uint4 b) {
    acc += __builtin_popcount(bitop<OP>(a.x, b.x));
    acc += __builtin_popcount(bitop<OP>(a.y, b.y));
    acc += __builtin_popcount(bitop<OP>(a.z, b.z));
    acc += __builtin_popcount(bitop<OP>(a.w, b.w));
    return acc;
}

// out tile (8 TY rows x 8 TX columns, TX TY = 256 threads) of batch blockIdx.z.  Thread
// (ty, tx) owns rows ty + TY i and columns 4 TX h + 4 tx + c (i < 8, h < 2, c < 4), so one
// float4 store instruction of a wave covers 64 / TX rows with 16 TX contiguous bytes each.
// CV uint4 (4 words) per row and LDS chunk.  128 x 128 (TX = 16) for general rows; 32 x 512
// (TX = 64) for rows of at most 8 words, where the output write is the whole cost and 2 KB
// contiguous per row and tile keep the DRAM pages open longer than 512 B.
template <int OP, int EPI, int TX, int CV>
__global__ __launch_bounds__(kThreads) void bool_reduce_kernel(
    const uint32_t *__restrict__ A, const uint32_t *__restrict__ Bw,
    const int32_t *__restrict__ popA, const int32_t *__restrict__ popB, int64_t n, int64_t m,
    int64_t W, int64_t d, double inv_d, float inv_df, float *__restrict__ out, bool vec_store) {
    constexpr bool kPops = EPI >= kJaccard;
    constexpr int TY = kThreads / TX, RT = 8 * TY, CT = 8 * TX;
    __shared__ uint4 As[RT][CV + 1];
    __shared__ uint4 Bs[CT][CV + 1];
    const int tid = threadIdx.x, tx = tid % TX, ty = tid / TX;
    const int64_t b = blockIdx.z;
    const int64_t row0 = (int64_t)blockIdx.y * RT, col0 = (int64_t)blockIdx.x * CT;
    const uint32_t *Ab = A + b * n * W;
    const uint32_t *Bb = Bw + b * m * W;

    uint32_t acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0;

    for (int64_t w0 = 0; w0 < W; w0 += 4 * CV) {
        const int q = (int)((W - w0) / 4 < CV ? (W - w0) / 4 : CV);
        for (int idx = tid; idx < RT * q; idx += kThreads) {
            const int r = idx / q, c = idx - r * q;
            const int64_t gr = row0 + r;
            uint4 u = {0u, 0u, 0u, 0u};
            if (gr < n) u = *reinterpret_cast<const uint4 *>(Ab + gr * W + w0 + 4 * c);
            As[r][c] = u;
        }
        for (int idx = tid; idx < CT * q; idx += kThreads) {
            const int r = idx / q, c = idx - r * q;
            const int64_t gc = col0 + r;
            uint4 v = {0u, 0u, 0u, 0u};
            if (gc < m) v = *reinterpret_cast<const uint4 *>(Bb + gc * W + w0 + 4 * c);
            Bs[r][c] = v;
        }
        __syncthreads();
        for (int c = 0; c < q; ++c) {
            uint4 a[8], bv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = As[ty + TY * i][c];
#pragma unroll
            for (int j = 0; j < 8; ++j) bv[j] = Bs[(j >> 2) * (4 * TX) + 4 * tx + (j & 3)][c];
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[i][j] = popacc<OP>(acc[i][j], a[i], bv[j]);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int64_t row = row0 + ty + TY * i;
        if (row >= n) continue;
        float *orow = out + (b * n + row) * m;
        uint32_t pa = 0;
        if constexpr (kPops) pa = (uint32_t)popA[b * n + row];
        const float df = (float)d;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t col = col0 + 4 * TX * h + 4 * tx;
            float v[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                uint32_t pb = 0;
                if constexpr (kPops) pb = col + c < m ? (uint32_t)popB[b * m + col + c] : 0u;
                v[c] = finish<OP, EPI>(acc[i][4 * h + c], pa, pb, (uint32_t)d, inv_d, df, inv_df);
            }
            if (vec_store && col + 3 < m) {
                floatx4 f = {v[0], v[1], v[2], v[3]};
                store_nt4(orow + col, f);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (col + c < m) store_nt(orow + col + c, v[c]);
            }
        }
    }
}

template <int OP, int EPI>
int launch_reduce(const uint32_t *a, const uint32_t *b, const int32_t *pa, const int32_t *pb,
                  int64_t batch, int64_t n, int64_t m, int64_t d, float *out, hipStream_t s) {
    const int64_t W = tpw_packed_words(d);
    const double inv_d = d < (int64_t)kFloatExactLimit ? 1.0 / (double)d : 0.0;
    const float inv_df = 1.0f / (float)d;  // as ATen's host-side reciprocal of a CPU scalar
    const bool vec_store = (m % 4 == 0) && aligned16(out);
    const LaunchEvents ev = launch_events("bool_reduce_kernel");
    if (W <= 8 && m > 256 && cdiv(n, 32) <= kMaxGridYZ) {
        dim3 grid((unsigned)cdiv(m, 512), (unsigned)cdiv(n, 32), (unsigned)batch);
        hipExtLaunchKernelGGL((bool_reduce_kernel<OP, EPI, 64, 2>), grid, dim3(kThreads), 0, s, ev.start, ev.stop, 0, a, b,
                           pa, pb, n, m, W, d, inv_d, inv_df, out, vec_store);
    } else {
        dim3 grid((unsigned)cdiv(m, kTile), (unsigned)cdiv(n, kTile), (unsigned)batch);
        hipExtLaunchKernelGGL((bool_reduce_kernel<OP, EPI, 16, kChunkVec>), grid, dim3(kThreads), 0, s, ev.start, ev.stop, 0,
                           a, b, pa, pb, n, m, W, d, inv_d, inv_df, out, vec_store);
    }
    return check_launch("bool_reduce_kernel");
}

// ---------------------------------------------------------------------------------------
// Bool bytes on the int8 matrix cores.  A torch.bool row is a 0/1 int8 vector, so the AND
// count of two rows is their int8 dot product: a 128 x 128 output tile is an int32 GEMM tile
// (v_mfma_i32_32x32x32_i8; 4 waves of 64 x 64 = 2 x 2 blocks of 32 x 32), and the other
// counts follow exactly from it and the two rows' popcounts: or = pa + pb - and,
// xor = ne = pa + pb - 2 and, eq = d - xor.  The epilogue is finish<> above, so results are
// those of the packed popcount kernel bit for bit.  Operands are staged in LDS in 128-byte
// chunks of each row (16-byte pad: 144-byte stride); lane (i + 32 h) feeds the MFMA bytes
// [64 h, 64 h + 64) of row i of a chunk as four 16-byte k pieces, A and B alike, so the k
// order inside a chunk is permuted identically on both sides and every dot product is
// unchanged.  The next chunk's global loads are issued before the current chunk's MFMAs.
constexpr int kBRowVec = 8;                // uint4 per 128-byte chunk row
constexpr int kBStride = kBRowVec + 1;     // in uint4
constexpr int kBStage = 68;                // floats per staged output row (64 + 4 pad)
typedef int int32x4 __attribute__((ext_vector_type(4)));
typedef int int32x16 __attribute__((ext_vector_type(16)));

// 16 bytes k .. k + 15 of row r of a [rows, d] byte matrix, zero past the row's end or the
// last row.  VEC: d % 16 == 0 and the base is 16-byte aligned.
template <bool VEC>
__device__ __forceinline__ uint4 load_bytes16(const uint8_t *__restrict__ x, int64_t rows, int64_t d,
                                              int64_t r, int64_t k) {
    uint4 v = {0u, 0u, 0u, 0u};
    if (r >= rows) return v;
    if constexpr (VEC) {
        if (k < d) v = *reinterpret_cast<const uint4 *>(x + r * d + k);
    } else {
        const uint8_t *p = x + r * d;
        uint32_t e[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t w = 0;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t kk = k + 4 * t + u;
                if (kk < d) w |= (uint32_t)p[kk] << (8 * u);
            }
            e[t] = w;
        }
        v = make_uint4(e[0], e[1], e[2], e[3]);
    }
    return v;
}

// The count of bitop<OP> (what the packed kernel's tile holds) from the AND count.
template <int OP, int EPI>
__device__ __forceinline__ uint32_t count_from_and(uint32_t c, uint32_t pa, uint32_t pb) {
    if constexpr (EPI >= kJaccard || OP == TPW_BIT_AND) return c;
    else if constexpr (OP == TPW_BIT_OR) return pa + pb - c;
    else return pa + pb - 2u * c;  // XOR, NE, and EQ (finish turns ne into d - ne)
}

// The AND counts of a 128 x 128 tile (the 32 x 32 MFMA accumulator layout: register r of lane
// l holds row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32) -> bitop counts -> the reference's
// float arithmetic -> the output.  Full tiles are staged per wave in the panels' LDS (free after
// the K loop's last barrier) and written as float4 rows; edge tiles element by element.
template <int OP, int EPI>
__device__ __forceinline__ void bool_epilogue(const int32x16 (&acc)[2][2], uint4 *smem, const uint32_t (&s_pop)[2][kTile],
                                              int64_t b, int64_t row0, int64_t col0, int64_t n, int64_t m, int64_t d,
                                              double inv_d, float inv_df, float *__restrict__ out, bool vec_store) {
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
    const int l32 = lane & 31, h = lane >> 5;
    const uint32_t du = (uint32_t)d;
    const float df = (float)d;
    uint32_t pbv[2];
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) pbv[ni] = s_pop[1][wc + ni * 32 + l32];
    const bool full = row0 + kTile <= n && col0 + kTile <= m;
    if (full && vec_store) {
        // each wave stages a 32 x 64 half of its tile in its own LDS slice (the operand panels
        // are free after the K loop's last barrier) and writes it as float4 rows, 16 lanes per
        // 256-byte segment
        float *stage = reinterpret_cast<float *>(smem) + wave * (32 * kBStage);
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
            // the popcounts of the lane's 16 rows: 4 groups of 4 consecutive rows
            uint4 paq[4];
#pragma unroll
            for (int g = 0; g < 4; ++g)
                paq[g] = *reinterpret_cast<const uint4 *>(&s_pop[0][wr + mi * 32 + 8 * g + 4 * h]);
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int rr = 8 * (r >> 2) + 4 * h + (r & 3);
                    const uint4 q4 = paq[r >> 2];
                    const uint32_t pav = (r & 3) == 0 ? q4.x : (r & 3) == 1 ? q4.y : (r & 3) == 2 ? q4.z : q4.w;
                    const uint32_t c = count_from_and<OP, EPI>((uint32_t)acc[mi][ni][r], pav, pbv[ni]);
                    stage[rr * kBStage + ni * 32 + l32] = finish<OP, EPI>(c, pav, pbv[ni], du, inv_d, df, inv_df);
                }
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes landed
            __builtin_amdgcn_wave_barrier();
            float *orow = out + (b * n + row0 + wr + mi * 32) * m + col0 + wc;
#pragma unroll
            for (int it = 0; it < 8; ++it) {
                const int rr = it * 4 + (lane >> 4), cc = (lane & 15) * 4;
                store_nt4(orow + (int64_t)rr * m + cc, *reinterpret_cast<const floatx4 *>(&stage[rr * kBStage + cc]));
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);  // reads done before the slice is rewritten
            __builtin_amdgcn_wave_barrier();
        }
        return;
    }
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const int64_t col = col0 + wc + ni * 32 + l32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rr = mi * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                const int64_t row = row0 + wr + rr;
                if (row < n && col < m) {
                    const uint32_t pav = s_pop[0][wr + rr];
                    const uint32_t c = count_from_and<OP, EPI>((uint32_t)acc[mi][ni][r], pav, pbv[ni]);
                    store_nt(out + (b * n + row) * m + col, finish<OP, EPI>(c, pav, pbv[ni], du, inv_d, df, inv_df));
                }
            }
        }
}

template <int OP, int EPI, bool VEC>
__global__ __launch_bounds__(kThreads, 2) void bool_mfma_kernel(
    const uint8_t *__restrict__ x1, const uint8_t *__restrict__ x2, const int32_t *__restrict__ popA,
    const int32_t *__restrict__ popB, int64_t n, int64_t m, int64_t d, double inv_d, float inv_df,
    float *__restrict__ out, int64_t tiles_n, int64_t tiles_m, int64_t total, bool vec_store) {
    // operand panels (As, Bs); after the K loop the same bytes stage the fp32 output
    __shared__ uint4 smem[2 * kTile * kBStride];
    uint4 *As = smem;
    uint4 *Bs = smem + kTile * kBStride;
    // popcounts of the tile's rows ([0]) and columns ([1])
    __shared__ __align__(16) uint32_t s_pop[2][kTile];

    int64_t b, tr, tc;
    xcd_tile_of(blockIdx.x, tiles_n, tiles_m, total, b, tr, tc);
    const int64_t row0 = tr * kTile, col0 = tc * kTile;
    const uint8_t *A = x1 + b * n * d;
    const uint8_t *B = x2 + b * m * d;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
    const int l32 = lane & 31, h = lane >> 5;
    {
        const int i = tid & (kTile - 1);
        if (tid < kTile) s_pop[0][i] = row0 + i < n ? (uint32_t)popA[b * n + row0 + i] : 0u;
        else s_pop[1][i] = col0 + i < m ? (uint32_t)popB[b * m + col0 + i] : 0u;
    }

    int32x16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0;

    const int64_t nchunks = (d + 127) / 128;  // d >= 1
    uint4 pa[4], pb[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int idx = tid + kThreads * q;
        const int r = idx >> 3, c = idx & 7;
        pa[q] = load_bytes16<VEC>(A, n, d, row0 + r, 16 * c);
        pb[q] = load_bytes16<VEC>(B, m, d, col0 + r, 16 * c);
    }
    for (int64_t kc = 0; kc < nchunks; ++kc) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int idx = tid + kThreads * q;
            const int r = idx >> 3, c = idx & 7;
            As[r * kBStride + c] = pa[q];
            Bs[r * kBStride + c] = pb[q];
        }
        __syncthreads();
        if (kc + 1 < nchunks) {
            const int64_t kb = (kc + 1) * 128;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int idx = tid + kThreads * q;
                const int r = idx >> 3, c = idx & 7;
                pa[q] = load_bytes16<VEC>(A, n, d, row0 + r, kb + 16 * c);
                pb[q] = load_bytes16<VEC>(B, m, d, col0 + r, kb + 16 * c);
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            int32x4 a[2], bv[2];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
                a[mi] = __builtin_bit_cast(int32x4, As[(wr + mi * 32 + l32) * kBStride + h * 4 + q]);
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
                bv[ni] = __builtin_bit_cast(int32x4, Bs[(wc + ni * 32 + l32) * kBStride + h * 4 + q]);
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[mi], bv[ni], acc[mi][ni], 0, 0, 0);
        }
        __syncthreads();
    }

    bool_epilogue<OP, EPI>(acc, smem, s_pop, b, row0, col0, n, m, d, inv_d, inv_df, out, vec_store);
}

// Set bytes per row of a [rows, d] bool matrix (one wave per row).  VEC (d % 16 == 0, 16-byte
// aligned rows): 16 bytes per lane and step; a bool byte is 0 or 1, so the popcount of a word
// of them is its number of true bytes.
__global__ void bool_row_counts_kernel(const uint8_t *__restrict__ x, int64_t rows, int64_t d,
                                       int32_t *__restrict__ counts, bool vec) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const uint8_t *p = x + row * d;
    uint32_t c = 0;
    if (vec) {
        for (int64_t k = 16 * (int64_t)lane; k < d; k += 1024) {
            const uint4 v = *reinterpret_cast<const uint4 *>(p + k);
            c += __builtin_popcount(v.x) + __builtin_popcount(v.y) + __builtin_popcount(v.z) +
                 __builtin_popcount(v.w);
        }
    } else {
        for (int64_t k = lane; k < d; k += 64) c += p[k] != 0;
    }
    for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
    if (lane == 0) counts[row] = (int32_t)c;
}

template <int OP, int EPI>
int launch_bool_mfma(const uint8_t *a, const uint8_t *b, const int32_t *pa, const int32_t *pb,
                     int64_t batch, int64_t n, int64_t m, int64_t d, float *out, hipStream_t s) {
    const int64_t tiles_n = cdiv(n, kTile), tiles_m = cdiv(m, kTile);
    const int64_t total = tiles_n * tiles_m * batch;
    const double inv_d = d < (int64_t)kFloatExactLimit ? 1.0 / (double)d : 0.0;
    const float inv_df = 1.0f / (float)d;  // as ATen's host-side reciprocal of a CPU scalar
    const bool vec = d % 16 == 0 && aligned16(a) && aligned16(b);
    const bool vec_store = m % 4 == 0 && aligned16(out);
    auto kernel = vec ? bool_mfma_kernel<OP, EPI, true> : bool_mfma_kernel<OP, EPI, false>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)total), dim3(kThreads), 0, s, a, b, pa, pb, n, m, d,
                       inv_d, inv_df, out, tiles_n, tiles_m, total, vec_store);
    return check_launch("bool_mfma_kernel");
}

int check_reduce_args(const uint32_t *a, const uint32_t *b, int64_t batch, int64_t n, int64_t m,
                      int64_t d, float *out) {
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 1, "invalid sizes batch=%lld n=%lld m=%lld d=%lld",
                (long long)batch, (long long)n, (long long)m, (long long)d);
    TPW_REQUIRE(cdiv(n, kTile) <= kMaxGridYZ && batch <= kMaxGridYZ,
                "too many rows (n=%lld) or batches (%lld)", (long long)n, (long long)batch);
    TPW_REQUIRE(d <= (int64_t)0x7fffffff, "d=%lld exceeds the 32-bit count range", (long long)d);
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(a && b && out, "null pointer");
    TPW_REQUIRE(aligned16(a) && aligned16(b), "packed words must be 16-byte aligned");
    return TPW_OK;
}


// ---------------------------------------------------------------- bool rows as fp4 (e2m1)
// A bool encoded as the fp4 value 0.0 or 1.0 (nibble 0x0 / 0x2) makes the AND count of two
// rows their fp4 dot product, which the gfx950 scaled MFMA computes exactly
// (v_mfma_scale_f32_32x32x64_f8f6f4, scales 1.0, fp32 accumulation: products are 0 or 1 and
// every partial sum is an integer below 2^24).  Half the bytes of the int8 layout and half its
// matrix-core cycles per feature.  Rows are 128-byte multiples (256 features), zero-padded;
// feature 2j is the low nibble of byte j.  A 128-byte chunk goes from global memory straight
// into LDS (global_load_lds_dwordx4, the 144-byte padded row layout of the int8 kernel); lane
// (i + 32 h) feeds the MFMA the 16-byte pieces h * 4 + q of row i, A and B alike.
typedef int int32x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;
constexpr int kFp4Slots = 9;  // 2 panels x 128 rows x 9 slots / 4 waves / 64 lanes

// One wave per row: each lane packs 32 features (16 output bytes) per step and counts them.
__global__ void pack_fp4_kernel(const uint8_t *__restrict__ x, int64_t rows, int64_t d, int64_t rb,
                                uint8_t *__restrict__ fp4, int32_t *__restrict__ counts, bool vec) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const uint8_t *p = x + row * d;
    uint8_t *q = fp4 + row * rb;
    uint32_t c = 0;
    for (int64_t k = 32 * (int64_t)lane; k < 2 * rb; k += 2048) {  // k: first feature of the piece
        uint32_t v[8];  // 32 bool bytes, 4 per word
        if (vec && k + 32 <= d) {
            const uint4 lo = *reinterpret_cast<const uint4 *>(p + k);
            const uint4 hi = *reinterpret_cast<const uint4 *>(p + k + 16);
            v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
            v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                uint32_t w = 0;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int64_t kk = k + 4 * t + u;
                    if (kk < d) w |= (uint32_t)p[kk] << (8 * u);
                }
                v[t] = w;
            }
        }
        uint32_t o[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t pair = 0;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                // bytes f0..f3 (bit 0 each) -> nibbles 0x2 at bits 1, 5, 9, 13
                const uint32_t w = v[2 * t + e] & 0x01010101u;
                c += __builtin_popcount(w);
                const uint32_t nib = ((w << 1) & 0x2u) | ((w >> 3) & 0x20u) | ((w >> 7) & 0x200u) | ((w >> 11) & 0x2000u);
                pair |= nib << (16 * e);
            }
            o[t] = pair;
        }
        *reinterpret_cast<uint4 *>(q + k / 2) = make_uint4(o[0], o[1], o[2], o[3]);
    }
    for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
    if (lane == 0) counts[row] = (int32_t)c;
}

template <int OP, int EPI>
__global__ __launch_bounds__(kThreads, 2) void bool_fp4_kernel(
    const uint8_t *__restrict__ x1, const uint8_t *__restrict__ x2, const int32_t *__restrict__ popA,
    const int32_t *__restrict__ popB, int64_t n, int64_t m, int64_t d, int64_t rb, double inv_d, float inv_df,
    float *__restrict__ out, int64_t tiles_n, int64_t tiles_m, int64_t total, bool vec_store) {
    // operand panels (As, Bs); after the K loop the same bytes stage the fp32 output
    __shared__ uint4 smem[2 * kTile * kBStride];
    const uint4 *As = smem;
    const uint4 *Bs = smem + kTile * kBStride;
    __shared__ __align__(16) uint32_t s_pop[2][kTile];

    int64_t b, tr, tc;
    xcd_tile_of(blockIdx.x, tiles_n, tiles_m, total, b, tr, tc);
    const int64_t row0 = tr * kTile, col0 = tc * kTile;
    const uint8_t *A = x1 + b * n * rb;
    const uint8_t *B = x2 + b * m * rb;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
    const int l32 = lane & 31, h = lane >> 5;
    {
        const int i = tid & (kTile - 1);
        if (tid < kTile) s_pop[0][i] = row0 + i < n ? (uint32_t)popA[b * n + row0 + i] : 0u;
        else s_pop[1][i] = col0 + i < m ? (uint32_t)popB[b * m + col0 + i] : 0u;
    }
    floatx16 facc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) facc[mi][ni][r] = 0.0f;

    // byte offsets (from the panel's batch base) of this lane's slot in each of its 9 wave
    // loads: slot s -> panel s / 1152, row (s % 1152) / 9, piece (s % 1152) % 9; the pad slot
    // loads piece 7 again (never read), rows past the edge load the last row (never stored)
    int32_t off[kFp4Slots];
#pragma unroll
    for (int j = 0; j < kFp4Slots; ++j) {
        const int sl = (wave * kFp4Slots + j) * 64 + lane;
        const int panel = sl >= kTile * kBStride;
        const int s2 = sl - panel * kTile * kBStride;
        const int r = s2 / kBStride, c0 = s2 - r * kBStride;
        const int c = c0 == kBRowVec ? kBRowVec - 1 : c0;
        const int64_t lim = panel ? m : n;
        int64_t row = (panel ? col0 : row0) + r;
        row = row < lim ? row : lim - 1;
        off[j] = (int32_t)(row * rb + c * 16);
    }
    const int64_t nchunks = rb / 128;
    for (int64_t kc = 0; kc < nchunks; ++kc) {
        const int64_t kb = kc * 128;
#pragma unroll
        for (int j = 0; j < kFp4Slots; ++j) {
            const int first = (wave * kFp4Slots + j) * 64;  // wave-uniform LDS slot
            const uint8_t *src = (first >= kTile * kBStride ? B : A) + kb + off[j];
            __builtin_amdgcn_global_load_lds((global_void *)src, (lds_void *)(smem + first), 16, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's slots have landed
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            int32x8 a[2], bv[2];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) {
                const uint4 v = As[(wr + mi * 32 + l32) * kBStride + h * 4 + q];
                a[mi] = int32x8{(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
            }
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const uint4 v = Bs[(wc + ni * 32 + l32) * kBStride + h * 4 + q];
                bv[ni] = int32x8{(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
            }
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)  // formats 4 / 4: fp4 e2m1; E8M0 scales 127 = 1.0
                    facc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[mi], bv[ni], facc[mi][ni], 4, 4,
                                                                                  0, 127, 0, 127);
        }
        __syncthreads();
    }
    int32x16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = (int)facc[mi][ni][r];
    bool_epilogue<OP, EPI>(acc, smem, s_pop, b, row0, col0, n, m, d, inv_d, inv_df, out, vec_store);
}

// The tile kernel of tile_mfma.hpp on the fp4 rows (every 128-byte chunk is full by
// construction): transposed scaled products, the counts finished per element while the tile is
// staged, float4 row segments out (dword rows when m % 4 != 0).  Needs a 16-byte aligned
// output and rows * row bytes < 2^32.
// Output stores of the tile kernels: plain stores, which let the L2 merge the waves' 256-byte
// row pieces (32768^2 x 1024 bits: pwxor_sum 0.95 -> 0.83 ms, hamming 0.96 -> 0.86 ms, jaccard
// 0.97 -> 0.91 ms), except for yule, whose epilogue is the longest and which runs faster with
// non-temporal stores (general IEEE divide: 1.13 -> 1.09 ms; short divide: yule / hamming 1.25
// -> 1.18).
template <int EPI>
constexpr bool kStoreNT = EPI == kCountMetric + TPW_BMET_YULE;

// Before the barrier that ends the K loop: rows of at most kSmallRowLimit features turn the
// tile's popcounts into floats in place (2 kT = kThreads entries, one per thread).
__device__ __forceinline__ void pops_to_float(bool small, uint32_t *s_pop) {
    static_assert(2 * tile::kT == tile::kThreads, "one popcount per thread");
    if (small) s_pop[threadIdx.x] = __float_as_uint((float)s_pop[threadIdx.x]);
}

// The output of the fp4 / bit tile kernels from their fp32 AND-count accumulators (transposed
// products: register 4 g + e of lane l32 + 32 h in block (mi, ni) is row wr + 32 mi + l32,
// column wc + 32 ni + 8 g + 4 h + e of the tile).  Rows of at most kSmallRowLimit features
// finish in float (finish_small, popcounts already floats in s_pop), longer rows on integer
// counts (finish); both give the same bits.  Any m: rows of m % 4 != 0 floats are written a
// dword per lane (the ragged mode of tile::store_tile), a separate instantiation (RAGGED) so
// that the aligned kernels' code is unchanged by it.
template <int OP, int EPI, bool RAGGED>
__device__ __forceinline__ void bool_tile_store(bool small, const floatx16 (&facc)[2][2], uint4 *smem,
                                                const uint32_t *s_pop, int wr, int wc, int l32, int h, int64_t d,
                                                double inv_d, float inv_df, float *__restrict__ out, int64_t b,
                                                int64_t row0, int64_t col0, int64_t n, int64_t m) {
    using tile::kT;
    const float df = (float)d;
    if (small) {
        float pav[2];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) pav[mi] = __uint_as_float(s_pop[wr + mi * 32 + l32]);
        tile::store_tile<float, kStoreNT<EPI>>(
            smem,
            [&](int mi, int ni, int g) {
                const uint4 pb = *reinterpret_cast<const uint4 *>(&s_pop[kT + wc + ni * 32 + 8 * g + 4 * h]);
                const float pbe[4] = {__uint_as_float(pb.x), __uint_as_float(pb.y), __uint_as_float(pb.z),
                                      __uint_as_float(pb.w)};
                floatx4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = finish_small<OP, EPI>(facc[mi][ni][4 * g + e], pav[mi], pbe[e], df, inv_df);
                return o;
            },
            out, b, row0, col0, n, m, RAGGED);
        return;
    }
    const uint32_t du = (uint32_t)d;
    uint32_t pav[2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) pav[mi] = s_pop[wr + mi * 32 + l32];
    tile::store_tile<float, kStoreNT<EPI>>(
        smem,
        [&](int mi, int ni, int g) {
            const uint4 pb = *reinterpret_cast<const uint4 *>(&s_pop[kT + wc + ni * 32 + 8 * g + 4 * h]);
            const uint32_t pbe[4] = {pb.x, pb.y, pb.z, pb.w};
            floatx4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t c = count_from_and<OP, EPI>((uint32_t)facc[mi][ni][4 * g + e], pav[mi], pbe[e]);
                o[e] = finish<OP, EPI>(c, pav[mi], pbe[e], du, inv_d, df, inv_df);
            }
            return o;
        },
        out, b, row0, col0, n, m, RAGGED);
}

template <int OP, int EPI, bool RAGGED>
__global__ __launch_bounds__(tile::kThreads, 4) void bool_fp4_tile_kernel(
    const uint8_t *__restrict__ x1, const uint8_t *__restrict__ x2, const int32_t *__restrict__ popA,
    const int32_t *__restrict__ popB, int64_t n, int64_t m, int64_t d, int64_t rb, double inv_d, float inv_df,
    float *__restrict__ out, int64_t tiles_n, int64_t tiles_m, int64_t total) {
    using namespace tile;
    __shared__ uint4 smem[kBuf];
    __shared__ __align__(16) uint32_t s_pop[2 * kT];  // row counts, then column counts
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
    const int l32 = lane & 31, h = lane >> 5;

    int64_t b, tr, tc;
    xcd_tile_of(blockIdx.x, tiles_n, tiles_m, total, b, tr, tc);
    const int64_t row0 = tr * kT, col0 = tc * kT;
    const uint8_t *A = x1 + b * n * rb;
    const uint8_t *B = x2 + b * m * rb;
    dma_tile_rows(popA + b * n, popB + b * m, true, wave, lane, row0, col0, n, m, s_pop);
    uint32_t off[kSlots];
    dma_offsets(off, wave, lane, row0, col0, n, m, rb);
    dma_chunk(A, B, off, wave, 0, smem);

    floatx16 facc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) facc[mi][ni][r] = 0.0f;

    const int nchunks = (int)(rb / 128);
    for (int kc = 0; kc < nchunks; ++kc) {
        if (kc > 0) {
            barrier_lds();  // every wave is done with chunk kc - 1
            dma_chunk(A, B, off, wave, (int64_t)kc * 128, smem);
        }
        barrier_all();  // chunk kc (and, the first time, the counts) has landed
        const uint4 *As = smem, *Bs = smem + kPanel;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int c = h * 4 + q;
            int32x8 a[2], bv[2];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) {
                const uint4 v = piece(As, wr + mi * 32 + l32, c);
                a[mi] = int32x8{(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
            }
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const uint4 v = piece(Bs, wc + ni * 32 + l32, c);
                bv[ni] = int32x8{(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
            }
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)  // transposed; formats 4 / 4: fp4 e2m1, E8M0 scales 127 = 1.0
                    facc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bv[ni], a[mi], facc[mi][ni], 4, 4,
                                                                                  0, 127, 0, 127);
        }
    }
    const bool small = d <= kSmallRowLimit;
    pops_to_float(small, s_pop);
    barrier_lds();  // the operand buffer becomes the output stage
    bool_tile_store<OP, EPI, RAGGED>(small, facc, smem, s_pop, wr, wc, l32, h, d, inv_d, inv_df, out, b, row0, col0, n, m);
}

// The tile kernel of tile_mfma.hpp on bit-packed rows (W uint32 words per row, W % 4 == 0,
// zero bits past d): a 128-byte chunk of a row is 1024 features, a quarter of the operand
// bytes the fp4 rows take, and each lane widens the bits it feeds the MFMA into fp4 e2m1
// nibbles in registers.  Lane (l32 + 32 h) reads logical piece 2 p + h (4 words) of its rows
// for pair p of the chunk and feeds word t of it to step t: bit 4 i + e of the word becomes
// nibble i of operand dword e (0x2 = 1.0 or 0), the same permutation of the features on both
// sides, so every AND count is unchanged.  A partial last chunk (W % 32 != 0) loads an
// in-row piece into the slots past the row's end and zeroes them in LDS before use.  Counts, popcounts and the epilogue are those of
// bool_fp4_tile_kernel, so the outputs are the same bit for bit.  Needs d < 2^24, a 16-byte
// aligned output and rows * W * 4 < 2^32.
template <int OP, int EPI, bool RAGGED>
__global__ __launch_bounds__(tile::kThreads, 4) void bool_bits_tile_kernel(
    const uint32_t *__restrict__ x1, const uint32_t *__restrict__ x2, const int32_t *__restrict__ popA,
    const int32_t *__restrict__ popB, int64_t n, int64_t m, int64_t d, int64_t W, double inv_d, float inv_df,
    float *__restrict__ out, int64_t tiles_n, int64_t tiles_m, int64_t total) {
    using namespace tile;
    __shared__ uint4 smem[kBuf];
    __shared__ __align__(16) uint32_t s_pop[2 * kT];  // row counts, then column counts
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
    const int l32 = lane & 31, h = lane >> 5;

    int64_t b, tr, tc;
    xcd_tile_of(blockIdx.x, tiles_n, tiles_m, total, b, tr, tc);
    const int64_t row0 = tr * kT, col0 = tc * kT;
    const int64_t rb = W * 4;
    const uint8_t *A = reinterpret_cast<const uint8_t *>(x1 + b * n * W);
    const uint8_t *B = reinterpret_cast<const uint8_t *>(x2 + b * m * W);
    dma_tile_rows(popA + b * n, popB + b * m, true, wave, lane, row0, col0, n, m, s_pop);
    uint32_t off[kSlots];
    dma_offsets(off, wave, lane, row0, col0, n, m, rb);
    const int nchunks = (int)((W + 31) / 32);
    const int vp = (int)(W - 32 * (int64_t)(nchunks - 1)) / 4;  // pieces of the last chunk, 1..8
    // last chunk: slot j of this lane holds logical piece swz(r, s & 7) of its row; past the
    // row's end it loads the chunk's piece 0 instead (in bounds) and is zeroed after landing
    uint32_t bad = 0;
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int sl = (wave * kSlots + j) * 64 + lane;
        bad |= (uint32_t)(swz((sl >> 3) & (kT - 1), sl & 7) >= vp) << j;
    }
    auto dma = [&](int kc) {
        const int64_t kb = (int64_t)kc * 128;
        const bool last = kc == nchunks - 1;
#pragma unroll
        for (int j = 0; j < kSlots; ++j) {
            const int first = (wave * kSlots + j) * 64;  // the wave's 64 slots lie in one panel
            const int sl = first + lane;
            const uint32_t o = (last && ((bad >> j) & 1)) ? off[j] - swz((sl >> 3) & (kT - 1), sl & 7) * 16 : off[j];
            dma16((first >= kPanel ? B : A) + kb, o, lds_addr(smem + first));
        }
    };
    dma(0);

    floatx16 facc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) facc[mi][ni][r] = 0.0f;

    const uint4 *As = smem, *Bs = smem + kPanel;
    // piece pair p of the chunk in LDS: 4 steps of 64 features
    auto pair = [&](int p) {
        uint4 a[2], bv[2];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) a[mi] = piece(As, wr + mi * 32 + l32, 2 * p + h);
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) bv[ni] = piece(Bs, wc + ni * 32 + l32, 2 * p + h);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int32x8 ax[2], bx[2];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) {
                const uint32_t x = t == 0 ? a[mi].x : t == 1 ? a[mi].y : t == 2 ? a[mi].z : a[mi].w;
                ax[mi] = int32x8{(int)((x << 1) & 0x22222222u), (int)(x & 0x22222222u), (int)((x >> 1) & 0x22222222u),
                                 (int)((x >> 2) & 0x22222222u), 0, 0, 0, 0};
            }
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const uint32_t x = t == 0 ? bv[ni].x : t == 1 ? bv[ni].y : t == 2 ? bv[ni].z : bv[ni].w;
                bx[ni] = int32x8{(int)((x << 1) & 0x22222222u), (int)(x & 0x22222222u), (int)((x >> 1) & 0x22222222u),
                                 (int)((x >> 2) & 0x22222222u), 0, 0, 0, 0};
            }
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)  // transposed; formats 4 / 4: fp4 e2m1, E8M0 scales 127 = 1.0
                    facc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bx[ni], ax[mi], facc[mi][ni], 4,
                                                                                  4, 0, 127, 0, 127);
        }
    };
    for (int kc = 0; kc < nchunks; ++kc) {
        if (kc > 0) {
            barrier_lds();  // every wave is done with chunk kc - 1
            dma(kc);
        }
        barrier_all();  // chunk kc (and, the first time, the counts) has landed
        if (kc == nchunks - 1 && vp < 8) {
            // the partial last chunk: zero the slots past the rows' end (they add nothing)
#pragma unroll
            for (int j = 0; j < kSlots; ++j)
                if ((bad >> j) & 1) smem[(wave * kSlots + j) * 64 + lane] = make_uint4(0, 0, 0, 0);
            barrier_lds();
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) pair(p);
    }
    const bool small = d <= kSmallRowLimit;
    pops_to_float(small, s_pop);
    barrier_lds();  // the operand buffer becomes the output stage
    bool_tile_store<OP, EPI, RAGGED>(small, facc, smem, s_pop, wr, wc, l32, h, d, inv_d, inv_df, out, b, row0, col0, n, m);
}

// Whether bool_bits_tile_kernel takes these packed rows (W words per row) and output.
bool bits_tile_fits(const uint32_t *a, const uint32_t *b, const int32_t *pa, const int32_t *pb, int64_t n,
                    int64_t m, int64_t d, int64_t W, const float *out) {
    return pa && pb && d >= 1 && d < (int64_t)kFloatExactLimit && W % 4 == 0 && W * 32 >= d && aligned16(a) &&
           aligned16(b) && aligned16(out) && (n > m ? n : m) * W * 4 < ((int64_t)1 << 32);
}

// Packed rows with their popcounts: the bit tile kernel where it fits, for the count metrics
// at any d and for the reductions over more than 256 features; else the popcount reduce kernel.
// Short rows' reductions write faster from the popcount kernel's 2 KB output row runs; their
// count metrics are faster on the tile kernel's float epilogue (16384^2 x 128: jaccard 0.287 ->
// 0.220 ms, dice 0.286 -> 0.230 ms).
template <int OP, int EPI>
int launch_counts(const uint32_t *a, const uint32_t *b, const int32_t *pa, const int32_t *pb, int64_t batch,
                  int64_t n, int64_t m, int64_t d, float *out, hipStream_t s) {
    const int64_t W = tpw_packed_words(d);
    if ((d > 256 || EPI >= kJaccard) && bits_tile_fits(a, b, pa, pb, n, m, d, W, out)) {
        const int64_t tiles_n = cdiv(n, kTile), tiles_m = cdiv(m, kTile);
        const int64_t total = tiles_n * tiles_m * batch;
        const double inv_d = 1.0 / (double)d;
        const float inv_df = 1.0f / (float)d;
        const LaunchEvents ev = launch_events("bool_bits_tile_kernel");
        if (m % 4 == 0)
            hipExtLaunchKernelGGL((bool_bits_tile_kernel<OP, EPI, false>), dim3((unsigned)total), dim3(tile::kThreads), 0,
                               s, ev.start, ev.stop, 0, a, b, pa, pb, n, m, d, W, inv_d, inv_df, out, tiles_n, tiles_m, total);
        else
            hipExtLaunchKernelGGL((bool_bits_tile_kernel<OP, EPI, true>), dim3((unsigned)total), dim3(tile::kThreads), 0,
                               s, ev.start, ev.stop, 0, a, b, pa, pb, n, m, d, W, inv_d, inv_df, out, tiles_n, tiles_m, total);
        return check_launch("bool_bits_tile_kernel");
    }
    return launch_reduce<OP, EPI>(a, b, pa, pb, batch, n, m, d, out, s);
}

int64_t fp4_row_bytes(int64_t d) { return (d + 255) / 256 * 128; }

template <int OP, int EPI>
int launch_bool_fp4(const uint8_t *a, const uint8_t *b, const int32_t *pa, const int32_t *pb, int64_t batch,
                    int64_t n, int64_t m, int64_t d, float *out, hipStream_t s) {
    const int64_t tiles_n = cdiv(n, kTile), tiles_m = cdiv(m, kTile);
    const int64_t total = tiles_n * tiles_m * batch;
    const double inv_d = d < (int64_t)kFloatExactLimit ? 1.0 / (double)d : 0.0;
    const float inv_df = 1.0f / (float)d;
    const bool vec_store = m % 4 == 0 && aligned16(out);
    if (aligned16(out) && (n > m ? n : m) * fp4_row_bytes(d) < ((int64_t)1 << 32)) {
        if (m % 4 == 0)
            hipLaunchKernelGGL((bool_fp4_tile_kernel<OP, EPI, false>), dim3((unsigned)total), dim3(tile::kThreads), 0,
                               s, a, b, pa, pb, n, m, d, fp4_row_bytes(d), inv_d, inv_df, out, tiles_n, tiles_m,
                               total);
        else
            hipLaunchKernelGGL((bool_fp4_tile_kernel<OP, EPI, true>), dim3((unsigned)total), dim3(tile::kThreads), 0,
                               s, a, b, pa, pb, n, m, d, fp4_row_bytes(d), inv_d, inv_df, out, tiles_n, tiles_m,
                               total);
        return check_launch("bool_fp4_tile_kernel");
    }
    hipLaunchKernelGGL((bool_fp4_kernel<OP, EPI>), dim3((unsigned)total), dim3(kThreads), 0, s, a, b, pa, pb, n, m,
                       d, fp4_row_bytes(d), inv_d, inv_df, out, tiles_n, tiles_m, total, vec_store);
    return check_launch("bool_fp4_kernel");
}

}  // namespace
}  // namespace tpw

using namespace tpw;

extern "C" int64_t tpw_packed_words(int64_t d) { return ((d + 31) / 32 + 3) / 4 * 4; }

extern "C" int tpw_pack_bool_rows(const uint8_t *x, int64_t rows, int64_t d, uint32_t *words,
                                  int32_t *row_popcounts, void *stream) {
    TPW_REQUIRE(rows >= 0 && d >= 1, "invalid sizes rows=%lld d=%lld", (long long)rows,
                (long long)d);
    if (rows == 0) return TPW_OK;
    TPW_REQUIRE(x && words, "null pointer");
    TPW_REQUIRE(aligned16(words), "words must be 16-byte aligned");
    const int64_t W = tpw_packed_words(d);
    const bool vec = (d % 16 == 0) && aligned16(x);
    const int64_t total = rows * W;
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(pack_bool_kernel, dim3((unsigned)cdiv(total, 256)), dim3(256), 0, s, x,
                       rows, d, W, words, vec);
    int rc = check_launch("pack_bool_kernel");
    if (rc != TPW_OK || !row_popcounts) return rc;
    hipLaunchKernelGGL(row_popcount_kernel, dim3((unsigned)cdiv(rows, 256)), dim3(256), 0, s,
                       words, rows, W, row_popcounts);
    return check_launch("row_popcount_kernel");
}

extern "C" int tpw_bool_pairwise_reduce(const uint32_t *x1w, const uint32_t *x2w, int64_t batch,
                                        int64_t n, int64_t m, int64_t d, int op, int reduction,
                                        float *out, void *stream) {
    int rc = check_reduce_args(x1w, x2w, batch, n, m, d, out);
    if (rc != TPW_OK) return rc;
    TPW_REQUIRE(op >= TPW_BIT_AND && op <= TPW_BIT_NE, "unknown bit op %d", op);
    TPW_REQUIRE(reduction == TPW_RED_SUM || reduction == TPW_RED_MEAN, "unknown reduction %d",
                reduction);
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    hipStream_t s = as_stream(stream);
#define TPW_CASE(OPC)                                                                         \
    case OPC:                                                                                 \
        return reduction == TPW_RED_SUM                                                       \
                   ? launch_reduce<OPC, kSum>(x1w, x2w, nullptr, nullptr, batch, n, m, d, out, s) \
                   : launch_reduce<OPC, kMean>(x1w, x2w, nullptr, nullptr, batch, n, m, d, out, s);
    switch (op) {
        TPW_CASE(TPW_BIT_AND)
        TPW_CASE(TPW_BIT_OR)
        TPW_CASE(TPW_BIT_XOR)
        TPW_CASE(TPW_BIT_EQ)
        default:
            // NE counts exactly like XOR on bits
            return reduction == TPW_RED_SUM
                       ? launch_reduce<TPW_BIT_XOR, kSum>(x1w, x2w, nullptr, nullptr, batch, n, m, d, out, s)
                       : launch_reduce<TPW_BIT_XOR, kMean>(x1w, x2w, nullptr, nullptr, batch, n, m, d, out, s);
    }
#undef TPW_CASE
}

extern "C" int tpw_bool_pairwise_reduce_counted(const uint32_t *x1w, const uint32_t *x2w, const int32_t *pop1,
                                                const int32_t *pop2, int64_t batch, int64_t n, int64_t m, int64_t d,
                                                int op, int reduction, float *out, void *stream) {
    int rc = check_reduce_args(x1w, x2w, batch, n, m, d, out);
    if (rc != TPW_OK) return rc;
    TPW_REQUIRE(op >= TPW_BIT_AND && op <= TPW_BIT_NE, "unknown bit op %d", op);
    TPW_REQUIRE(reduction == TPW_RED_SUM || reduction == TPW_RED_MEAN, "unknown reduction %d",
                reduction);
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(pop1 && pop2, "null popcount pointer");
    hipStream_t s = as_stream(stream);
#define TPW_CASE(OPC, K)                                                                                  \
    case OPC:                                                                                             \
        return reduction == TPW_RED_SUM                                                                   \
                   ? launch_counts<K, kSum>(x1w, x2w, pop1, pop2, batch, n, m, d, out, s)                  \
                   : launch_counts<K, kMean>(x1w, x2w, pop1, pop2, batch, n, m, d, out, s);
    switch (op) {
        TPW_CASE(TPW_BIT_AND, TPW_BIT_AND)
        TPW_CASE(TPW_BIT_OR, TPW_BIT_OR)
        TPW_CASE(TPW_BIT_XOR, TPW_BIT_XOR)
        TPW_CASE(TPW_BIT_EQ, TPW_BIT_EQ)
        default:
            // NE counts exactly like XOR on bits
            return reduction == TPW_RED_SUM
                       ? launch_counts<TPW_BIT_XOR, kSum>(x1w, x2w, pop1, pop2, batch, n, m, d, out, s)
                       : launch_counts<TPW_BIT_XOR, kMean>(x1w, x2w, pop1, pop2, batch, n, m, d, out, s);
    }
#undef TPW_CASE
}

extern "C" int tpw_jaccard_bool(const uint32_t *x1w, const uint32_t *x2w, const int32_t *pop1,
                                const int32_t *pop2, int64_t batch, int64_t n, int64_t m,
                                int64_t d, float *out, void *stream) {
    int rc = check_reduce_args(x1w, x2w, batch, n, m, d, out);
    if (rc != TPW_OK) return rc;
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(pop1 && pop2, "null popcount pointer");
    return launch_counts<TPW_BIT_AND, kJaccard>(x1w, x2w, pop1, pop2, batch, n, m, d, out, as_stream(stream));
}

extern "C" int tpw_bool_count_metric(const uint32_t *x1w, const uint32_t *x2w, const int32_t *pop1,
                                     const int32_t *pop2, int64_t batch, int64_t n, int64_t m,
                                     int64_t d, int metric, float *out, void *stream) {
    int rc = check_reduce_args(x1w, x2w, batch, n, m, d, out);
    if (rc != TPW_OK) return rc;
    TPW_REQUIRE(metric >= TPW_BMET_HAMMING && metric <= TPW_BMET_YULE, "unknown metric %d", metric);
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(pop1 && pop2, "null popcount pointer");
    hipStream_t s = as_stream(stream);
#define TPW_MET(CODE)                                                                             \
    case CODE:                                                                                    \
        return launch_counts<TPW_BIT_AND, kCountMetric + CODE>(x1w, x2w, pop1, pop2, batch, n, m, d, \
                                                               out, s);
    switch (metric) {
        TPW_MET(TPW_BMET_HAMMING)
        TPW_MET(TPW_BMET_JACCARD)
        TPW_MET(TPW_BMET_DICE)
        TPW_MET(TPW_BMET_KULCZYNSKI1)
        TPW_MET(TPW_BMET_KULSINSKI)
        TPW_MET(TPW_BMET_ROGERSTANIMOTO)
        TPW_MET(TPW_BMET_RUSSELLRAO)
        TPW_MET(TPW_BMET_SOKALMICHENER)
        TPW_MET(TPW_BMET_SOKALSNEATH)
        default: return launch_counts<TPW_BIT_AND, kCountMetric + TPW_BMET_YULE>(x1w, x2w, pop1, pop2, batch, n, m, d, out, s);
    }
#undef TPW_MET
}

extern "C" int tpw_bool_row_counts(const uint8_t *x, int64_t rows, int64_t d, int32_t *counts,
                                   void *stream) {
    TPW_REQUIRE(rows >= 0 && d >= 0, "invalid sizes rows=%lld d=%lld", (long long)rows, (long long)d);
    TPW_REQUIRE(d <= (int64_t)0x7fffffff, "d=%lld exceeds the 32-bit count range", (long long)d);
    if (rows == 0) return TPW_OK;
    TPW_REQUIRE(x && counts, "null pointer");
    hipLaunchKernelGGL(bool_row_counts_kernel, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0,
                       as_stream(stream), x, rows, d, counts, d % 16 == 0 && aligned16(x));
    return check_launch("bool_row_counts_kernel");
}

namespace {
int check_bytes_args(const uint8_t *a, const uint8_t *b, const int32_t *pa, const int32_t *pb,
                     int64_t batch, int64_t n, int64_t m, int64_t d, float *out) {
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 1, "invalid sizes batch=%lld n=%lld m=%lld d=%lld",
                (long long)batch, (long long)n, (long long)m, (long long)d);
    TPW_REQUIRE(d <= (int64_t)0x7fffffff, "d=%lld exceeds the 32-bit count range", (long long)d);
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(cdiv(n, kTile) * cdiv(m, kTile) * batch <= (int64_t)0x7fffffff, "output too large for one launch");
    TPW_REQUIRE(a && b && pa && pb && out, "null pointer");
    return TPW_OK;
}
}  // namespace

extern "C" int tpw_bool_bytes_reduce(const uint8_t *x1, const uint8_t *x2, const int32_t *x1_counts,
                                     const int32_t *x2_counts, int64_t batch, int64_t n, int64_t m,
                                     int64_t d, int op, int reduction, float *out, void *stream) {
    TPW_REQUIRE(op >= TPW_BIT_AND && op <= TPW_BIT_NE, "unknown bit op %d", op);
    TPW_REQUIRE(reduction == TPW_RED_SUM || reduction == TPW_RED_MEAN, "unknown reduction %d",
                reduction);
    int rc = check_bytes_args(x1, x2, x1_counts, x2_counts, batch, n, m, d, out);
    if (rc != TPW_OK) return rc;
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    hipStream_t s = as_stream(stream);
#define TPW_CASE(OPC, K)                                                                        \
    case OPC:                                                                                   \
        return reduction == TPW_RED_SUM                                                         \
                   ? launch_bool_mfma<K, kSum>(x1, x2, x1_counts, x2_counts, batch, n, m, d, out, s) \
                   : launch_bool_mfma<K, kMean>(x1, x2, x1_counts, x2_counts, batch, n, m, d, out, s);
    switch (op) {
        TPW_CASE(TPW_BIT_AND, TPW_BIT_AND)
        TPW_CASE(TPW_BIT_OR, TPW_BIT_OR)
        TPW_CASE(TPW_BIT_XOR, TPW_BIT_XOR)
        TPW_CASE(TPW_BIT_EQ, TPW_BIT_EQ)
        TPW_CASE(TPW_BIT_NE, TPW_BIT_XOR)  // NE counts exactly like XOR on bits
        default: break;
    }
#undef TPW_CASE
    return TPW_ERR_INVALID;
}

extern "C" int tpw_bool_bytes_count_metric(const uint8_t *x1, const uint8_t *x2,
                                           const int32_t *x1_counts, const int32_t *x2_counts,
                                           int64_t batch, int64_t n, int64_t m, int64_t d, int metric,
                                           float *out, void *stream) {
    TPW_REQUIRE(metric >= TPW_BMET_HAMMING && metric <= TPW_BMET_YULE, "unknown metric %d", metric);
    int rc = check_bytes_args(x1, x2, x1_counts, x2_counts, batch, n, m, d, out);
    if (rc != TPW_OK) return rc;
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    hipStream_t s = as_stream(stream);
#define TPW_MET(CODE)                                                                                 \
    case CODE:                                                                                        \
        return launch_bool_mfma<TPW_BIT_AND, kCountMetric + CODE>(x1, x2, x1_counts, x2_counts, batch, n, \
                                                                  m, d, out, s);
    switch (metric) {
        TPW_MET(TPW_BMET_HAMMING)
        TPW_MET(TPW_BMET_JACCARD)
        TPW_MET(TPW_BMET_DICE)
        TPW_MET(TPW_BMET_KULCZYNSKI1)
        TPW_MET(TPW_BMET_KULSINSKI)
        TPW_MET(TPW_BMET_ROGERSTANIMOTO)
        TPW_MET(TPW_BMET_RUSSELLRAO)
        TPW_MET(TPW_BMET_SOKALMICHENER)
        TPW_MET(TPW_BMET_SOKALSNEATH)
        TPW_MET(TPW_BMET_YULE)
        default: break;
    }
#undef TPW_MET
    return TPW_ERR_INVALID;
}

extern "C" int64_t tpw_bool_fp4_row_bytes(int64_t d) { return d <= 0 ? 0 : fp4_row_bytes(d); }

extern "C" int tpw_pack_bool_fp4(const uint8_t *x, int64_t rows, int64_t d, uint8_t *fp4, int32_t *counts,
                                 void *stream) {
    TPW_REQUIRE(rows >= 0 && d >= 1, "invalid sizes rows=%lld d=%lld", (long long)rows, (long long)d);
    TPW_REQUIRE(d < (int64_t)kFloatExactLimit, "d=%lld: the fp4 layout counts exactly below 2^24 features",
                (long long)d);
    if (rows == 0) return TPW_OK;
    TPW_REQUIRE(x && fp4 && counts, "null pointer");
    TPW_REQUIRE(aligned16(fp4), "the fp4 rows must be 16-byte aligned");
    hipLaunchKernelGGL(pack_fp4_kernel, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, as_stream(stream), x, rows, d,
                       fp4_row_bytes(d), fp4, counts, d % 16 == 0 && aligned16(x));
    return check_launch("pack_fp4_kernel");
}

namespace {
int check_fp4_args(const uint8_t *a, const uint8_t *b, const int32_t *pa, const int32_t *pb, int64_t batch,
                   int64_t n, int64_t m, int64_t d, float *out) {
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 1, "invalid sizes batch=%lld n=%lld m=%lld d=%lld",
                (long long)batch, (long long)n, (long long)m, (long long)d);
    TPW_REQUIRE(d < (int64_t)kFloatExactLimit, "d=%lld: the fp4 layout counts exactly below 2^24 features",
                (long long)d);
    TPW_REQUIRE((n > m ? n : m) * fp4_row_bytes(d) < ((int64_t)1 << 31),
                "rows x row bytes must stay below 2^31 per batch for the fp4 kernel");
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    TPW_REQUIRE(cdiv(n, kTile) * cdiv(m, kTile) * batch <= (int64_t)0x7fffffff, "output too large for one launch");
    TPW_REQUIRE(a && b && pa && pb && out, "null pointer");
    TPW_REQUIRE(aligned16(a) && aligned16(b), "the fp4 rows must be 16-byte aligned");
    return TPW_OK;
}
}  // namespace

extern "C" int tpw_bool_fp4_reduce(const uint8_t *x1, const uint8_t *x2, const int32_t *x1_counts,
                                   const int32_t *x2_counts, int64_t batch, int64_t n, int64_t m, int64_t d, int op,
                                   int reduction, float *out, void *stream) {
    TPW_REQUIRE(op >= TPW_BIT_AND && op <= TPW_BIT_NE, "unknown bit op %d", op);
    TPW_REQUIRE(reduction == TPW_RED_SUM || reduction == TPW_RED_MEAN, "unknown reduction %d", reduction);
    int rc = check_fp4_args(x1, x2, x1_counts, x2_counts, batch, n, m, d, out);
    if (rc != TPW_OK) return rc;
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    hipStream_t s = as_stream(stream);
#define TPW_CASE(OPC, K)                                                                                  \
    case OPC:                                                                                             \
        return reduction == TPW_RED_SUM                                                                   \
                   ? launch_bool_fp4<K, kSum>(x1, x2, x1_counts, x2_counts, batch, n, m, d, out, s)        \
                   : launch_bool_fp4<K, kMean>(x1, x2, x1_counts, x2_counts, batch, n, m, d, out, s);
    switch (op) {
        TPW_CASE(TPW_BIT_AND, TPW_BIT_AND)
        TPW_CASE(TPW_BIT_OR, TPW_BIT_OR)
        TPW_CASE(TPW_BIT_XOR, TPW_BIT_XOR)
        TPW_CASE(TPW_BIT_EQ, TPW_BIT_EQ)
        TPW_CASE(TPW_BIT_NE, TPW_BIT_XOR)  // NE counts exactly like XOR on bits
        default: break;
    }
#undef TPW_CASE
    return TPW_ERR_INVALID;
}

extern "C" int tpw_bool_fp4_count_metric(const uint8_t *x1, const uint8_t *x2, const int32_t *x1_counts,
                                         const int32_t *x2_counts, int64_t batch, int64_t n, int64_t m, int64_t d,
                                         int metric, float *out, void *stream) {
    TPW_REQUIRE(metric >= TPW_BMET_HAMMING && metric <= TPW_BMET_YULE, "unknown metric %d", metric);
    int rc = check_fp4_args(x1, x2, x1_counts, x2_counts, batch, n, m, d, out);
    if (rc != TPW_OK) return rc;
    if (batch == 0 || n == 0 || m == 0) return TPW_OK;
    hipStream_t s = as_stream(stream);
#define TPW_MET(CODE)                                                                                       \
    case CODE:                                                                                              \
        return launch_bool_fp4<TPW_BIT_AND, kCountMetric + CODE>(x1, x2, x1_counts, x2_counts, batch, n, m, d, \
                                                                 out, s);
    switch (metric) {
        TPW_MET(TPW_BMET_HAMMING)
        TPW_MET(TPW_BMET_JACCARD)
        TPW_MET(TPW_BMET_DICE)
        TPW_MET(TPW_BMET_KULCZYNSKI1)
        TPW_MET(TPW_BMET_KULSINSKI)
        TPW_MET(TPW_BMET_ROGERSTANIMOTO)
        TPW_MET(TPW_BMET_RUSSELLRAO)
        TPW_MET(TPW_BMET_SOKALMICHENER)
        TPW_MET(TPW_BMET_SOKALSNEATH)
        TPW_MET(TPW_BMET_YULE)
        default: break;
    }
#undef TPW_MET
    return TPW_ERR_INVALID;
}

namespace tpw {
namespace {
// One thread per denominator o: x = phase + k step (k < count, phase = o 2654435761 mod step)
// through div_count, and div_count_r with y = RN(1 / o), against __fdiv_rn, bit for bit.
__global__ __launch_bounds__(256) void count_division_check_kernel(int64_t o_lo, int64_t o_hi, int64_t step,
                                                                   int64_t count,
                                                                   unsigned long long *__restrict__ mismatches) {
    const int64_t o = o_lo + (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (o > o_hi) return;
    const float of = (float)o;
    const float y = __fdiv_rn(1.0f, of);
    const int64_t phase = (int64_t)(((uint64_t)o * 2654435761u) % (uint64_t)step);
    unsigned long long bad = 0;
    for (int64_t k = 0; k < count; ++k) {
        const float xf = (float)(phase + k * step);
        const uint32_t ref = __float_as_uint(__fdiv_rn(xf, of));
        bad += __float_as_uint(div_count(xf, of)) != ref;
        bad += __float_as_uint(div_count_r(xf, of, y)) != ref;
    }
    if (bad) atomicAdd(mismatches, bad);
}
}  // namespace
}  // namespace tpw

extern "C" int tpw_count_division_check(int64_t o_lo, int64_t o_hi, int64_t x_step, int64_t x_count,
                                        unsigned long long *mismatches, void *stream) {
    TPW_REQUIRE(o_lo >= 1 && o_lo <= o_hi && o_hi <= 2 * kSmallRowLimit, "denominators must lie in [1, 2^21]");
    TPW_REQUIRE(x_step >= 1 && x_count >= 1 && (x_step - 1) + (x_count - 1) * x_step <= 4 * kSmallRowLimit,
                "numerators must lie in [0, 2^22]");
    TPW_REQUIRE((o_hi - o_lo + 1) * x_count <= ((int64_t)1 << 36), "too many quotients for one check");
    TPW_REQUIRE(mismatches, "null pointer");
    hipLaunchKernelGGL(count_division_check_kernel, dim3((unsigned)cdiv(o_hi - o_lo + 1, 256)), dim3(256), 0,
                       as_stream(stream), o_lo, o_hi, x_step, x_count, mismatches);
    return check_launch("count_division_check_kernel");
}
