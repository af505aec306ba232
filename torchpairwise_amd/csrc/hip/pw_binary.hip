// Unreduced pairwise binary ops (pwand, pwor, pwxor, pweq, pwne, pwlt, pwgt, pwle, pwge):
// out[b, i, j, k] = op(x1[b, i, k], x2[b, j, k]) as bool bytes, [batch, n, m, d].
//
// The output (n m d bytes per batch) is the whole cost: per output byte there is one x1 and
// one x2 element to read, both from rows that stay in the caches (x1 row i for the m d outputs
// of its slice, the x2 slice [m, d] for every i).  The output is therefore taken as one flat
// byte array: each thread owns 16 consecutive bytes (one 16-byte store), walks (b, i, j, k)
// incrementally from its first byte, and reads x1[b, i, k] and x2[b, j, k] for each.  The x2
// reads of a wave are contiguous (they follow the output index within a slice).
//
// Element types: bool / uint8 (bytes), int8, int16, int32, int64, float, double, float16 and
// bfloat16 (compared as float, as c10's operators compare them).  The logical ops are used on
// bool only (the reference dispatches them for bool alone), where &, |, ^ of 0 / 1 bytes are
// the logical results.
#include "common.hpp"

namespace tpw {
namespace {

struct H16 {
    uint16_t bits;
};
struct B16 {
    uint16_t bits;
};
__device__ __forceinline__ float ld(H16 v) { return (float)__builtin_bit_cast(_Float16, v.bits); }
__device__ __forceinline__ float ld(B16 v) { return bf16_to_f32(v.bits); }
template <typename T>
__device__ __forceinline__ T ld(T v) {
    return v;
}

// op codes: TPW_BIT_AND / OR / XOR / EQ / NE, TPW_CMP_LT / GT / LE / GE
template <int OP, typename T>
__device__ __forceinline__ uint32_t apply(T a, T b) {
    const auto x = ld(a);
    const auto y = ld(b);
    if constexpr (OP == TPW_BIT_AND) return (uint32_t)((x & y) != 0);
    else if constexpr (OP == TPW_BIT_OR) return (uint32_t)((x | y) != 0);
    else if constexpr (OP == TPW_BIT_XOR) return (uint32_t)((x ^ y) != 0);
    else if constexpr (OP == TPW_BIT_EQ) return (uint32_t)(x == y);
    else if constexpr (OP == TPW_BIT_NE) return (uint32_t)(x != y);
    else if constexpr (OP == TPW_CMP_LT) return (uint32_t)(x < y);
    else if constexpr (OP == TPW_CMP_GT) return (uint32_t)(x > y);
    else if constexpr (OP == TPW_CMP_LE) return (uint32_t)(x <= y);
    else return (uint32_t)(x >= y);
}

template <int OP, typename T>
__global__ __launch_bounds__(256) void pw_binary_kernel(const T *__restrict__ x1, const T *__restrict__ x2,
                                                        int64_t n, int64_t m, int64_t d, int64_t total,
                                                        uint8_t *__restrict__ out) {
    const int64_t f0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16;
    if (f0 >= total) return;
    const int64_t md = m * d;
    int64_t bi = f0 / md;  // b n + i
    const int64_t t = f0 - bi * md;
    int64_t j = t / d, k = t - (t / d) * d;
    int64_t b = bi / n;
    const int cnt = total - f0 < 16 ? (int)(total - f0) : 16;
    uint32_t w0 = 0, w1 = 0, w2 = 0, w3 = 0;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        if (e < cnt) {
            const uint32_t v = apply<OP, T>(x1[bi * d + k], x2[(b * m + j) * d + k]) << (8 * (e & 3));
            if (e < 4) w0 |= v;
            else if (e < 8) w1 |= v;
            else if (e < 12) w2 |= v;
            else w3 |= v;
            if (++k == d) {
                k = 0;
                if (++j == m) {
                    j = 0;
                    ++bi;
                    b = bi / n;
                }
            }
        }
    }
    if (cnt == 16) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 v = {w0, w1, w2, w3};
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(out + f0));
    } else {
        for (int e = 0; e < cnt; ++e) {
            const uint32_t w = e < 4 ? w0 : e < 8 ? w1 : e < 12 ? w2 : w3;
            out[f0 + e] = (uint8_t)(w >> (8 * (e & 3)));
        }
    }
}

template <int OP>
int launch_op(const void *x1, const void *x2, int dtype, int64_t n, int64_t m, int64_t d, int64_t total,
              uint8_t *out, hipStream_t s) {
    const dim3 grid((unsigned)cdiv(total, 256 * 16)), block(256);
#define TPW_PWB(T)                                                                                             \
    hipLaunchKernelGGL((pw_binary_kernel<OP, T>), grid, block, 0, s, static_cast<const T *>(x1),               \
                       static_cast<const T *>(x2), n, m, d, total, out);                                       \
    break
    if constexpr (OP <= TPW_BIT_XOR) {
        TPW_REQUIRE(dtype == TPW_U8, "logical ops take bool (TPW_U8) elements, got dtype %d", dtype);
        hipLaunchKernelGGL((pw_binary_kernel<OP, uint8_t>), grid, block, 0, s, static_cast<const uint8_t *>(x1),
                           static_cast<const uint8_t *>(x2), n, m, d, total, out);
    } else {
        switch (dtype) {
            case TPW_F32: TPW_PWB(float);
            case TPW_F64: TPW_PWB(double);
            case TPW_F16: TPW_PWB(H16);
            case TPW_BF16: TPW_PWB(B16);
            case TPW_I8: TPW_PWB(int8_t);
            case TPW_U8: TPW_PWB(uint8_t);
            case TPW_I16: TPW_PWB(int16_t);
            case TPW_I32: TPW_PWB(int32_t);
            case TPW_I64: TPW_PWB(int64_t);
            default: TPW_REQUIRE(false, "unsupported dtype %d", dtype);
        }
    }
#undef TPW_PWB
    return check_launch("pw_binary_kernel");
}

}  // namespace
}  // namespace tpw

using namespace tpw;

extern "C" int tpw_pairwise_binary(const void *x1, const void *x2, int dtype, int op, int64_t batch, int64_t n,
                                   int64_t m, int64_t d, uint8_t *out, void *stream) {
    TPW_REQUIRE(batch >= 0 && n >= 0 && m >= 0 && d >= 0, "invalid sizes");
    const int64_t total = batch * n * m * d;
    if (total == 0) return TPW_OK;
    TPW_REQUIRE(x1 && x2 && out, "null pointer");
    TPW_REQUIRE(aligned16(out), "out must be 16-byte aligned");
    TPW_REQUIRE(cdiv(total, 256 * 16) <= 0x7fffffffLL, "output too large");
    hipStream_t s = as_stream(stream);
    switch (op) {
        case TPW_BIT_AND: return launch_op<TPW_BIT_AND>(x1, x2, dtype, n, m, d, total, out, s);
        case TPW_BIT_OR: return launch_op<TPW_BIT_OR>(x1, x2, dtype, n, m, d, total, out, s);
        case TPW_BIT_XOR: return launch_op<TPW_BIT_XOR>(x1, x2, dtype, n, m, d, total, out, s);
        case TPW_BIT_EQ: return launch_op<TPW_BIT_EQ>(x1, x2, dtype, n, m, d, total, out, s);
        case TPW_BIT_NE: return launch_op<TPW_BIT_NE>(x1, x2, dtype, n, m, d, total, out, s);
        case TPW_CMP_LT: return launch_op<TPW_CMP_LT>(x1, x2, dtype, n, m, d, total, out, s);
        case TPW_CMP_GT: return launch_op<TPW_CMP_GT>(x1, x2, dtype, n, m, d, total, out, s);
        case TPW_CMP_LE: return launch_op<TPW_CMP_LE>(x1, x2, dtype, n, m, d, total, out, s);
        case TPW_CMP_GE: return launch_op<TPW_CMP_GE>(x1, x2, dtype, n, m, d, total, out, s);
        default: TPW_REQUIRE(false, "unknown op %d", op);
    }
    return TPW_OK;
}
