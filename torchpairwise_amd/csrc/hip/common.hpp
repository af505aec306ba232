// Shared helpers of the gfx950 kernel library (device side and host side).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "torchpairwise_amd.h"

namespace tpw {

// Records a printf-style message as the calling thread's last error.
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

// Turns a pending launch failure into TPW_ERR_LAUNCH (with a message naming `what`).
int check_launch(const char *what);

// Start / stop events for one kernel launch (hipExtLaunchKernelGGL stamps them as part of the
// dispatch, so they add no packets of their own): a free event pair of the launch timer when
// tpw_launch_timer_arm armed it for this kernel family on the current device, else null events
// (a plain launch).  launch_timer.hip.
struct LaunchEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};
LaunchEvents launch_events(const char *family);

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Largest grid.y / grid.z the launcher may use.
constexpr int64_t kMaxGridYZ = 65535;

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ void store_nt(float *p, float v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void store_nt4(float *p, floatx4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<floatx4 *>(p));
}

// Correctly rounded fp32 square root.  (On this toolchain __fsqrt_rn lowers to the bare
// 1-ulp v_sqrt_f32; sqrtf / __builtin_sqrtf get the fma-based rounding fix-up.)
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }

// x / y within 2 ulp: the hardware reciprocal (v_rcp_f32, 1 ulp) times x, where the IEEE
// divide takes about ten instructions.  Denominators outside [2^-126, 2^126] (zero, denormal,
// inf, NaN, or a reciprocal that could flush) take the IEEE divide, behind a branch that whole
// waves of ordinary values skip.  For the floating-point backward weights, whose results carry
// summation error anyway; bit-exact paths keep the IEEE divide.
__device__ __forceinline__ float fast_div(float x, float y) {
    const float ay = __builtin_fabsf(y);
    float q = x * __builtin_amdgcn_rcpf(y);
    if (__builtin_expect(!(ay >= 0x1p-126f && ay <= 0x1p126f), 0)) q = __fdiv_rn(x, y);
    return q;
}

// bf16 (stored as uint16_t bits) <-> fp32; fp32 -> bf16 rounds to nearest even, as
// c10::BFloat16 does.
// fp32 -> bf16, round to nearest even, on gfx950's v_cvt_pk_bf16_f32; NaN becomes 0x7fc0, as
// torch's conversion gives, so elementwise results match the CPU bit for bit.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    const uint16_t r = __builtin_bit_cast(uint16_t, (__bf16)f);
    return f != f ? (uint16_t)0x7fc0 : r;
}
// Two values in one v_cvt_pk_bf16_f32 (lo in bits 0-15); a NaN keeps the hardware's pattern.
typedef float tpw_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 tpw_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_rne(float lo, float hi) {
    const tpw_f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, tpw_bf16x2));
}
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(uint16_t v) { return bf16_to_f32(v); }
__device__ __forceinline__ void from_f32(float *p, float v) { *p = v; }
__device__ __forceinline__ void from_f32(uint16_t *p, float v) { *p = f32_to_bf16_rne(v); }

// Maps a linear workgroup id to (batch, tile row, tile col) of a tiles_n x tiles_m x batch
// output grid.  Consecutive workgroup ids go round-robin over the 8 XCDs (id % 8 selects
// the XCD), so when total % 8 == 0 each XCD gets a contiguous range of tiles; within a
// batch the tiles run in groups of 8 tile rows, column by column, so that the blocks
// resident on one XCD share operand panels in its L2.
__device__ __forceinline__ void xcd_tile_of(int64_t bid, int64_t tiles_n, int64_t tiles_m,
                                            int64_t total, int64_t &b, int64_t &tr, int64_t &tc) {
    constexpr int64_t kGroupRows = 8;
    int64_t t = bid;
    if ((total & 7) == 0) t = (bid & 7) * (total >> 3) + (bid >> 3);
    const int64_t per_batch = tiles_n * tiles_m;
    b = t / per_batch;
    t -= b * per_batch;
    const int64_t in_group = kGroupRows * tiles_m;
    const int64_t g = t / in_group;
    const int64_t first = g * kGroupRows;
    const int64_t gsize = tiles_n - first < kGroupRows ? tiles_n - first : kGroupRows;
    const int64_t o = t - g * in_group;
    tr = first + o % gsize;
    tc = o / gsize;
}

// Raw buffer resource over the `elems` floats that start at `base` (word 3 0x00020000: the
// 32-bit data format of gfx9 raw buffers).  A dword load at a byte offset at or past the end
// returns 0 without touching memory; elems <= 0 makes every load return 0.  The range is
// clamped to 2^32 - 1 bytes, so lane offsets must stay below that.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_over(const float *base, int64_t elems) {
    const int64_t bytes = elems > 0 ? elems * 4 : 0;
    const uint32_t num = bytes >= (int64_t)0xffffffffLL ? 0xffffffffu : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, (int)num, 0x00020000);
}
__device__ __forceinline__ float buffer_load(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_offset, 0, 0));
}
// Four floats at a 16-byte aligned byte offset (whole in range or whole out: the caller keeps
// array lengths and offsets multiples of 4 floats).
typedef unsigned int tpw_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ floatx4 buffer_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset) {
    return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_offset, 0, 0));
}

// Parameters of the kernel-function epilogues (polynomial, sigmoid) of the MFMA kernel.
struct KerParams {
    float gamma = 0.0f, coef0 = 0.0f;
    int degree = 0;
    float eps = 0.0f;  // the radius of the neighbour-mask epilogue
};

// S = x1 . x2^T in fp32 on the matrix cores for fp32 or bf16 inputs (inner.hip).
int inner_dot_f32(const void *x1, const void *x2, int dtype, int64_t batch, int64_t n, int64_t m,
                  int64_t d, float *out, hipStream_t s);

// out[b] = sign * (A[b] . B[b]^T) + coef[b*M + row] * X[b][row][col] on the matrix cores,
// A [batch, M, K], B [batch, N, K], X and out [batch, M, N] of type dtype (inner.hip).
int inner_grad_gemm(const void *A, const void *B, int dtype, int64_t batch, int64_t M, int64_t N,
                    int64_t K, float sign, const float *coef, const void *X, void *out, hipStream_t s);

// The same product in fp32 with A stored k-major [batch, K, M] when a_kmajor (else [batch, M,
// K]) and B k-major [batch, K, N] (b_kmajor must be true).  coef == nullptr: coef[row] is the
// sum over K of A's row (for A = W^T, the column sums of W).  Only the shapes
// grad_product_f32_fits accepts (whole 32-element K chunks, 16-byte aligned rows and pieces).
bool grad_product_f32_fits(const float *A, bool a_kmajor, const float *B, bool b_kmajor, int64_t M, int64_t N,
                           int64_t K, const float *X, const float *out);
int grad_product_f32(const float *A, bool a_kmajor, const float *B, bool b_kmajor, int64_t batch, int64_t M,
                     int64_t N, int64_t K, float sign, const float *coef, const float *X, float *out,
                     hipStream_t s);
// The same in bf16 (bits), K a multiple of 64 (coef == nullptr: the row sums of A's bf16
// values); k-major bf16 pieces come from transposing LDS reads.
bool grad_product_bf16_fits(const uint16_t *A, bool a_kmajor, const uint16_t *B, bool b_kmajor, int64_t M,
                            int64_t N, int64_t K, const uint16_t *X, const uint16_t *out);
int grad_product_bf16(const uint16_t *A, bool a_kmajor, const uint16_t *B, bool b_kmajor, int64_t batch, int64_t M,
                      int64_t N, int64_t K, float sign, const float *coef, const uint16_t *X, uint16_t *out,
                      hipStream_t s);

// Backward of _ppminkowski / _wminkowski (w != nullptr) at p = +-inf (lp_inf_backward.hip):
// grad_x1, grad_x2 and, weighted, per-row weight-gradient partials wrows [batch, n, d].
int lp_inf_backward(const float *g, const float *x1, const float *x2, const float *w, int64_t batch, int64_t n,
                    int64_t m, int64_t d, bool neg, float *gx1, float *gx2, float *wrows, hipStream_t s);

}  // namespace tpw

#define TPW_REQUIRE(cond, ...)          \
    do {                                \
        if (!(cond)) {                  \
            tpw::set_error(__VA_ARGS__); \
            return TPW_ERR_INVALID;     \
        }                               \
    } while (0)
