// Row-wise "k smallest" mask over a distance matrix: the k-nearest-neighbour mask of
// torchpairwise.k_neighbors_mask.
//
// The reference computes it as dists.argsort(1)[:, :k + 1] followed by index_put_ of `true`
// into a zero [N, M] bool tensor (csrc/ops/neighbors.cpp:29-34): a full sort of every row.
// Here one workgroup owns one row, selects its `count` = min(k + 1, M) smallest entries and
// writes the whole bool row, so the distances are read once from HBM and the mask written
// once: the kernel is HBM-bound (4 bytes read + 1 byte written per element for fp32).
//
// Order: ascending value, NaN after +inf, -0 == +0 (the order of a comparison sort), ties
// broken by the lower column index.  Each element gets a unique 64-bit key
// (order_key(value) << 32 | column), so "the count smallest keys" is well defined and the
// selected set equals the first `count` entries of a stable ascending argsort.  (The
// reference's argsort is not stable: on ties across the boundary its choice is
// implementation-defined; everywhere else the sets are identical.)
//
// Two selection strategies:
//   * count <= 16: every thread keeps its own sorted list of its L smallest keys (L = next
//     power of two >= count) while streaming the row; the workgroup then pops the global
//     minimum of the list heads `count` times.  About one compare per element.
//   * count > 16: radix-2 select on the 32-bit order keys (one counting pass per bit below
//     the common prefix of the row's min and max keys), then, only when the boundary value
//     is tied, a second radix-2 select on the column index among the tied entries.
// The list selection streams the row twice (the second read mostly hits L2 / the infinity
// cache); the radix selection caches rows of up to 16384 keys in LDS, longer rows are
// re-read on each pass.
#include "common.hpp"

namespace tpw {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ float load_f32(const float *p) { return *p; }
__device__ __forceinline__ float load_f32(const uint16_t *p) { return bf16_to_f32(*p); }
struct Half16 {
    uint16_t bits;
};
__device__ __forceinline__ float load_f32(const Half16 *p) {
    return (float)__builtin_bit_cast(_Float16, p->bits);
}

// Monotone map of a float onto uint32 for ascending order: -inf smallest, +inf below NaN,
// every NaN maps to the top value, -0 and +0 to the same key.
__device__ __forceinline__ uint32_t order_key(float v) {
    if (v != v) return 0xffffffffu;
    uint32_t b = __float_as_uint(v == 0.f ? 0.f : v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// ---------------------------------------------------------------- workgroup reductions
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        uint64_t y = __shfl_xor(x, off, 64);
        x = y < x ? y : x;
    }
    return x;
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x = min(x, (uint32_t)__shfl_xor(x, off, 64));
    return x;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x = max(x, (uint32_t)__shfl_xor(x, off, 64));
    return x;
}

// Block-wide reductions through a double-buffered LDS slot: `phase` alternates between
// calls, so one barrier per call suffices (a slot is rewritten only two calls later, after
// the intervening call's barrier has ordered every read of it).
struct Reducer {
    uint64_t *slots;  // [2][kWaves]
    int phase = 0;

    __device__ uint64_t min_u64(uint64_t x) {
        x = wave_min_u64(x);
        uint64_t *s = slots + phase * kWaves;
        phase ^= 1;
        if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = x;
        __syncthreads();
        uint64_t r = s[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) r = s[w] < r ? s[w] : r;
        return r;
    }
    __device__ uint32_t sum_u32(uint32_t x) {
        x = wave_sum_u32(x);
        uint64_t *s = slots + phase * kWaves;
        phase ^= 1;
        if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = x;
        __syncthreads();
        uint32_t r = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) r += (uint32_t)s[w];
        return r;
    }
    // min in the low half, max in the high half
    __device__ void min_max_u32(uint32_t lo, uint32_t hi, uint32_t &mn, uint32_t &mx) {
        lo = wave_min_u32(lo);
        hi = wave_max_u32(hi);
        uint64_t *s = slots + phase * kWaves;
        phase ^= 1;
        if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = ((uint64_t)hi << 32) | lo;
        __syncthreads();
        mn = 0xffffffffu;
        mx = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            mn = min(mn, (uint32_t)s[w]);
            mx = max(mx, (uint32_t)(s[w] >> 32));
        }
    }
};

// The row's order keys, either cached in LDS (CACHED, one HBM read per row) or streamed
// from memory on every pass, kUnroll loads in flight per thread.
constexpr int kUnroll = 16;
constexpr int64_t kCacheCols = 16384;  // 64 KB of keys per workgroup

template <typename T, bool CACHED>
struct RowKeys {
    const T *row;
    int64_t cols;
    uint32_t *lds;  // [cols] when CACHED

    __device__ void load() {
        if constexpr (CACHED) {
            stream([&](uint32_t k, uint32_t j) { lds[j] = k; });
            __syncthreads();
        }
    }
    template <typename F>
    __device__ void stream(F &&f) const {
        for (int64_t base = 0; base < cols; base += (int64_t)kThreads * kUnroll) {
            float v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t j = base + threadIdx.x + (int64_t)u * kThreads;
                v[u] = j < cols ? load_f32(row + j) : 0.f;
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t j = base + threadIdx.x + (int64_t)u * kThreads;
                if (j < cols) f(order_key(v[u]), (uint32_t)j);
            }
        }
    }
    // f(key, column) for every entry of the row owned by this thread
    template <typename F>
    __device__ void for_each(F &&f) const {
        if constexpr (CACHED) {
            for (int64_t j = threadIdx.x; j < cols; j += kThreads) f(lds[j], (uint32_t)j);
        } else {
            stream(f);
        }
    }
};

// Writes mask[j] = (key(j) << 32 | j) <= thr for the whole row.
template <typename T, bool CACHED>
__device__ void write_mask(const RowKeys<T, CACHED> &keys, uint64_t thr, uint8_t *mrow) {
    keys.for_each([&](uint32_t k, uint32_t j) {
        mrow[j] = (((uint64_t)k << 32) | j) <= thr ? 1 : 0;
    });
}

// count <= L <= 16: per-thread sorted lists, then `count` pops of the workgroup minimum.
template <typename T, int L, bool CACHED>
__global__ __launch_bounds__(kThreads) void smallest_list_kernel(const T *__restrict__ dist,
                                                                 int64_t cols, int count,
                                                                 uint8_t *__restrict__ mask) {
    __shared__ uint64_t slots[2 * kWaves];
    extern __shared__ uint32_t row_keys[];
    const int64_t r = blockIdx.x;
    RowKeys<T, CACHED> keys{dist + r * cols, cols, row_keys};
    keys.load();

    uint64_t lst[L];
#pragma unroll
    for (int s = 0; s < L; ++s) lst[s] = ~0ull;
    keys.for_each([&](uint32_t k, uint32_t j) {
        const uint64_t key = ((uint64_t)k << 32) | j;
        if (key < lst[L - 1]) {
            lst[L - 1] = key;
#pragma unroll
            for (int s = L - 1; s > 0; --s) {
                if (lst[s] < lst[s - 1]) {
                    const uint64_t t = lst[s];
                    lst[s] = lst[s - 1];
                    lst[s - 1] = t;
                }
            }
        }
    });

    Reducer red{slots};
    uint64_t thr = 0;
    for (int c = 0; c < count; ++c) {
        thr = red.min_u64(lst[0]);
        if (lst[0] == thr) {  // keys are unique: exactly one thread owns the minimum
#pragma unroll
            for (int s = 0; s < L - 1; ++s) lst[s] = lst[s + 1];
            lst[L - 1] = ~0ull;
        }
    }
    write_mask(keys, thr, mask + r * cols);
}

// count > 16: radix-2 select on the order key, then on the column among tied keys.
template <typename T, bool CACHED>
__global__ __launch_bounds__(kThreads) void smallest_radix_kernel(const T *__restrict__ dist,
                                                                  int64_t cols, int count,
                                                                  uint8_t *__restrict__ mask) {
    __shared__ uint64_t slots[2 * kWaves];
    extern __shared__ uint32_t row_keys[];
    const int64_t r = blockIdx.x;
    RowKeys<T, CACHED> keys{dist + r * cols, cols, row_keys};
    keys.load();
    Reducer red{slots};

    // common prefix of the row's smallest and largest keys: the selected boundary value
    // shares it, so only the bits below the highest differing bit need a counting pass
    uint32_t lo = 0xffffffffu, hi = 0;
    keys.for_each([&](uint32_t k, uint32_t) {
        lo = min(lo, k);
        hi = max(hi, k);
    });
    uint32_t kmin, kmax;
    red.min_max_u32(lo, hi, kmin, kmax);
    const uint32_t diff = kmin ^ kmax;
    // t = largest value with #(key < t) <= count - 1, i.e. the count-th smallest key
    uint32_t t = kmin;
    if (diff) {
        const int top = 31 - __builtin_clz(diff);
        t = kmin & ~((2u << top) - 1u);  // common prefix, zeros below (2u << 31 wraps to 0)
        for (int b = top; b >= 0; --b) {
            const uint32_t c = t | (1u << b);
            uint32_t n = 0;
            keys.for_each([&](uint32_t k, uint32_t) { n += k < c; });
            if (red.sum_u32(n) <= (uint32_t)(count - 1)) t = c;
        }
    }
    uint32_t n_lt = 0, n_eq = 0;
    keys.for_each([&](uint32_t k, uint32_t) {
        n_lt += k < t;
        n_eq += k == t;
    });
    n_lt = red.sum_u32(n_lt);
    n_eq = red.sum_u32(n_eq);
    const uint32_t need = (uint32_t)count - n_lt;  // 1 <= need <= n_eq
    uint32_t jmax = 0xffffffffu;                    // every tied entry selected
    if (need < n_eq) {
        // the need-th smallest column among the entries equal to t
        uint32_t jt = 0;
        const int top = 31 - __builtin_clz((uint32_t)(cols - 1) | 1u);
        for (int b = top; b >= 0; --b) {
            const uint32_t c = jt | (1u << b);
            uint32_t n = 0;
            keys.for_each([&](uint32_t k, uint32_t j) { n += (k == t) & (j < c); });
            if (red.sum_u32(n) <= need - 1) jt = c;
        }
        jmax = jt;
    }
    write_mask(keys, ((uint64_t)t << 32) | jmax, mask + r * cols);
}

__global__ void fill_kernel(uint8_t *__restrict__ mask, int64_t n, uint8_t value) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        mask[i] = value;
}

template <typename T, bool CACHED>
int launch_rows(const void *dist, int64_t rows, int64_t cols, int count, uint8_t *mask,
                hipStream_t s) {
    const T *d = static_cast<const T *>(dist);
    const dim3 grid((unsigned)rows), block(kThreads);
    const size_t lds = CACHED ? (size_t)cols * sizeof(uint32_t) : 0;
    if (count > 16) {
        hipLaunchKernelGGL((smallest_radix_kernel<T, CACHED>), grid, block, lds, s, d, cols, count, mask);
        return check_launch("smallest_radix_kernel");
    }
#define TPW_LIST(LL)                                                                                       \
    hipLaunchKernelGGL((smallest_list_kernel<T, LL, CACHED>), grid, block, lds, s, d, cols, count, mask); \
    return check_launch("smallest_list_kernel")
    if (count <= 1) { TPW_LIST(1); }
    if (count <= 2) { TPW_LIST(2); }
    if (count <= 4) { TPW_LIST(4); }
    if (count <= 8) { TPW_LIST(8); }
    TPW_LIST(16);
#undef TPW_LIST
}

// LDS a workgroup may allocate on the current device (queried once per device).
size_t lds_per_block() {
    static size_t cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 65536;
    if (!cached[dev]) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            v = 65536;
        cached[dev] = (size_t)v;
    }
    return cached[dev];
}

// The list selection reads the row twice (list pass, mask pass) and streams it; the radix
// selection makes one pass per key bit and caches the row's keys in LDS when they fit
// (next to the 64 bytes of reduction slots).
template <typename T>
int launch(const void *dist, int64_t rows, int64_t cols, int count, uint8_t *mask, hipStream_t s) {
    if (count > 16 && cols <= kCacheCols &&
        (size_t)cols * sizeof(uint32_t) + 2 * kWaves * sizeof(uint64_t) <= lds_per_block())
        return launch_rows<T, true>(dist, rows, cols, count, mask, s);
    return launch_rows<T, false>(dist, rows, cols, count, mask, s);
}

}  // namespace
}  // namespace tpw

using namespace tpw;

extern "C" int tpw_row_smallest_mask(const void *dist, int dtype, int64_t rows, int64_t cols,
                                     int64_t count, void *mask, void *stream) {
    TPW_REQUIRE(rows >= 0 && cols >= 0 && count >= 0, "invalid sizes");
    if (rows == 0 || cols == 0) return TPW_OK;
    TPW_REQUIRE(dist && mask, "null pointer");
    TPW_REQUIRE(rows <= 0x7fffffff, "rows = %lld exceeds the grid limit 2^31 - 1", (long long)rows);
    TPW_REQUIRE(cols <= 0x7fffffff, "cols = %lld exceeds 2^31 - 1", (long long)cols);
    hipStream_t s = as_stream(stream);
    uint8_t *m = static_cast<uint8_t *>(mask);
    if (count == 0 || count >= cols) {  // nothing / everything selected
        const int64_t n = rows * cols;
        const unsigned grid = (unsigned)(cdiv(n, 256) < 8192 ? cdiv(n, 256) : 8192);
        hipLaunchKernelGGL(fill_kernel, dim3(grid), dim3(256), 0, s, m, n, (uint8_t)(count != 0));
        return check_launch("fill_kernel");
    }
    switch (dtype) {
        case TPW_F32: return launch<float>(dist, rows, cols, (int)count, m, s);
        case TPW_BF16: return launch<uint16_t>(dist, rows, cols, (int)count, m, s);
        case TPW_F16: return launch<Half16>(dist, rows, cols, (int)count, m, s);
        default:
            tpw::set_error("row_smallest_mask: unsupported dtype %d (float32, bfloat16, float16)", dtype);
            return TPW_ERR_INVALID;
    }
}
