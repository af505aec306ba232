// Shared pieces of the 128 x 128 matrix-core tile kernels (inner.hip, popcount.hip).
//
// Block = 256 threads, 4 waves in a 2 x 2 grid, 64 x 64 outputs per wave as 2 x 2 blocks of a
// 32 x 32 MFMA.  A K chunk is 128 bytes of every operand row; the chunk's A and B panels
// (128 rows each) sit in LDS as 16-byte pieces with no padding: piece c of row r is stored at
// position swz(r, c) of the row, which makes the MFMA's 16-byte reads of one piece across 16
// consecutive rows conflict-free.  The chunk travels from global memory straight into LDS
// (global_load_lds_dwordx4, one 16-byte slot per lane and instruction).
//
// Products are formed transposed (B rows as the MFMA's first operand), so the accumulator
// register 4 g + e of lane (l32 + 32 h) holds output row l32 of the 32 x 32 block and column
// 8 g + 4 h + e: four consecutive columns per register quad.  The epilogue therefore writes
// 16-byte pieces of output rows into an LDS stage (the operand buffer, free after the K loop)
// and the whole tile leaves in contiguous row segments (256 bytes of bf16 or 512 bytes of fp32
// per row and instruction group).
#pragma once

#include "common.hpp"

namespace tpw {
namespace tile {

constexpr int kT = 128;           // output rows and columns per tile
constexpr int kThreads = 256;     // 4 waves
constexpr int kPanel = kT * 8;    // uint4 per operand panel (128 rows x 8 pieces)
constexpr int kBuf = 2 * kPanel;  // A | B panels: 32 KiB
constexpr int kSlots = 8;         // DMA slots per lane and chunk: 2048 pieces / 256 lanes

// Position of logical piece c in row r.  An involution in c for fixed r, so the DMA slot at
// position p of row r carries logical piece swz(r, p).
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r & 7) ^ ((r >> 3) & 1)); }

// 16 bytes per lane from sbase + voff into LDS at lds_base + 16 * lane.  Issued through inline
// asm: the compiler cannot tell which LDS bytes a DMA writes and would otherwise wait for every
// DMA in flight before any later LDS read.  Waits for these loads are explicit (barrier_all).
__device__ __forceinline__ void dma16(const void *sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base)
                 : "memory", "m0");
}
// The same for 4 bytes per lane (LDS lds_base + 4 * lane).
__device__ __forceinline__ void dma4(const void *sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base)
                 : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t)(uintptr_t)p; }

// Per-row values of the tile (128 for its rows, then 128 for its columns, 4 bytes each) into
// LDS `dst` by DMA: wave w < 2 loads rows 64 w .. 64 w + 63, wave 2 + w the columns; indices past
// the edge read the last element (never used).  `wave` must be wave-uniform.  Visible after
// the next barrier_all.
__device__ __forceinline__ void dma_tile_rows(const void *rows_base, const void *cols_base, bool cols, int wave,
                                              int lane, int64_t row0, int64_t col0, int64_t n, int64_t m, void *dst) {
    if (wave >= 2 && !cols) return;
    const bool c = wave >= 2;
    const int64_t lim = c ? m : n;
    int64_t i = (c ? col0 : row0) + 64 * (wave & 1) + lane;
    i = i < lim ? i : lim - 1;
    dma4(c ? cols_base : rows_base, (uint32_t)(i * 4), lds_addr(reinterpret_cast<uint32_t *>(dst) + 64 * wave));
}

// Workgroup barrier after this wave's LDS operations have completed (_all: and its vector
// memory operations, the DMA included).  Also a compiler barrier for memory accesses.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void barrier_all() {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Byte offsets (from each panel's batch base) of this lane's 8 DMA slots for the tile at
// (row0, col0): slot s = (8 wave + j) 64 + lane covers panel s >> 10 (A rows, then B rows),
// row (s >> 3) & 127 and position s & 7; rows past the edge read the last row, whose outputs
// are never stored.  Requires rows * row_bytes < 2^32.
__device__ __forceinline__ void dma_offsets(uint32_t (&off)[kSlots], int wave, int lane, int64_t row0, int64_t col0,
                                            int64_t n, int64_t m, int64_t row_bytes) {
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int s = (wave * kSlots + j) * 64 + lane;
        const int panel = s >> 10, r = (s >> 3) & (kT - 1), p = s & 7;
        const int64_t lim = panel ? m : n;
        int64_t row = (panel ? col0 : row0) + r;
        row = row < lim ? row : lim - 1;
        off[j] = (uint32_t)(row * row_bytes + swz(r, p) * 16);
    }
}

// DMA of the 128-byte K chunk starting at byte kb of every row into the panels at buf.
// `wave` must be wave-uniform (an SGPR).
__device__ __forceinline__ void dma_chunk(const uint8_t *A, const uint8_t *B, const uint32_t (&off)[kSlots], int wave,
                                          int64_t kb, uint4 *buf) {
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int first = (wave * kSlots + j) * 64;  // the wave's 64 slots lie in one panel
        dma16((first >= kPanel ? B : A) + kb, off[j], lds_addr(buf + first));
    }
}

// k-major operands (stored [K, rows], `stride` bytes per K row): a chunk's panel is 1024
// pieces, 32 fp32 K rows of 512 bytes (the tile's 128 rows, 32 pieces) or 64 bf16 K rows of
// 256 bytes (16 pieces), each K row's tile segment contiguous in memory.  Panel slot s holds K
// row s / PK at position s % PK (PK pieces per K row) of logical piece
//   fp32: (s % 32) ^ 8 for K rows 16..31 (columns xor 32: the two half-waves' 4-byte reads
//         below fall on different banks),
//   bf16: (s % 16) ^ 4 (kr & 3) (the four K rows of one transposing read land on disjoint
//         banks).
// Pieces past the operand's `lim` rows (a multiple of 16 / ES) read its last piece.
template <int ES>
__device__ __forceinline__ uint32_t kmajor_offset(int s, int64_t row0, int64_t lim, int64_t stride) {
    constexpr int PK = 128 * ES / 16, EPP = 16 / ES;  // pieces per K row, elements per piece
    const int kr = s / PK;
    const int lp = ES == 4 ? (s % PK) ^ ((kr >> 4) << 3) : (s % PK) ^ (4 * (kr & 3));
    int64_t r = row0 + EPP * lp;
    r = r < lim ? r : lim - EPP;
    return (uint32_t)(kr * stride + r * ES);
}

// dma_offsets for either panel stored k-major (AK: the A rows, BK: the B rows; `a_stride` /
// `b_stride` bytes per K row, ES bytes per element) or k-contiguous (`row_bytes` per row).
template <bool AK, bool BK, int ES = 4>
__device__ __forceinline__ void dma_offsets_k(uint32_t (&off)[kSlots], int wave, int lane, int64_t row0, int64_t col0,
                                              int64_t n, int64_t m, int64_t row_bytes, int64_t a_stride,
                                              int64_t b_stride) {
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int s = (wave * kSlots + j) * 64 + lane;
        const int panel = s >> 10;
        if ((panel == 0 && AK) || (panel == 1 && BK)) {
            off[j] = panel ? kmajor_offset<ES>(s & (kPanel - 1), col0, m, b_stride)
                           : kmajor_offset<ES>(s & (kPanel - 1), row0, n, a_stride);
        } else {
            const int r = (s >> 3) & (kT - 1), p = s & 7;
            const int64_t lim = panel ? m : n;
            int64_t row = (panel ? col0 : row0) + r;
            row = row < lim ? row : lim - 1;
            off[j] = (uint32_t)(row * row_bytes + swz(r, p) * 16);
        }
    }
}

// dma_chunk with a separate chunk offset per panel (ka bytes into A, kb into B).
__device__ __forceinline__ void dma_chunk2(const uint8_t *A, const uint8_t *B, const uint32_t (&off)[kSlots], int wave,
                                           int64_t ka, int64_t kb, uint4 *buf) {
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int first = (wave * kSlots + j) * 64;
        dma16(first >= kPanel ? B + kb : A + ka, off[j], lds_addr(buf + first));
    }
}

// One 16-byte K piece of the lane's two A rows and two B rows into the 2 x 2 accumulator
// blocks, formed transposed (B rows as the MFMA's first operand): the accumulators hold four
// consecutive output columns per register quad.  fp32: four 32x32x2 steps; bf16: one 32x32x16.
__device__ __forceinline__ void mfma_piece_t(floatx16 (&acc)[2][2], const uint4 (&a)[2], const uint4 (&b)[2], float) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const uint32_t av = e == 0 ? a[mi].x : e == 1 ? a[mi].y : e == 2 ? a[mi].z : a[mi].w;
                const uint32_t bv = e == 0 ? b[ni].x : e == 1 ? b[ni].y : e == 2 ? b[ni].z : b[ni].w;
                acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(bv), __uint_as_float(av),
                                                                  acc[mi][ni], 0, 0, 0);
            }
        }
    }
}
__device__ __forceinline__ void mfma_piece_t(floatx16 (&acc)[2][2], const uint4 (&a)[2], const uint4 (&b)[2],
                                             uint16_t) {
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8, b[ni]), __builtin_bit_cast(bf16x8, a[mi]), acc[mi][ni], 0, 0, 0);
        }
    }
}

// Logical piece c of row r of a panel.
__device__ __forceinline__ uint4 piece(const uint4 *panel, int r, int c) { return panel[r * 8 + swz(r, c)]; }

// The fp32 values at K = 16 h + 4 q + (0..3) of row r of a k-major panel, as one piece (the same
// K order as piece(panel, r, 4 h + q) of a k-contiguous panel).
__device__ __forceinline__ uint4 kpiece(const uint4 *panel, int r, int h, int q) {
    const float *f = reinterpret_cast<const float *>(panel) + (16 * h + 4 * q) * kT + (r ^ (32 * h));
    return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[kT]), __float_as_uint(f[2 * kT]),
                      __float_as_uint(f[3 * kT]));
}

// The bf16 values at K = 32 h + 8 q + (0..7) of row rb + (lane % 16) of a k-major panel, as
// one piece (the same K order as piece(panel, r, 4 h + q) of a k-contiguous bf16 panel); rb is
// the first of the 16 rows that the lane's group of 16 lanes covers (a multiple of 16).  Two
// transposing reads (ds_read_b64_tr_b16): within a group of 16 lanes, lane j points at the 4
// elements of K row K0 + j / 4, rows rb + 4 (j % 4) .. + 3, and lane i receives K rows
// K0 .. K0 + 3 of row rb + i.  KRB: bytes per K row in the panel (256: 128 tile rows; 512:
// 256), piece positions xor 4 (kr & 3).
template <int KRB = 256>
__device__ __forceinline__ uint4 kpiece_bf16(const uint4 *panel, int rb, int lane, int h, int q) {
    typedef short v4s __attribute__((ext_vector_type(4)));
    const int j = lane & 15;
    uint2 v[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int kr = 32 * h + 8 * q + 4 * t + (j >> 2);
        const int byte = 2 * (rb + 4 * (j & 3));  // in the K row's tile segment
        const int pos = (byte >> 4) ^ (4 * (kr & 3));
        const uint8_t *addr = reinterpret_cast<const uint8_t *>(panel) + kr * KRB + pos * 16 + (byte & 15);
        const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4s *)(uintptr_t)lds_addr(addr));
        v[t] = __builtin_bit_cast(uint2, r);
    }
    return make_uint4(v[0].x, v[0].y, v[1].x, v[1].y);
}

// A 16-byte output store: non-temporal (kNT), or a plain store that the L2 holds and combines
// with the neighbouring waves' pieces of the same rows before write-back (faster for the
// output-bound boolean kernels, slower by 1-2 % for the matrix-core-bound distance kernels).
template <bool kNT, typename V>
__device__ __forceinline__ void store16(V *p, V v) {
    if constexpr (kNT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

// One wave's 32 x (32 NI) fp32 outputs through its own LDS slice `sl` (NI * 4 KiB; no
// workgroup barrier), written as (NI * 128)-byte row segments, 8 NI lanes per row.  value(ni,
// g) returns the lane's register quad g of block ni: row grow0 + l32, columns gcol0 + 32 ni +
// 8 g + 4 h + (0..3).  Rows >= n and columns >= m are not stored (m a multiple of 4, out
// 16-byte aligned).  Stage unit u of row r sits at u ^ (r & 15).  With `ragged` (rows of
// m % 4 != 0 floats, so no 16-byte row segments) each store instruction writes one row's
// 32 NI values instead, a dword per lane: 128 NI contiguous bytes, 32 instructions per slice.
template <int NI, bool kNT = true, class F>
__device__ __forceinline__ void store_wave_rows_f32(floatx4 *sl, F &&value, float *__restrict__ out, int64_t b,
                                                    int64_t grow0, int64_t gcol0, int64_t n, int64_t m,
                                                    bool ragged = false) {
    constexpr int U = NI * 8;    // 16-byte units per stage row
    constexpr int RPI = 64 / U;  // rows per store instruction
    const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
    const int ul = lane % U, rl = lane / U;
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int u = ni * 8 + 2 * g + h;
            sl[l32 * U + (u ^ (l32 & 15))] = value(ni, g);
        }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    if (ragged) {
        const float *sf = reinterpret_cast<const float *>(sl);
        const int c = lane % (32 * NI);
        const int64_t gcol = gcol0 + c;
        const bool col_ok = lane < 32 * NI && gcol < m;
#pragma unroll 8
        for (int r = 0; r < 32; ++r) {
            const float v = sf[(r * U + ((c >> 2) ^ (r & 15))) * 4 + (c & 3)];
            const int64_t grow = grow0 + r;
            if (col_ok && grow < n) store16<kNT>(out + (b * n + grow) * m + gcol, v);
        }
    } else {
        const int64_t gcol = gcol0 + 4 * ul;
#pragma unroll
        for (int it = 0; it < 32 / RPI; ++it) {
            const int r = it * RPI + rl;
            const floatx4 v = sl[r * U + (ul ^ (r & 15))];
            const int64_t grow = grow0 + r;
            if (grow < n && gcol < m) store16<kNT>(reinterpret_cast<floatx4 *>(out + (b * n + grow) * m + gcol), v);
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the slice is rewritten
    __builtin_amdgcn_wave_barrier();
}

// The same for bf16 outputs (rounded to nearest even): 32 x (32 NI) values through an (NI * 2)
// KiB slice, (NI * 64)-byte row segments, 4 NI lanes per row; m a multiple of 8.
template <int NI, bool kNT = true, class F>
__device__ __forceinline__ void store_wave_rows_bf16(uint4 *sl, F &&value, uint16_t *__restrict__ out, int64_t b,
                                                     int64_t grow0, int64_t gcol0, int64_t n, int64_t m) {
    constexpr int U = NI * 4;    // 16-byte units (8 values) per stage row
    constexpr int RPI = 64 / U;  // rows per store instruction
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
    const int ul = lane % U, rl = lane / U;
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const floatx4 o = value(ni, g);
            const int u = ni * 4 + g;  // columns 8 g .. 8 g + 7 of block ni; this lane's half h
            reinterpret_cast<uint2 *>(sl)[(l32 * U + (u ^ (l32 & 15))) * 2 + h] =
                make_uint2(f32x2_to_bf16x2_rne(o[0], o[1]), f32x2_to_bf16x2_rne(o[2], o[3]));
        }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    const int64_t gcol = gcol0 + 8 * ul;
#pragma unroll
    for (int it = 0; it < 32 / RPI; ++it) {
        const int r = it * RPI + rl;
        const u32x4 v = reinterpret_cast<const u32x4 *>(sl)[r * U + (ul ^ (r & 15))];
        const int64_t grow = grow0 + r;
        if (grow < n && gcol < m) store16<kNT>(reinterpret_cast<u32x4 *>(out + (b * n + grow) * m + gcol), v);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the slice is rewritten
    __builtin_amdgcn_wave_barrier();
}

// Writes the tile through the LDS stage `st` (>= 32 KiB, free) in row segments.  value(mi, ni,
// g) returns the 4 outputs of the lane's register quad g of block (mi, ni) as float: row
// wr + 32 mi + l32, columns wc + 32 ni + 8 g + 4 h + (0..3).  Rows >= n and columns >= m are not
// stored; m must be a multiple of 16 / sizeof(OutT) and out 16-byte aligned (a 16-byte store
// unit is then wholly inside or outside), except that fp32 and bf16 outputs take any m with
// `ragged` set (fp32: dword row stores, store_wave_rows_f32; bf16: whole 16-byte units
// funnel-shifted from the stage, 2-byte stores for each row piece's head and tail).  bf16 stages the rounded values of the whole tile (one
// pass of 128 rows x 256 bytes, one workgroup barrier); fp32 per wave (store_wave_rows_f32, an
// 8 KiB slice each).  Stage unit u of row r sits at u ^ (r & 15): conflict-free 16-byte accesses
// across 16 rows and within 16-unit groups.
template <typename OutT, bool kNT = true, class F>
__device__ __forceinline__ void store_tile(uint4 *st, F &&value, OutT *__restrict__ out, int64_t b, int64_t row0,
                                           int64_t col0, int64_t n, int64_t m, bool ragged = false) {
    if constexpr (sizeof(OutT) == 4) {
        const int wave = threadIdx.x >> 6;
        const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
        floatx4 *sl = reinterpret_cast<floatx4 *>(st) + wave * 512;
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
            store_wave_rows_f32<2, kNT>(
                sl, [&](int ni, int g) { return value(mi, ni, g); }, out, b, row0 + wr + mi * 32, col0 + wc, n, m,
                ragged);
        return;
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
    const int l32 = lane & 31, h = lane >> 5;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    constexpr int UPR = kT * (int)sizeof(OutT) / 16;  // 16-byte units per stage row
    constexpr int XM = UPR < 16 ? UPR - 1 : 15;       // unit swizzle mask (stays inside the row)
    constexpr int PR = kBuf * 16 / (kT * (int)sizeof(OutT)) < kT ? kBuf * 16 / (kT * (int)sizeof(OutT)) : kT;
    constexpr int NPASS = kT / PR;
    constexpr int LPR = UPR;     // lanes per row when storing
    constexpr int RPI = 64 / LPR;  // rows per store instruction
    constexpr int ITERS = PR / (4 * RPI);
    static_assert(PR % 64 == 0 && ITERS * 4 * RPI == PR, "stage geometry");
#pragma unroll
    for (int pass = 0; pass < NPASS; ++pass) {
        if (NPASS == 1 || wr / PR == pass) {
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) {
                const int r = wr + mi * 32 + l32 - pass * PR;  // row within the pass
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const floatx4 o = value(mi, ni, g);
                        const int col = wc + ni * 32 + 8 * g + 4 * h;
                        if constexpr (sizeof(OutT) == 2) {
                            const int u = col >> 3;
                            reinterpret_cast<uint2 *>(st)[(r * UPR + (u ^ (r & XM))) * 2 + h] =
                                make_uint2(f32x2_to_bf16x2_rne(o[0], o[1]), f32x2_to_bf16x2_rne(o[2], o[3]));
                        } else if constexpr (sizeof(OutT) == 1) {
                            // bool bytes: 1 where the value is not 0
                            const int u = col >> 4;
                            const uint32_t q = (uint32_t)(o[0] != 0.0f) | (uint32_t)(o[1] != 0.0f) << 8 |
                                               (uint32_t)(o[2] != 0.0f) << 16 | (uint32_t)(o[3] != 0.0f) << 24;
                            reinterpret_cast<uint32_t *>(st)[(r * UPR + (u ^ (r & XM))) * 4 + ((col >> 2) & 3)] = q;
                        } else {
                            const int u = col >> 2;
                            reinterpret_cast<floatx4 *>(st)[r * UPR + (u ^ (r & 15))] = o;
                        }
                    }
            }
        }
        barrier_lds();
        if constexpr (sizeof(OutT) == 2) {
            if (ragged) {
                // rows of m % 8 != 0 values: a row piece starts anywhere inside a 16-byte unit
                // (out itself 16-byte aligned).  16 lanes per row write the piece's whole units,
                // each funnel-shifted from two stage units; then 16 lanes per row its head and
                // tail values (at most 7 + 7), 2 bytes each.
                static_assert(NPASS == 1 && RPI == 4, "bf16 stage geometry");
                const int j = lane & 15, rq = lane >> 4;
                const uint16_t *sh = reinterpret_cast<const uint16_t *>(st);
                const int V = (int)(m - col0 < kT ? m - col0 : kT);  // values in the piece
#pragma unroll 2
                for (int it = 0; it < ITERS; ++it) {
                    const int r = (wave * ITERS + it) * RPI + rq;
                    const int64_t grow = row0 + r;
                    if (grow >= n) continue;
                    const int64_t e0 = (b * n + grow) * m + col0;  // the piece's first value
                    const int sft = (int)((8 - (e0 & 7)) & 7);     // values before the first unit
                    const int K = V > sft ? (V - sft) >> 3 : 0;    // whole units
                    if (j < K) {
                        const int c0 = sft + 8 * j, u0 = c0 >> 3;  // value c0 sits at c0 & 7 = sft
                        const u32x4 A = reinterpret_cast<const u32x4 *>(st)[r * UPR + (u0 ^ (r & XM))];
                        const u32x4 B = sft != 0 ? reinterpret_cast<const u32x4 *>(st)[r * UPR + ((u0 + 1) ^ (r & XM))] : A;
                        const uint32_t w[8] = {A[0], A[1], A[2], A[3], B[0], B[1], B[2], B[3]};
                        const int q = sft >> 1;
                        u32x4 o;
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const uint32_t lo = q == 0 ? w[k] : q == 1 ? w[k + 1] : q == 2 ? w[k + 2] : w[k + 3];
                            const uint32_t hi = q == 0 ? w[k + 1] : q == 1 ? w[k + 2] : q == 2 ? w[k + 3] : w[k + 4];
                            o[k] = (sft & 1) ? (lo >> 16) | (hi << 16) : lo;
                        }
                        store16<kNT>(reinterpret_cast<u32x4 *>(out + e0 + c0), o);
                    }
                    const int headN = sft < V ? sft : V, tail0 = sft + 8 * K;
                    const int tailN = V > tail0 ? V - tail0 : 0;
                    if (j < headN + tailN) {
                        const int c = j < headN ? j : tail0 + (j - headN);
                        store16<kNT>(reinterpret_cast<uint16_t *>(out + e0 + c),
                                     sh[(r * UPR + ((c >> 3) ^ (r & XM))) * 8 + (c & 7)]);
                    }
                }
                return;
            }
        }
        const int ul = lane % LPR, rl = lane / LPR;
        const int64_t gcol = col0 + ul * (16 / (int)sizeof(OutT));
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const int r = (wave * ITERS + it) * RPI + rl;
            const u32x4 v = reinterpret_cast<const u32x4 *>(st)[r * UPR + (ul ^ (r & XM))];
            const int64_t grow = row0 + pass * PR + r;
            if (grow < n && gcol < m) store16<kNT>(reinterpret_cast<u32x4 *>(out + (b * n + grow) * m + gcol), v);
        }
        if (pass + 1 < NPASS) barrier_lds();  // the next pass rewrites the stage
    }
}

}  // namespace tile
}  // namespace tpw
