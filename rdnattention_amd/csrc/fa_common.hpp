// Shared device-side building blocks for the gfx950 (CDNA4) attention kernels.
//
// Everything here is written for 64-lane wavefronts and the CDNA4 matrix
// cores.  The MFMA operand conventions the kernels rely on:
//
//   v_mfma_f32_32x32x16_f16   D[32x32] += A[32x16] * B[16x32]
//     A: lane l holds 8 halves of row m = l%32, reduction slots of group g = l/32
//     B: lane l holds 8 halves of column n = l%32, the same reduction slots
//     D: lane l holds D[8*(i/4) + 4*g + (i%4)][l%32], i = 0..15
//
// Only the D layout is load-bearing.  The reduction-slot order inside an
// A/B register is the same for A and B, so any consistent assignment of the
// reduction index to (g, element) gives the same dot product; the kernels
// pick the one that makes every operand a single 16-byte LDS read.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "fa_mask.hpp"

namespace rdna_amd {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef int i4 __attribute__((ext_vector_type(4)));
typedef int i16x __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f16x mfma_32x32x16_f16(h8 a, h8 b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ i16x mfma_32x32x32_i8(i4 a, i4 b, i16x c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) {
    // v_exp_f32: 2^x; exp2(-inf) = 0.
    return __builtin_amdgcn_exp2f(x);
}

// ds_read_b64_tr_b16 (gfx950 LDS transpose read).  Within each 16-lane
// group, lane i receives as half k the half (i % 4) of the 8-byte word whose
// address lane 4k + i/4 supplies.  So if lane j of the group points at
// row (j / 4), columns 4 * (j % 4) .. +3 of a row-major 4 x 16 block, lane i
// gets column i of the block: the four rows' values, i.e. a transposed read.
typedef __fp16 fp16x4_raw __attribute__((__vector_size__(4 * sizeof(__fp16))));
__device__ __forceinline__ h4 lds_read_tr16(const _Float16* p) {
    typedef __attribute__((address_space(3))) fp16x4_raw lds_h4;
    const auto* lp = reinterpret_cast<const __attribute__((address_space(3))) char*>(
        (uint32_t)reinterpret_cast<uintptr_t>(p));
    fp16x4_raw r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_h4*)lp);
    return __builtin_bit_cast(h4, r);
}

// max(x[l], x[l ^ 32]): combine the two half-waves that hold the same query
// column.  v_permlane32_swap exchanges lanes 0-31 of one operand with lanes
// 32-63 of the other, so the pair {r[0], r[1]} is {x[l % 32], x[32 + l % 32]}
// in every lane.
__device__ __forceinline__ float pair_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float pair_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// acc + the sum of the eight halves of v, two per v_dot2c_f32_f16 (fp32
// accumulation).  Used for the softmax row sum: summing the fp16 P that the
// P V MFMA consumes keeps numerator and denominator on the same weights.
__device__ __forceinline__ float sum_h8(h8 v, float acc) {
    const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        const h2 pr = {v[e], v[e + 1]};
        acc = __builtin_amdgcn_fdot2(pr, one, acc, false);
    }
    return acc;
}

// Max of v(0) .. v(N - 1) as a tree of v_max3 (depth ceil(log3 N)) instead of
// a chain: dependent VALU instructions issue about 8 cycles apart (a chain of
// dependent fmas measured 7.8 cycles each), so the 16-deep v_max3 chain of a
// 32-score row cost ~130 cycles of latency before any exponential could start.
template <int N, class V>
__device__ __forceinline__ float max_tree(V&& v) {
    static_assert(N >= 1, "max of no values");
    if constexpr (N == 1) {
        return v(0);
    } else if constexpr (N == 2) {
        return fmaxf(v(0), v(1));
    } else if constexpr (N == 3) {
        return fmaxf(fmaxf(v(0), v(1)), v(2));
    } else {
        constexpr int M = (N + 2) / 3;
        float m[M];
#pragma unroll
        for (int i = 0; i < M; i++) {
            m[i] = 3 * i + 2 < N ? fmaxf(fmaxf(v(3 * i), v(3 * i + 1)), v(3 * i + 2))
                                 : (3 * i + 1 < N ? fmaxf(v(3 * i), v(3 * i + 1)) : v(3 * i));
        }
        return max_tree<M>([&](int i) { return m[i]; });
    }
}

// acc + the sum of the 32 halves of p[0..3], as four independent v_dot2c
// chains of four (sum_h8 each) added in a fixed order, instead of one chain
// of sixteen
__device__ __forceinline__ float sum_h8x4(const h8 (&p)[4], float acc) {
    const float s0 = sum_h8(p[0], 0.0f), s1 = sum_h8(p[1], 0.0f);
    const float s2 = sum_h8(p[2], 0.0f), s3 = sum_h8(p[3], 0.0f);
    return acc + ((s0 + s1) + (s2 + s3));
}

// s_waitcnt immediates (gfx9 encoding: vmcnt [3:0] and [15:14], expcnt
// [6:4], lgkmcnt [11:8]); the counters not named are left unwaited.
constexpr int waitcnt_vm(int n) {
    return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8);
}
constexpr int waitcnt_lgkm(int n) {
    return 0xf | (0x3 << 14) | (0x7 << 4) | ((n & 0xf) << 8);
}

__device__ __forceinline__ bool wave_any(bool pred) {
    return __builtin_amdgcn_ballot_w64(pred) != 0;
}

// Workgroup -> (head group, row tile).  The hardware deals workgroups to the
// 8 XCDs round-robin (wg % 8), each XCD with its own L2.  With chunk > 0 (and
// n_hg a multiple of 8 * chunk) each XCD works through `chunk` head groups at
// a time, all of their row tiles heaviest first, so the K/V those concurrent
// workgroups stream stays in that XCD's L2; chunk == 0 keeps head groups
// fastest over the whole grid.
__device__ __forceinline__ void wg_tile(int wg, int n_hg, int n_rt, int chunk, int& hg, int& rt) {
    if (chunk > 0) {
        const int xcd = wg & 7;
        const int slot = wg >> 3;
        const int per_chunk = chunk * n_rt;
        const int c = slot / per_chunk;
        const int idx = slot - c * per_chunk;
        rt = n_rt - 1 - idx / chunk;
        hg = xcd + 8 * (c * chunk + idx % chunk);
    } else {
        hg = wg % n_hg;
        rt = n_rt - 1 - wg / n_hg;
    }
}

// Output tile of one wave: 32 query rows (q0 + l32, l32 = lane % 32) x D
// columns held as O^T MFMA accumulators (oacc[dt][4 qq + e] = column
// dt*32 + 8 qq + 4 g + e, g = lane / 32), each scaled by factors(d0)[e] with
// d0 = dt*32 + 8 qq + 4 g, rounded to fp16 and stored to rows q0 .. q0 + 31
// (those < sq) at obase + row * o_ss. The tile passes through `slot`, 32 rows
// at a stride of LDO halves in LDS that only this wave uses: written in the
// accumulator layout, read back along rows and stored 16 bytes per lane, so
// every store instruction writes whole rows (full cache lines). The stores
// are non-temporal: the output is not read again, and streaming it past the
// L2 keeps the K/V tiles that other row tiles reuse resident. (Stored from the
// accumulator layout, one instruction writes 8 bytes of 32 rows, and such
// partial lines must merge in the L2.)
template <int D, int LDO, class Factors>
__device__ __forceinline__ void store_o_tile(const f16x (&oacc)[D / 32], Factors&& factors, _Float16* slot,
                                             _Float16* obase, int q0, int sq, int64_t o_ss, int lane) {
    const int l32 = lane & 31;
    const int g = lane >> 5;
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++) {
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            const int d0 = dt * 32 + 8 * qq + 4 * g;
            const f4 c = factors(d0);
            h4 o4 = {(_Float16)(oacc[dt][4 * qq + 0] * c[0]), (_Float16)(oacc[dt][4 * qq + 1] * c[1]),
                     (_Float16)(oacc[dt][4 * qq + 2] * c[2]), (_Float16)(oacc[dt][4 * qq + 3] * c[3])};
            *reinterpret_cast<h4*>(slot + l32 * LDO + d0) = o4;
        }
    }
    // LPR lanes per row (D/8 of them active), RPI rows per instruction; the
    // indices come from an opaque copy of the lane id so that the compiler
    // cannot hoist the addresses above the caller's key-tile loop (they would
    // stay live through it)
    constexpr int OCH = D / 8;
    static_assert(D % 32 == 0 && OCH <= 64, "output tile width");
    constexpr int LPR = OCH <= 4 ? 4 : (OCH <= 8 ? 8 : (OCH <= 16 ? 16 : (OCH <= 32 ? 32 : 64)));
    constexpr int RPI = 64 / LPR;
    int lane_e = lane;
    asm volatile("" : "+v"(lane_e));
    const int r0 = lane_e / LPR;
    const int ch = lane_e % LPR;
    _Float16* const orow0 = obase + (int64_t)(q0 + r0) * o_ss + 8 * ch;
#pragma unroll
    for (int c = 0; c < 32 / RPI; c++) {
        const int r = r0 + RPI * c;
        if (ch < OCH) {
            const h8 o8 = *reinterpret_cast<const h8*>(slot + r * LDO + 8 * ch);
            if (q0 + r < sq) {
                __builtin_nontemporal_store(o8, reinterpret_cast<h8*>(orow0 + (int64_t)(RPI * c) * o_ss));
            }
        }
    }
}

// Work item `k` of persistent workgroup `w` in a grid of `P`, for `n` items
// numbered like the workgroups of a one-item-per-workgroup grid (which
// wg_tile places on XCD id % 8); -1 once the workgroup has none left.
// Workgroups go to the XCDs round-robin, so with P a multiple of 8 workgroup
// w takes only ids of its own XCD: in rounds of P/8 ids, dealt in alternating
// (snake) order so that the heaviest and lightest row tiles of a round pair
// up. Every id < n is taken exactly once (each round's slots map one-to-one
// onto the XCD's workgroups), and a workgroup's ids increase with k.
__device__ __forceinline__ int persistent_item(int w, int P, int k, int n) {
    int id;
    if ((P & 7) == 0) {
        const int per_xcd = P >> 3;
        const int l = w >> 3;
        const int slot = (k & 1) ? per_xcd - 1 - l : l;
        id = (w & 7) + 8 * (k * per_xcd + slot);
    } else {
        id = w + k * P;
    }
    return id < n ? id : -1;
}

// Raw buffer resource (gfx9 V#: stride 0, DATA_FORMAT 32): loads at byte
// offsets >= num_records return 0, which is how rows past the end of K/V read
// as zeros without per-load branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t num_records) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)num_records, 0x00020000);
}

// make_rsrc of wave-uniform values that the compiler may hold in vector
// registers (a phi behind a lane-dependent branch): it would otherwise wrap
// every load through the descriptor in a loop over its distinct values.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_uniform(uint64_t base, uint32_t num_records) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32));
    return make_rsrc(reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo),
                     (uint32_t)__builtin_amdgcn_readfirstlane((int)num_records));
}

__device__ __forceinline__ h8 buffer_load_h8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    u4 x = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return __builtin_bit_cast(h8, x);
}

// HBM -> LDS copy of 16 bytes per lane (buffer_load_dwordx4 ... lds): lane i
// reads the buffer at voff and writes LDS bytes [lds + 16 i, lds + 16 i + 16).
// Issued from inline asm so the compiler's waitcnt insertion does not treat it
// as a store to every LDS location (it would otherwise wait for all of them
// before each LDS read); callers wait on vmcnt themselves.  The V# is built
// by hand: base, stride 0, num_records, DATA_FORMAT 32.
typedef int i32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4_t make_rsrc_v(const void* base, uint32_t num_records) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    i32x4_t r;
    r[0] = (int)(uint32_t)a;
    r[1] = (int)(uint32_t)(a >> 32);
    r[2] = (int)num_records;
    r[3] = 0x00020000;
    return r;
}
__device__ __forceinline__ void dma_load16(i32x4_t rsrc, uint32_t voff, uint32_t lds_byte_addr) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(lds_byte_addr)
                 : "memory", "m0");
}
// HBM -> LDS copy of 4 bytes per lane (buffer_load_dword ... lds): lane i
// reads the dword at voff and writes LDS bytes [lds + 4 i, lds + 4 i + 4).
// Each lane's dword is range-checked on its own, so a vector of floats that
// ends inside a 16-byte chunk is copied exactly.
__device__ __forceinline__ void dma_load4(i32x4_t rsrc, uint32_t voff, uint32_t lds_byte_addr) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dword %0, %1, 0 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(lds_byte_addr)
                 : "memory", "m0");
}
// dma_load16 with a wave-uniform byte offset `soff` (the instruction's scalar
// offset) added to voff: a loop over rows then keeps one vector offset.
__device__ __forceinline__ void dma_load16_s(i32x4_t rsrc, uint32_t voff, uint32_t soff, uint32_t lds_byte_addr) {
    asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(soff), "s"(lds_byte_addr)
                 : "memory", "m0");
}
// dma_load16 with the non-temporal cache policy, for bytes read exactly once
// (split-K decode streams K/V once): they then do not displace lines that are
// reused. Kernels whose workgroups share K/V through the L2 use dma_load16.
__device__ __forceinline__ void dma_load16_nt(i32x4_t rsrc, uint32_t voff, uint32_t lds_byte_addr) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(lds_byte_addr)
                 : "memory", "m0");
}

// Bytes of one key tile: min(rows_left, TILE_ROWS) rows of row_bytes at a
// stride of stride_bytes (<= 2^25 and TILE_ROWS <= 64, so the result fits 32
// bits), 0 when rows_left <= 0.
template <int TILE_ROWS>
__device__ __forceinline__ uint32_t tile_bytes(int rows_left, uint32_t stride_bytes, uint32_t row_bytes) {
    static_assert(TILE_ROWS <= 64, "tile byte range must fit 32 bits");
    if (rows_left <= 0) {
        return 0;
    }
    const uint32_t rows = (uint32_t)(rows_left < TILE_ROWS ? rows_left : TILE_ROWS);
    return (rows - 1) * stride_bytes + row_bytes;
}

// RoPE on 8 consecutive channels (4 interleaved pairs) of one row:
// (a, b) -> (a*c - b*s, a*s + b*c) in fp32, rounded to fp16, where c/s are
// table columns col0 .. col0+3 (src/rdna/fa2_forward_f16.hip:63-77).
__device__ __forceinline__ h8 rope8_cs(h8 x, f4 c, f4 s) {
    h8 y;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float a = (float)x[2 * i];
        float b = (float)x[2 * i + 1];
        y[2 * i] = (_Float16)(a * c[i] - b * s[i]);
        y[2 * i + 1] = (_Float16)(a * s[i] + b * c[i]);
    }
    return y;
}

// rope8_cs with the rotated values multiplied by `mul` before the one
// rounding to fp16
__device__ __forceinline__ h8 rope8_cs_mul(h8 x, f4 c, f4 s, float mul) {
    h8 y;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float a = (float)x[2 * i];
        float b = (float)x[2 * i + 1];
        y[2 * i] = (_Float16)((a * c[i] - b * s[i]) * mul);
        y[2 * i + 1] = (_Float16)((a * s[i] + b * c[i]) * mul);
    }
    return y;
}

// fp16(x * mul), one rounding
__device__ __forceinline__ h8 scale8(h8 x, float mul) {
    h8 y;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        y[e] = (_Float16)((float)x[e] * mul);
    }
    return y;
}

__device__ __forceinline__ h8 rope8(h8 x, const float* cos_row, const float* sin_row, int col0) {
    return rope8_cs(x, *reinterpret_cast<const f4*>(cos_row + col0), *reinterpret_cast<const f4*>(sin_row + col0));
}

// Q^T operand of one query row for the 32x32x16 MFMAs: out[s] = Q[row][16s + 8g .. +7],
// RoPE-rotated with the table row of this position when `rope`, negated when `neg`, zero
// when !valid. `qrow`, `cos_row` and `sin_row` must point at readable rows even when
// !valid. Within a chunk of CH slices every load is issued before any is used, so a chunk
// costs one memory round trip (with the RoPE loads inside a per-slice branch the compiler
// waited for each slice's loads in turn); chunks bound the registers the tables hold
// (a D = 512 row with all its tables live would need 384).
//
// With `mul` != 0 the values are multiplied by mul in fp32 before their one
// rounding to fp16 (and `neg` is ignored: the sign is mul's), the
// pre-scaling of the kernels whose QK^T yields log2-unit scores.
template <int NS, int CH = NS>
__device__ __forceinline__ void load_q_operand(h8 (&out)[NS], const _Float16* qrow, const float* cos_row,
                                               const float* sin_row, int g, bool valid, bool rope, bool neg,
                                               float mul = 0.0f) {
#pragma unroll
    for (int s0 = 0; s0 < NS; s0 += CH) {
        constexpr int n = CH; // the last chunk may be partial: slices s0 + s >= NS are skipped
        h8 x[n];
#pragma unroll
        for (int s = 0; s < n; s++) {
            if (s0 + s < NS) {
                x[s] = *reinterpret_cast<const h8*>(qrow + 16 * (s0 + s) + 8 * g);
            }
        }
        if (rope) {
            f4 c[n], sn[n];
#pragma unroll
            for (int s = 0; s < n; s++) {
                if (s0 + s < NS) {
                    c[s] = *reinterpret_cast<const f4*>(cos_row + 8 * (s0 + s) + 4 * g);
                    sn[s] = *reinterpret_cast<const f4*>(sin_row + 8 * (s0 + s) + 4 * g);
                }
            }
#pragma unroll
            for (int s = 0; s < n; s++) {
                if (s0 + s < NS) {
                    x[s] = mul != 0.0f ? rope8_cs_mul(x[s], c[s], sn[s], mul) : rope8_cs(x[s], c[s], sn[s]);
                }
            }
        } else if (mul != 0.0f) {
#pragma unroll
            for (int s = 0; s < n; s++) {
                if (s0 + s < NS) {
                    x[s] = scale8(x[s], mul);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < n; s++) {
            if (s0 + s < NS) {
                out[s0 + s] = valid ? ((neg && mul == 0.0f) ? -x[s] : x[s]) : h8{};
            }
        }
        // the next chunk's loads are not hoisted above this chunk's rotation
        __builtin_amdgcn_sched_barrier(0);
    }
}

} // namespace rdna_amd
