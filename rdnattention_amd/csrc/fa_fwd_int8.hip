// INT8 FlashAttention forward for gfx950 at head_dim 64: Q K^T and P V both on
// int8 MFMA (v_mfma_i32_32x32x32_i8, exact int32 accumulation), fp16 output.
// Head_dim 128 and the per-token V scale run fa_fwd_int8_f16pv.hip (P V on
// fp16 MFMA; its header gives the measured reason).  This file also holds the
// INT8 host entry (fwd_int8, the score export, the launch parameters).
//
// Replaces the reference's forwardKernelInt8QK
// (src/rdna/fa2_forward_int8qk.hip:229-495) and keeps its numeric scheme:
//
//   S_ij  = sum_d q_i8 k_i8                          (exact int32, :254-278)
//   s_ij  = S_ij * qs_i * ks_j * scale * log2(e)      (fp32, log2 domain, :301)
//   per 64-key block, aligned to key 0 (the reference's Bc = 64):
//     m'  = max(m, max_j s_ij);  O *= 2^(m - m'),  l *= 2^(m - m')
//     p   = 2^(s - m'),  l += sum p                  (unquantised p)
//     pq  = min(127, round(p * 127))                 (P as integers 0..127)
//     O  += sum_j pq_j v_j                           (exact int32, :354-382)
//   out = O * v_scale / (127 l)  (0 when no key is visible)
//
// O is held as O_f * 2^(m_a - m_c) + O_int: O_int is the int32 accumulator of
// the P V MFMAs, the exact sum of every block since the running maxima of the
// wave's 32 query rows last moved (all relative to the current maxima m_c),
// and O_f (fp32, relative to m_a) holds everything before.  While no row
// maximum moves, blocks accumulate in int32 with no VALU work at all; when one
// moves, the wave folds O_int into O_f once (one conversion and one fma per
// accumulator) and restarts the int32 chain; it also folds after kI8FoldTiles
// tiles without a move, before the int32 sums could overflow.  Each block's sum is therefore
// the reference's exact int32 sum, and its weight 2^(m_b - m_final) is applied
// in fp32 as the reference's per-block rescale does.
//
// Deliberate differences, all far below the INT8 tolerance: round() is
// round-half-to-even (v_cvt_pk_u8_f32) where the reference calls lroundf
// (half away from zero), 127 p is evaluated as 2^(s - m' + log2 127) (kept at
// most 127 by the exponent offset, int8_exp_offset, so the min(127) is
// implied and a quantised P never reaches 128, which the signed int8 MFMA
// operand would read as -128), s is formed as
// (S * ks) * (qs * scale * log2(e)), and v_scale/127 is applied once at the end.
//
// Kernel structure: 8 waves in two groups of four that alternate an MFMA phase
// (P V of the previous tile, Q K^T of this one) and a softmax phase, S^T = K Q^T
// so that a lane owns one query column, and P^T going from the softmax straight
// into the B operand of O^T = V^T P^T as packed bytes.  K, V and the per-token
// K scales go from HBM to LDS by DMA (buffer_load ... lds), issued by group A
// two tiles ahead into four tile slots, so neither group stages anything
// through registers.  Tiles are stored unpadded with 16-byte chunks swizzled
// per row (i8_swz); the V^T operands come from ds_read_b64_tr_b8 transpose
// reads.  The grid is persistent (persistent_item), and O leaves through an LDS
// buffer as whole-row non-temporal stores (store_o_tile).
//
// SCORES (a test instantiation): the same kernel with the softmax, P V and
// output compiled out; every S^T accumulator block its first GEMM produces is
// written to an int32 score buffer, so the tests can check the production
// GEMM's scores bit for bit.
#include "fa_common.hpp"
#include "fa_host.hpp"
#include "fa_int8.hpp"
#include "fa_internal.hpp"
#include "fa_prefill.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace rdna_amd {

#if !defined(RDNATTENTION_NO_INT8)

namespace {

typedef int i2 __attribute__((ext_vector_type(2)));

constexpr int kI8Slots = 4;                  // K/V tile slots in LDS (DMAs run two tiles ahead)
constexpr int kI8OpDepth = 4;                // LDS operands in flight in the MFMA phase
// P V tiles the int32 accumulators may sum between two folds: each tile adds
// at most 64 * 127 * 127 = 1032256 per accumulator, so 1024 tiles stay below
// 2^30 (2080 would pass 2^31)
constexpr int kI8FoldTiles = 1024;

template <int D>
struct I8Cfg {
    // One wave per 32 query rows holds 32 + 32 O^T accumulators (int32 and
    // fp32) at D = 64; at D = 128 they would take 128 registers (see the
    // header), so this kernel is built for D = 64 only.
    static_assert(D == 64, "head_dim 128 runs fa_fwd_int8_f16pv");
    static constexpr int CH = D / 16;          // 16-byte chunks per int8 row
    static constexpr int TILE = kI8BN * D;     // bytes of one K (or V) tile, rows unpadded
    static constexpr int BLOCKS = TILE / 1024; // 1 KB DMA blocks (64 lanes x 16 bytes) per tile
    static constexpr int BPW = BLOCKS / 4;     // blocks per issuing wave (group A's four waves)
    static constexpr int NS = D / 32;          // Q K^T reduction steps (32 per MFMA)
    static constexpr int NDT = D / 32;         // O^T row tiles (32 columns each)
    static constexpr int QB = 32 * D / 1024;   // DMA blocks of one wave's 32 Q rows
    static constexpr int LDO = D + 8;          // halves; output staging rows (conflict-free)
    static_assert(BLOCKS % 4 == 0 && BPW >= 1 && QB >= 1, "tiles split into whole DMA blocks per wave");
    static_assert(NS * 2 * 8 == 16 * NDT, "the fold rides on the Q K^T MFMAs, 8 accumulators each");
};

// Chunk swizzle of the K, V and Q tiles in LDS (64-byte rows): byte b of
// 16-byte chunk c of tile row r sits at r * 64 + 16 * (c ^ i8_swz(r)) + b.
// The two read patterns then use every bank once per 256 bytes:
//   K and Q operands (ds_read_b128): 16 consecutive rows, one chunk;
//   V^T operand (ds_read_b64_tr_b8): rows {0-3, 8-11} + 4 g, two adjacent
//   chunks, two 8-byte halves each, over 32 lanes.
// The swizzle depends only on row bits 2-3, so rows 16 and 32 apart share it.
__host__ __device__ constexpr int i8_swz(int r) {
    return (r >> 2) & 3;
}

// ds_read_b64_tr_b8 (gfx950 LDS transpose read).  Within each 16-lane group,
// lane i receives as byte k the byte (i % 8) of the 8-byte word whose address
// lane 2k + i / 8 supplies: if lane j points at row j / 2, bytes 8 (j % 2) ..
// +7 of an 8-row x 16-byte block, lane i gets column i of the block, the
// eight rows' bytes in order.
__device__ __forceinline__ i2 lds_read_tr8(const int8_t* p) {
    typedef __attribute__((address_space(3))) i2 lds_i2;
    const auto* lp = reinterpret_cast<const __attribute__((address_space(3))) char*>(
        (uint32_t)reinterpret_cast<uintptr_t>(p));
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i2*)lp);
}

__device__ __forceinline__ i32x4_t uniform_rsrc(i32x4_t r) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
        r[e] = __builtin_amdgcn_readfirstlane(r[e]);
    }
    return r;
}

// KSV: per-token K scales (p.ksv) staged per tile; otherwise p.k_scale is
// folded into the per-row factor.
template <int D, bool KSV, bool SCORES>
__global__ __launch_bounds__(kI8Threads, 1) void fa_fwd_int8(Int8Params p) {
    using C = I8Cfg<D>;
    // [slot][K, V][TILE]; DMA destinations, so the base is 1 KB aligned
    __shared__ __attribute__((aligned(1024))) int8_t sKV[kI8Slots * 2 * C::TILE];
    __shared__ __attribute__((aligned(1024))) int8_t sQ[kI8Waves * 32 * D]; // [wave][32 rows][D], swizzled
    __shared__ __attribute__((aligned(16))) float sks[kI8Slots * kI8BN];
    __shared__ __attribute__((aligned(16))) _Float16 sO[kI8Waves * 32 * C::LDO];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const int grp = wave >> 2;
    const uint32_t kv_lds = (uint32_t)reinterpret_cast<uintptr_t>(sKV);
    const uint32_t ks_lds = (uint32_t)reinterpret_cast<uintptr_t>(sks);

    // LDS operand offsets within a tile, fixed per lane:
    //   K (and Q) operand of reduction step st (+ 32 D for keys 32..63): row
    //   l32, chunk 2 st + g;
    //   V^T operand of O^T row tile dt: lane j of a 16-lane group reads the 8 bytes
    //   8 (j & 1) .. +7 of chunk 2 dt + (lane >> 4 & 1) in key row kb(j) (+ 16 D for
    //   the second read, + 32 D for keys 32..63), kb = 8 (j/2 / 4) + 4 g + (j/2 % 4).
    int kofs[C::NS], vofs[C::NDT];
    {
        const int sw = i8_swz(l32);
#pragma unroll
        for (int st = 0; st < C::NS; st++) {
            kofs[st] = l32 * D + 16 * ((2 * st + g) ^ sw);
        }
        const int k8 = (lane & 15) >> 1;
        const int kb = 8 * (k8 >> 2) + 4 * g + (k8 & 3);
        const int swv = i8_swz(kb);
#pragma unroll
        for (int dt = 0; dt < C::NDT; dt++) {
            vofs[dt] = kb * D + 16 * ((2 * dt + ((lane >> 4) & 1)) ^ swv) + 8 * (lane & 1);
        }
    }
    // DMA source offsets of this lane in the BPW blocks a group-A wave issues per
    // tile: physical chunk P = 64 (wave BPW + jj) + lane holds row P / CH, logical
    // chunk (P % CH) ^ swz(row)
    uint32_t dk[C::BPW], dv[C::BPW];
#pragma unroll
    for (int jj = 0; jj < C::BPW; jj++) {
        const int P = 64 * ((wave & 3) * C::BPW + jj) + lane;
        const int r = P / C::CH;
        const int c = (P % C::CH) ^ i8_swz(r);
        dk[jj] = (uint32_t)((int64_t)r * p.k_ss + 16 * c);
        dv[jj] = (uint32_t)((int64_t)r * p.v_ss + 16 * c);
    }
    constexpr int DPT = 2 * C::BPW; // K/V DMAs per group-A wave per tile (wave 0 adds one for the K scales)

    auto run_tile = [&](const int wg) {
        int hg, rt;
        wg_tile(wg, p.n_head_groups, p.n_row_tiles, p.hg_chunk, hg, rt);
        const int per_b = p.Hkv * p.groups_per_kv;
        const int b = hg / per_b;
        const int rem = hg - b * per_b;
        const int kvh = rem / p.groups_per_kv;
        const int sub = rem - kvh * p.groups_per_kv;
        const int h = kvh * p.ratio + sub * p.G + (wave % p.G);
        const int wg_q0 = rt * p.rows_per_wg;
        const int q0 = wg_q0 + (wave / p.G) * 32;
        const int q = q0 + l32;
        const bool wave_active = q0 < p.Sq;
        const int q_hi = min(q0 + 31, p.Sq - 1);
        const int Sk = p.mask.sk;

        const int8_t* qbase = p.q + b * p.q_sb + h * p.q_sh;
        const int8_t* kbase = p.k + b * p.k_sb + kvh * p.k_sh;
        const int8_t* vbase = p.v + b * p.v_sb + kvh * p.v_sh;
        _Float16* obase = p.o + b * p.o_sb + h * p.o_sh;
        const float* ksbase = KSV ? p.ksv + ((int64_t)b * p.Hkv + kvh) * Sk : nullptr;

        float qs = p.q_scale;
        if (p.qsv != nullptr && q < p.Sq) {
            qs = p.qsv[((int64_t)b * p.Hq + h) * p.Sq + q];
        }
        // s_j = t_j * qc with t_j = S_j * ks_j (S_j alone when the K scale is a
        // single number, folded into qc).  When every lane's qc is positive the
        // row max is taken over t; otherwise t is first scaled by qc in place
        // and qeff = 1.
        const float qc = KSV ? qs * p.scale_log2e : qs * p.k_scale * p.scale_log2e;
        const bool qpos = !wave_any(!(qc > 0.0f));
        const float qeff = qpos ? qc : 1.0f;

        const int wg_q_hi = min(wg_q0 + p.rows_per_wg, p.Sq) - 1;
        int klo, khi;
        visible_key_range(p.mask, wg_q0, wg_q_hi, klo, khi);
        int t_begin = 0, n = 0;
        if (khi >= klo) {
            t_begin = klo / kI8BN;
            n = khi / kI8BN + 1 - t_begin;
        }
        int row_lo, row_hi;
        row_key_bounds(p.mask, q, row_lo, row_hi);

        // Q rows q0 .. q0 + 31 go by DMA into this wave's Q area, laid out like
        // a K tile's first 32 rows; the Q^T operand of reduction step st is then
        // a K-operand-shaped read: lane holds Q[q][32 st + 16 g .. +15]
        const int8_t* const sQu = sQ + wave * (32 * D);
        if (n > 0) {
            const i32x4_t rq = uniform_rsrc(make_rsrc_v(qbase + (int64_t)q0 * p.q_ss,
                                                        tile_bytes<32>(p.Sq - q0, (uint32_t)p.q_ss, D)));
            const uint32_t mq = (uint32_t)__builtin_amdgcn_readfirstlane((int)reinterpret_cast<uintptr_t>(sQu));
#pragma unroll
            for (int j = 0; j < C::QB; j++) {
                const int P = 64 * j + lane;
                const int r = P / C::CH;
                const int c = (P % C::CH) ^ i8_swz(r);
                dma_load16(rq, (uint32_t)((int64_t)r * p.q_ss + 16 * c),
                           (uint32_t)__builtin_amdgcn_readfirstlane((int)(mq + 1024 * j)));
            }
        }

        // O = of * 2^(m_a - m_c) + oint (see the header); l relative to m_c
        i16x oint[C::NDT];
        f16x of[C::NDT];
#pragma unroll
        for (int dt = 0; dt < C::NDT; dt++) {
            oint[dt] = i16x{};
            of[dt] = f16x{};
        }
        float m_c = -INFINITY, m_a = -INFINITY, l_c = 0.0f, beta = 0.0f;
        bool live = false, fold = false; // wave-uniform
        int run_tiles = 0;               // P V tiles summed in oint since its chain last restarted
        // S^T accumulators of the current tile (keys 0..31 and 32..63), turned
        // into t = S * ks in place (as fp32 bit patterns) before the softmax
        i16x sacc[2];
        sacc[0] = i16x{};
        sacc[1] = i16x{};
        i4 pb[2]; // P^T operands of keys 0..31 and 32..63: bytes 0..127
        pb[0] = i4{};
        pb[1] = i4{};
        int cls_prev = 0;

        // ---- DMA of tile x (K, V and the per-token K scales) into slot x % 4,
        // issued by group A's waves
        auto issue = [&](int x) {
            const int key0 = (t_begin + x) * kI8BN;
            const uint32_t slot = (uint32_t)(x & (kI8Slots - 1));
            const i32x4_t rk = uniform_rsrc(make_rsrc_v(kbase + (int64_t)key0 * p.k_ss,
                                                        tile_bytes<kI8BN>(Sk - key0, (uint32_t)p.k_ss, D)));
            const i32x4_t rv = uniform_rsrc(make_rsrc_v(vbase + (int64_t)key0 * p.v_ss,
                                                        tile_bytes<kI8BN>(Sk - key0, (uint32_t)p.v_ss, D)));
            const uint32_t mk = (uint32_t)__builtin_amdgcn_readfirstlane(
                (int)(kv_lds + slot * (2 * C::TILE) + (uint32_t)((wave & 3) * C::BPW * 1024)));
#pragma unroll
            for (int jj = 0; jj < C::BPW; jj++) {
                dma_load16(rk, dk[jj], mk + 1024 * jj);
            }
#pragma unroll
            for (int jj = 0; jj < C::BPW; jj++) {
                dma_load16(rv, dv[jj], mk + C::TILE + 1024 * jj);
            }
            if (KSV && wave == 0) {
                // the tile's 64 K scales, one dword per lane (keys past Sk read 0)
                const int left = Sk - key0;
                const i32x4_t rs =
                    uniform_rsrc(make_rsrc_v(ksbase + key0, (uint32_t)(4 * (left < kI8BN ? left : kI8BN))));
                dma_load4(rs, (uint32_t)(4 * lane), ks_lds + slot * (kI8BN * 4));
            }
        };
        // group A: wait until at most one tile's DMAs (the one issued last) are
        // in flight, or none
        auto wait_dmas = [&](bool keep_one) {
            if (!keep_one) {
                __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
            } else if (KSV && wave == 0) {
                __builtin_amdgcn_s_waitcnt(waitcnt_vm(DPT + 1));
            } else {
                __builtin_amdgcn_s_waitcnt(waitcnt_vm(DPT));
            }
        };

        // fold of 8 accumulators (flat index 8 u .. 8 u + 7 over [dt][e]) into
        // O_f (the next P V MFMA of their column tile restarts the chain)
        auto fold_slice = [&](int u) {
#pragma unroll
            for (int f = 8 * u; f < 8 * u + 8; f++) {
                of[f >> 4][f & 15] = fmaf(of[f >> 4][f & 15], beta, (float)oint[f >> 4][f & 15]);
            }
        };
        // dequantisation of 4 scores in place (group u: keys 32 (u / 4) + 8 (u %
        // 4) + 4 g .. +3)
        auto dequant_group = [&](int u, const float* ksl) {
            const int kt = u >> 2, r4 = u & 3;
            if constexpr (KSV) {
                const f4 ks = *reinterpret_cast<const f4*>(&ksl[32 * kt + 8 * r4 + 4 * g]);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    sacc[kt][4 * r4 + e] = __float_as_int((float)sacc[kt][4 * r4 + e] * ks[e]);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    sacc[kt][4 * r4 + e] = __float_as_int((float)sacc[kt][4 * r4 + e]);
                }
            }
        };

        // M(i): S(i)^T = K(i) Q^T (i < n), then O^T += V(i-1)^T P(i-1)^T (i >= 1):
        // one stream of MFMAs whose LDS operands are read kI8OpDepth MFMAs
        // ahead.  The fold (when the previous softmax moved a row max) rides on
        // the Q K^T MFMAs and the first P V MFMA of each column tile then
        // restarts its int32 chain; the dequantisation of S(i) rides on the P V
        // MFMAs.
        auto mfma_stream = [&](auto do_pv_c, auto do_s_c, auto fold_c, int i) {
            // The MFMA phase runs at raised wave priority: each SIMD also holds
            // the other group's wave in its softmax phase, whose VALU stream
            // otherwise delays the issue of the next MFMA (-2.7 % at head_dim 64 in
            // same-box A/B runs; the INT8 head_dim 128 kernel, whose softmax
            // side is its critical path, measured slower with it)
            __builtin_amdgcn_s_setprio(1);
            constexpr bool DO_PV = decltype(do_pv_c)::value;
            constexpr bool DO_S = decltype(do_s_c)::value;
            constexpr bool FOLD = decltype(fold_c)::value;
            constexpr int NSK = DO_S ? 2 * C::NS : 0;   // (st, kt)
            constexpr int NPV = DO_PV ? 2 * C::NDT : 0; // (kt, dt)
            constexpr int T = NSK + NPV;
            constexpr int DEPTH = T < kI8OpDepth ? T : kI8OpDepth;
            constexpr int GPS = NPV > 0 ? 8 / NPV : 0; // dequant groups per P V MFMA
            const int8_t* sk = sKV + (i & (kI8Slots - 1)) * (2 * C::TILE);
            const int8_t* sv = sKV + ((i - 1) & (kI8Slots - 1)) * (2 * C::TILE) + C::TILE;
            const float* ksl = sks + (i & (kI8Slots - 1)) * kI8BN;
            auto q_op = [&](int st) -> i4 { return *reinterpret_cast<const i4*>(sQu + kofs[st]); };
            auto op = [&](int j) -> i4 {
                if (j < NSK) {
                    const int st = j >> 1, kt = j & 1;
                    return *reinterpret_cast<const i4*>(sk + kofs[st] + kt * 32 * D);
                }
                const int jp = j - NSK, kt = jp / C::NDT, dt = jp % C::NDT;
                const int8_t* a = sv + vofs[dt] + kt * 32 * D;
                const i2 lo = lds_read_tr8(a);
                const i2 hi = lds_read_tr8(a + 16 * D);
                return i4{lo[0], lo[1], hi[0], hi[1]};
            };
            if constexpr (FOLD && !DO_S) {
#pragma unroll
                for (int u = 0; u < 2 * C::NDT; u++) {
                    fold_slice(u);
                }
            }
            if constexpr (DO_S) {
                sacc[0] = i16x{};
                sacc[1] = i16x{};
            }
            i4 ring[DEPTH > 0 ? DEPTH : 1];
#pragma unroll
            for (int j = 0; j < DEPTH; j++) {
                ring[j] = op(j);
            }
            // Q^T operands: step st's read one step ahead of its first use
            i4 qcur = DO_S ? q_op(0) : i4{}, qnext = i4{};
#pragma unroll
            for (int j = 0; j < T; j++) {
                const i4 a = ring[j % DEPTH];
                if (j + DEPTH < T) {
                    ring[j % DEPTH] = op(j + DEPTH);
                }
                if (j < NSK) {
                    const int st = j >> 1, kt = j & 1;
                    if (kt == 0 && st + 1 < C::NS) {
                        qnext = q_op(st + 1);
                    }
                    sacc[kt] = mfma_32x32x32_i8(a, qcur, sacc[kt]);
                    if (kt == 1) {
                        qcur = qnext;
                    }
                    if constexpr (FOLD) {
                        fold_slice(j); // 2 NS slots x 8 = 16 NDT accumulators
                    }
                } else {
                    const int jp = j - NSK, kt = jp / C::NDT, dt = jp % C::NDT;
                    if (FOLD && kt == 0) {
                        oint[dt] = mfma_32x32x32_i8(a, pb[0], i16x{});
                    } else {
                        oint[dt] = mfma_32x32x32_i8(a, pb[kt], oint[dt]);
                    }
                    if constexpr (DO_S && !SCORES) {
#pragma unroll
                        for (int u = GPS * jp; u < GPS * jp + GPS; u++) {
                            dequant_group(u, ksl);
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_s_setprio(0);
            if constexpr (DO_S && SCORES) {
                // the two S^T blocks of this tile: lane holds query q, keys
                // kt0 + 32 kt + 8 (e / 4) + 4 g + e % 4
                if (q < p.Sq) {
                    const int kt0 = (t_begin + i) * kI8BN;
                    int32_t* srow = p.scores + (((int64_t)b * p.Hq + h) * p.Sq + q) * Sk;
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int k0 = kt0 + 8 * (e >> 2) + 4 * g + (e & 3);
                        if (k0 < Sk) {
                            srow[k0] = sacc[0][e];
                        }
                        if (k0 + 32 < Sk) {
                            srow[k0 + 32] = sacc[1][e];
                        }
                    }
                }
            } else if constexpr (DO_S && !DO_PV) {
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    dequant_group(u, ksl);
                }
            }
        };
        auto phase_m = [&](int i) {
            if (!wave_active) {
                return;
            }
            const bool do_pv = !SCORES && i >= 1 && cls_prev != 0;
            int cls_now = 0;
            if (i < n) {
                const int kt0 = (t_begin + i) * kI8BN;
                cls_now = classify_tile(p.mask, q0, q_hi, kt0, kt0 + kI8BN - 1);
            }
            using T_ = std::true_type;
            using F_ = std::false_type;
            if (do_pv && cls_now != 0) {
                if (fold) {
                    mfma_stream(T_{}, T_{}, T_{}, i);
                } else {
                    mfma_stream(T_{}, T_{}, F_{}, i);
                }
            } else if (do_pv) {
                if (fold) {
                    mfma_stream(T_{}, F_{}, T_{}, i);
                } else {
                    mfma_stream(T_{}, F_{}, F_{}, i);
                }
            } else if (cls_now != 0) {
                mfma_stream(F_{}, T_{}, F_{}, i);
            }
            if (do_pv) {
                run_tiles = fold ? 1 : run_tiles + 1;
                live = true;
                fold = false;
            }
            cls_prev = cls_now;
        };

        // V(i): the scheme's exact running max over the 64-key block and P as
        // bytes 0..127; a moved maximum rescales l now and schedules the fold
        // of O_int for the next MFMA phase
        auto phase_v = [&](int i) {
            if (SCORES || !wave_active || cls_prev == 0) {
                return;
            }
            if (!qpos) {
#pragma unroll
                for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        sacc[kt][e] = __float_as_int(__int_as_float(sacc[kt][e]) * qc);
                    }
                }
            }
            if (cls_prev == 2) {
                const int kt0 = (t_begin + i) * kI8BN + 4 * g;
                const int a = row_lo - kt0;
                const int bnd = row_hi - kt0;
#pragma unroll
                for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int off = 32 * kt + 8 * (e >> 2) + (e & 3);
                        sacc[kt][e] = (off < a || off > bnd) ? __float_as_int(-INFINITY) : sacc[kt][e];
                    }
                }
            }
            float mx = __int_as_float(sacc[0][0]);
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    mx = fmaxf(mx, __int_as_float(sacc[kt][e]));
                }
            }
            mx = pair_max(mx) * qeff; // qeff > 0: -inf stays -inf
            const float m_new = fmaxf(m_c, mx);
            // a moved maximum folds O_int; so does a chain of kI8FoldTiles P V
            // tiles (rows whose maximum settled early, on long key ranges),
            // before the int32 sums could overflow
            if (wave_any(m_new > m_c) || (live && run_tiles >= kI8FoldTiles)) {
                // l *= 2^(m_c - m_new): 1 where the row max stayed, 0 for a first visible key
                l_c *= (m_c == -INFINITY) ? 0.0f : fast_exp2(m_c - m_new);
                if (live) {
                    beta = (m_c == -INFINITY) ? 0.0f : fast_exp2(m_a - m_c); // m_a = -inf -> 0
                    m_a = m_c;
                    fold = true;
                }
                m_c = m_new;
            }
            const float c0 = int8_exp_offset(m_c); // y <= 127: a packed 128 would read as -128
            float psum = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    uint32_t word = 0;
#pragma unroll
                    for (int e = 4 * w; e < 4 * w + 4; e++) {
                        const float y = fast_exp2(fmaf(__int_as_float(sacc[kt][e]), qeff, c0)); // 127 p, <= 127
                        psum += y;
                        word = __builtin_amdgcn_cvt_pk_u8_f32(y, (uint32_t)(e & 3), word);
                    }
                    pb[kt][w] = (int)word;
                }
            }
            l_c += psum;
        };

        if (grp == 0 && n > 0) {
            issue(0);
            if (n > 1) {
                issue(1);
            }
            wait_dmas(n > 1); // Q and tile 0 landed
        } else if (n > 0) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); // Q landed
        }
        __syncthreads();
        // Group A: M(i) in phase 2i, V(i) in phase 2i + 1; group B one phase
        // later.  Tile x is read in phases 2x .. 2x + 3 (K in M(x), V in M(x + 1),
        // by A then B).  Its DMAs are issued at the start of phase 2x - 4 into
        // the slot tile x - 4 left at the end of phase 2x - 5, and group A waits
        // for them at the end of phase 2x - 1.  Both groups pass 2n + 3 barriers.
        if (n > 0) {
            if (grp == 0) {
                for (int i = 0; i < n; i++) {
                    if (i + 2 < n) {
                        issue(i + 2);
                    }
                    phase_m(i);
                    __syncthreads();
                    phase_v(i);
                    wait_dmas(i + 2 < n); // tile i + 1 landed
                    __syncthreads();
                }
                phase_m(n);
                __syncthreads();
                __syncthreads();
            } else {
                __syncthreads();
                for (int i = 0; i < n; i++) {
                    phase_m(i);
                    __syncthreads();
                    phase_v(i);
                    __syncthreads();
                }
                phase_m(n);
                __syncthreads();
            }
        }

        if (SCORES || !wave_active) {
            return;
        }
        // O = (of * 2^(m_a - m_c) + oint) * v_scale / l (times the per-channel V
        // scales of this kv head when given), through this wave's sO slot
        const float bf = (m_c == -INFINITY) ? 0.0f : fast_exp2(m_a - m_c);
#pragma unroll
        for (int dt = 0; dt < C::NDT; dt++) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                of[dt][e] = fmaf(of[dt][e], bf, (float)oint[dt][e]);
            }
        }
        const float l = pair_sum(l_c);
        const float f = l > 0.0f ? p.v_scale / l : 0.0f;
        const float* vch = p.vch != nullptr ? p.vch + ((int64_t)b * p.Hkv + kvh) * D : nullptr;
        store_o_tile<D, C::LDO>(
            of,
            [&](int d0) {
                return vch != nullptr ? f * *reinterpret_cast<const f4*>(vch + d0) : f4{f, f, f, f};
            },
            sO + wave * 32 * C::LDO, obase, q0, p.Sq, p.o_ss, lane);
    };
    for (int item = 0;; item++) {
        const int wg = persistent_item(blockIdx.x, gridDim.x, item, p.n_items);
        if (wg < 0) {
            break;
        }
        run_tile(wg);
    }
}

template <int D, bool KSV, bool SCORES>
int launch_int8(const Int8Params& p, int64_t n_wg, hipStream_t stream, std::string& err) {
    // persistent: as many workgroups as the device holds at once, each
    // walking its share of the n_wg row tiles
    const int64_t resident =
        resident_workgroups(reinterpret_cast<const void*>(&fa_fwd_int8<D, KSV, SCORES>), kI8Threads, err);
    if (resident <= 0) {
        return -1;
    }
    const int64_t grid = std::min(n_wg, resident);
    KernelTimerGuard timer(stream);
    hipLaunchKernelGGL((fa_fwd_int8<D, KSV, SCORES>), dim3((uint32_t)grid), dim3(kI8Threads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

} // namespace

int64_t int8_params(const AttnArgs& a, Int8Params& p, std::string& err) {
    if (a.ks[2] < 0 || a.vs[2] < 0 || a.ks[2] > (1 << 24) || a.vs[2] > (1 << 24)) {
        err = "key/value seq strides must be in [0, 2^24] elements";
        return -1;
    }
    p = Int8Params{};
    p.q = static_cast<const int8_t*>(a.q);
    p.k = static_cast<const int8_t*>(a.k);
    p.v = static_cast<const int8_t*>(a.v);
    p.o = static_cast<_Float16*>(a.o);
    p.qsv = a.q_scale_vec;
    p.ksv = a.k_scale_vec;
    p.vch = a.v_channel;
    p.vtok = a.v_token;
    p.q_scale = a.q_scale;
    p.k_scale = a.k_scale;
    p.v_scale = a.v_scale;
    p.scale_log2e = a.scale * 1.442695041f; // the reference's kLog2E (fa2_forward_int8qk.hip:60)
    p.q_sb = a.qs[0];
    p.q_sh = a.qs[1];
    p.q_ss = a.qs[2];
    p.k_sb = a.ks[0];
    p.k_sh = a.ks[1];
    p.k_ss = a.ks[2];
    p.v_sb = a.vs[0];
    p.v_sh = a.vs[1];
    p.v_ss = a.vs[2];
    p.o_sb = a.os[0];
    p.o_sh = a.os[1];
    p.o_ss = a.os[2];
    p.Hq = a.Hq;
    p.Sq = a.Sq;
    p.Hkv = a.Hkv;
    p.ratio = a.Hq / a.Hkv;
    p.G = (p.ratio % 4 == 0) ? 4 : ((p.ratio % 2 == 0) ? 2 : 1);
    p.rows_per_wg = 32 * kI8Waves / p.G;
    p.n_row_tiles = (a.Sq + p.rows_per_wg - 1) / p.rows_per_wg;
    p.groups_per_kv = p.ratio / p.G;
    p.n_head_groups = a.B * a.Hkv * p.groups_per_kv;
    p.hg_chunk = xcd_head_group_chunk(p.n_head_groups, 2 * (int64_t)a.Sk * a.D);
    p.mask = MaskSpec{a.Sk, a.Sk - a.Sq, a.causal ? 1 : 0, a.window > 0 ? a.window : 0};
    const int64_t n_wg = (int64_t)p.n_row_tiles * p.n_head_groups;
    if (n_wg <= 0 || n_wg > INT32_MAX) {
        err = "launch grid out of range";
        return -1;
    }
    p.n_items = (int32_t)n_wg;
    return n_wg;
}

int fwd_int8(const AttnArgs& a, hipStream_t stream, std::string& err) {
    Int8Params p;
    const int64_t n_wg = int8_params(a, p, err);
    if (n_wg < 0) {
        return -1;
    }
    if (a.D == 64 && p.vtok == nullptr) {
        return p.ksv != nullptr ? launch_int8<64, true, false>(p, n_wg, stream, err)
                                : launch_int8<64, false, false>(p, n_wg, stream, err);
    }
    if (a.D == 64 || a.D == 128) {
        return launch_int8_f16pv(p, a.D, false, n_wg, stream, err);
    }
    err = "unsupported head_dim (only 64 and 128 are compiled in for the int8 kernel)";
    return -1;
}

int int8_scores(const AttnArgs& in, int32_t* scores, hipStream_t stream, std::string& err) {
    // the production kernel's SCORES instantiation for this head dim: its K
    // tiles, LDS layout, operand ring and MFMAs, with V staged from K and no
    // output
    AttnArgs a = in;
    a.v = a.k;
    a.vs[0] = a.ks[0], a.vs[1] = a.ks[1], a.vs[2] = a.ks[2];
    a.o = nullptr;
    a.causal = 0;
    a.window = 0;
    a.k_scale_vec = nullptr;
    a.v_token = nullptr;
    Int8Params p;
    const int64_t n_wg = int8_params(a, p, err);
    if (n_wg < 0) {
        return -1;
    }
    p.scores = scores;
    switch (a.D) {
    case 64: return launch_int8<64, false, true>(p, n_wg, stream, err);
    case 128: return launch_int8_f16pv(p, 128, true, n_wg, stream, err);
    default: break;
    }
    err = "unsupported head_dim (only 64 and 128 are compiled in for the int8 kernel)";
    return -1;
}

#else // RDNATTENTION_NO_INT8: the reference's RDNATTENTION_ENABLE_INT8=OFF build (CMakeLists.txt:33)

int fwd_int8(const AttnArgs&, hipStream_t, std::string& err) {
    err = "this library was built without the INT8 kernel";
    return -1;
}

int int8_scores(const AttnArgs&, int32_t*, hipStream_t, std::string& err) {
    err = "this library was built without the INT8 kernel";
    return -1;
}

#endif

} // namespace rdna_amd
