// INT8 FlashAttention forward for gfx950 with P V on fp16 MFMA: the kernel for
// head_dim 128 and for the per-token V scale extension (fa_fwd_int8.hip runs
// head_dim 64 with both GEMMs on int8 MFMA).
//
// Q K^T and the softmax follow the reference's scheme (forwardKernelInt8QK,
// src/rdna/fa2_forward_int8qk.hip:229-495):
//
//   S_ij  = sum_d q_i8 k_i8                          (exact int32)
//   s_ij  = S_ij * qs_i * ks_j * scale * log2(e)      (fp32, log2 domain)
//   per 64-key block, aligned to key 0 (the reference's Bc = 64):
//     m'  = max(m, max_j s_ij);  O *= 2^(m - m'),  l *= 2^(m - m')
//     p   = 2^(s - m'),  l += sum p                  (unquantised p)
//     pq  = min(127, round(p * 127))                 (P as integers 0..127)
//     O  += sum_j pq_j v_j
//   out = O * v_scale / (127 l)  (0 when no key is visible)
//
// Why P V runs on fp16 MFMA here: pq (0..127) and v (-127..127) are exact fp16
// integers and their products exact in fp32, and with O and l kept relative
// to a lagging reference m_ref <= m (raised only when m exceeds it by more
// than 2^8) each block's P enters the product as pq * fp16(2^(m - m_ref)), so
// O needs one fp32 accumulator per element and no per-block fold.  Summing
// the blocks in int32 on int8 MFMA instead needs an int32 and an fp32
// accumulator per element and a fold whenever a row maximum moves; at
// head_dim 128 that is 128 registers per 32-row tile, which forces wave pairs
// per tile (128 query rows per workgroup) and measured 1.6x slower than this
// kernel on the causal GQA S = 8192 shape.  At head_dim 64 it is 9 % faster,
// so fa_fwd_int8.hip serves that head dim.
//
// The running max m is exact per block, as the scheme requires (pq depends
// on it).  The P V products pq * fp16(f) are rounded once to fp16 (relative
// 2^-11, values <= 127 * 256) and the row sum uses sum p * the same factor, so
// O / l is the scheme's ratio.
//
// Deliberate differences, all far below the INT8 tolerance: round() is
// round-half-to-even (v_rndne_f32) where the reference calls lroundf (half
// away from zero), 127 p is evaluated as 2^(s - m' + log2 127), the per-block
// v_scale/127 factor is applied once at the end, and P is scaled by the
// reference factor above.
//
// Kernel structure is the FP16 ping-pong design (fa_fwd_f16.hip): 8 waves in
// two groups alternating MFMA and VALU phases, S^T = K Q^T so a lane owns one
// query column, and P^T going from the S accumulator straight into the B
// operand of O^T = V^T P^T.  An MFMA phase issues the Q K^T MFMAs first and
// the P V MFMAs after them, with the dequantisation of the scores riding on
// the P V MFMAs.  Per score the softmax side costs one dequantisation fma
// (the Q K^T chains start at the bit pattern of 1.5 2^23, so the int32 sum
// read as fp32 is 1.5 2^23 + S), half a max3, the exponent fma, the
// exponent, the row-sum add, one v_fma_mix (fp16(1 + 127 p 2^-10) rounds
// 127 p to an integer) and half a packed fma (times the reference factor).  V is converted to fp16 while it is staged into
// LDS (a byte permute against the fp16 exponent of 1024, then one packed
// subtract; with a per-token V scale, fp16(sat(v * vs)) per row) and its V^T
// operands come from ds_read_b64_tr_b16 transpose reads.  The grid is
// persistent (persistent_item), and O leaves through an LDS buffer as
// whole-row non-temporal stores (store_o_tile).
//
// VTOK (an extension; the reference lists a per-token V scale as missing
// because the scale sits inside the P V sum, FEATURES.md:191, :201-202): V
// row j is dequantised by its own scale vs_j while it is staged,
// v'_j = fp16(sat(v_j * vs_j)), and P V runs on these fp16 values.
//
// SCORES (a test instantiation): the same kernel with the softmax, P V and
// output compiled out; every S^T accumulator block its first GEMM produces is
// written to an int32 score buffer, so the tests can check the production
// GEMM's scores bit for bit.
#include "fa_common.hpp"
#include "fa_host.hpp"
#include "fa_internal.hpp"
#include "fa_int8.hpp"
#include "fa_prefill.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace rdna_amd {

#if !defined(RDNATTENTION_NO_INT8)

namespace {

typedef int8_t i8x8 __attribute__((ext_vector_type(8)));
typedef int i2 __attribute__((ext_vector_type(2)));

template <int D>
struct I8Cfg {
    // K: int8 rows of D bytes at a D+16 byte stride (16 rows read with
    // ds_read_b128 land in distinct banks); V: converted to fp16 while staged,
    // rows at D+32 halves (conflict-free 4-row transpose reads)
    static constexpr int LDK = D + 16;         // bytes
    static constexpr int LDV = D + 32;         // halves
    static constexpr int TILE_K = kI8BN * LDK; // bytes
    static constexpr int TILE_V = kI8BN * LDV; // halves
    static constexpr int NS = D / 32;          // int8 QK^T reduction steps (32 per MFMA)
    static constexpr int NDT = D / 32;         // O^T row tiles
    static constexpr int KCH = D / 16;         // 16-byte int8 chunks per row
    static constexpr int HALF_TASK = 32 * KCH; // one group's chunks of one K (or V) tile
    static constexpr int CT = (HALF_TASK + 255) / 256;
    static constexpr int LDO = D + 8; // halves; output staging rows (conflict-free like K rows)
};

constexpr int kI8OpDepth = 6;                // MFMA operands in flight in the MFMA phase (4: +1 %)
constexpr float kI8RefThreshold = 8.0f;      // log2 units: P is scaled by at most 2^8 (127 * 256 < 65504)
// Start of the Q K^T chains: the int32 bit pattern of this float (1.5 2^23),
// so the accumulator read as fp32 is kI8Bias + S, exact for |S| < 2^22
constexpr float kI8Bias = 12582912.0f;
// P enters P V as pq f 2^-10 (the quantisation's fp16 step, see phase_v);
// the output factor multiplies the 2^10 back
constexpr float kI8PScale = 0x1p-10f;

__device__ __forceinline__ i4 buffer_load_i4(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    u4 x = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
    return __builtin_bit_cast(i4, x);
}

// 16 signed bytes -> two h8 (exact: every int8 is an fp16 integer).  Flipping
// the sign bit gives u = v + 128 as an unsigned byte; a byte permute pairs each
// u with the high byte 0x64, i.e. the fp16 value 1024 + u (exact: the ulp in
// [1024, 2048) is 1), and one packed subtract of 1152 leaves v.  Five VALU
// instructions per 4 values.
__device__ __forceinline__ void i8x16_to_h8x2(i4 w, h8& lo, h8& hi) {
    const h2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
    h2 r[8];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t u = (uint32_t)w[c] ^ 0x80808080u;
        // byte selects: 0-3 pick bytes of u, 4 picks byte 0 of 0x64646464
        const uint32_t p01 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
        const uint32_t p23 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
        r[2 * c] = __builtin_bit_cast(h2, p01) - off;
        r[2 * c + 1] = __builtin_bit_cast(h2, p23) - off;
    }
    lo = {r[0][0], r[0][1], r[1][0], r[1][1], r[2][0], r[2][1], r[3][0], r[3][1]};
    hi = {r[4][0], r[4][1], r[5][0], r[5][1], r[6][0], r[6][1], r[7][0], r[7][1]};
}

// 16 signed bytes of one V row -> two h8 of fp16(sat(v * vs)): the product in
// fp32 (v exact, vs as given), saturated to the fp16 range so that no V value
// becomes infinite (a zero P times an infinite V would be NaN for every row
// sharing the tile), then rounded once to fp16
__device__ __forceinline__ void i8x16_to_h8x2_scaled(i4 w, float vs, h8& lo, h8& hi) {
    const i8x8 a = __builtin_bit_cast(i8x8, i2{w[0], w[1]});
    const i8x8 b = __builtin_bit_cast(i8x8, i2{w[2], w[3]});
#pragma unroll
    for (int e = 0; e < 8; e++) {
        lo[e] = (_Float16)__builtin_amdgcn_fmed3f((float)a[e] * vs, -65504.0f, 65504.0f);
        hi[e] = (_Float16)__builtin_amdgcn_fmed3f((float)b[e] * vs, -65504.0f, 65504.0f);
    }
}

// Scheme (the reference's, fa2_forward_int8qk.hip:281-382), per 64-key block b
// aligned to key 0, with s_j = S_j * qs * ks_j * scale * log2(e):
//   m_b  = max(m_{b-1}, max_j s_j)     (exact: pq below depends on it)
//   y_j  = 127 * 2^(s_j - m_b)         (computed as 2^(s_j - m_b + log2 127))
//   pq_j = round(y_j) in [0, 127]
//   f_b  = fp16(2^(m_b - m_ref))       (m_ref <= m_b: raised, with O and l
//                                       rescaled, only when m_b - m_ref > 8)
//   l   += f_b * sum_j y_j              (unquantised p, in units of 1/127)
//   O   += sum_j fp16(pq_j * f_b) v_j
//   out  = O * v_scale / l
// S runs on int8 MFMA (exact int32).  P V runs on fp16 MFMA and accumulates
// straight into fp32, so O needs no per-block int32 -> fp32 conversion.
//
// VTOK (an extension; the reference has no per-token V scale): V row j is
// dequantised by its own scale vs_j while it is staged,
// v'_j = fp16(sat(v_j * vs_j)), and P V runs on these fp16 values.
//
// SCORES: the S^T accumulators of every computed key tile are written to
// p.scores and nothing else is computed (test instantiation).
template <int D, bool VTOK, bool SCORES>
__global__ __launch_bounds__(kI8Threads, 1) void fa_fwd_int8_f16pv(Int8Params p) {
    using C = I8Cfg<D>;
    __shared__ __attribute__((aligned(16))) int8_t sKs[2 * C::TILE_K];
    __shared__ __attribute__((aligned(16))) _Float16 sVs[2 * C::TILE_V];
    __shared__ __attribute__((aligned(16))) float sks[2][kI8BN]; // K scale of each key of a tile
    __shared__ __attribute__((aligned(16))) float sbk[2][kI8BN]; // -kI8Bias * that scale
    __shared__ __attribute__((aligned(16))) _Float16 sO[kI8Waves * 32 * C::LDO];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const int grp = wave >> 2;
    const int gtid = tid & 255;

    // Persistent: this workgroup walks its share of the row tiles (one per
    // workgroup of a one-tile-per-workgroup grid, see persistent_item). Every
    // group passes the same barriers per tile and leaves a tile only after its
    // last LDS read of K/V, so the next tile's prologue may overwrite them;
    // each wave's sO slot is its own.
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
        const float* ksbase = p.ksv ? p.ksv + ((int64_t)b * p.Hkv + kvh) * Sk : nullptr;
        const float* vtbase = VTOK ? p.vtok + ((int64_t)b * p.Hkv + kvh) * Sk : nullptr;

        // Q^T operand: lane holds Q[q][32s + 16g .. +15]
        i4 qreg[C::NS];
        float qs = p.q_scale;
        {
            const bool valid = q < p.Sq;
            const int8_t* qrow = qbase + (int64_t)(valid ? q : 0) * p.q_ss;
#pragma unroll
            for (int s = 0; s < C::NS; s++) {
                qreg[s] = valid ? *reinterpret_cast<const i4*>(qrow + 32 * s + 16 * g) : i4{};
            }
            if (p.qsv != nullptr && valid) {
                qs = p.qsv[((int64_t)b * p.Hq + h) * p.Sq + q];
            }
        }
        // s_j = t_j * qc with t_j = S_j * ks_j.  When every lane's qc is positive
        // the row max is taken over t (one multiply per score saved); otherwise t
        // is first scaled by qc in place and qeff = 1.
        const float qc = qs * p.scale_log2e;
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
        // class of key tile t_begin + i for this wave's rows (0 skip, 1 no mask, 2 masked)
        const TileClasses tcls = wave_active ? tile_classes<kI8BN>(p.mask, q0, q_hi) : TileClasses{1, 0, 1, 0};

        f16x oacc[C::NDT];
#pragma unroll
        for (int dt = 0; dt < C::NDT; dt++) {
            oacc[dt] = f16x{};
        }
        // m_run: the scheme's exact running max; m_ref: the lagging reference
        // O and l are kept relative to (m_ref <= m_run)
        float m_run = -INFINITY, m_ref = -INFINITY, l_run = 0.0f;
        const i16x bias16 = SCORES ? i16x{} : (i16x{} + __float_as_int(kI8Bias));
        f16x tsc[2]; // scores of the current tile, dequantised by ks (t = S * ks)
        tsc[0] = f16x{};
        tsc[1] = f16x{};
        h8 pb[4]; // P^T operands of the four 16-key groups: integers 0..127 in fp16
#pragma unroll
        for (int u = 0; u < 4; u++) {
            pb[u] = h8{};
        }
        int cls_prev = 0;

        // ---- staging (one group's 32 rows of K and V per pair; ks by group A)
        i4 kreg[C::CT], vreg[C::CT];
        uint32_t coff_k[C::CT], coff_v[C::CT];
        int clk[C::CT], clv[C::CT];
#pragma unroll
        for (int it = 0; it < C::CT; it++) {
            const int e = gtid + it * 256;
            const bool ok = C::HALF_TASK % 256 == 0 || e < C::HALF_TASK;
            const int row = 32 * grp + (ok ? e / C::KCH : 0);
            const int ch = ok ? e - (e / C::KCH) * C::KCH : 0;
            coff_k[it] = (uint32_t)((int64_t)row * p.k_ss + 16 * ch);
            coff_v[it] = (uint32_t)((int64_t)row * p.v_ss + 16 * ch);
            clk[it] = ok ? row * C::LDK + 16 * ch : -1;
            clv[it] = ok ? row * C::LDV + 16 * ch : -1;
        }
        float ksreg = 0.0f;
        float vsreg[C::CT]; // VTOK: the scale of each staged V row
        auto load_pair = [&](int x) {
            const int tk = t_begin + x, tv = t_begin + x - 1;
            const auto rk = make_rsrc(kbase + (int64_t)tk * kI8BN * p.k_ss,
                                      x < n ? tile_bytes<kI8BN>(Sk - tk * kI8BN, (uint32_t)p.k_ss, D) : 0u);
            const auto rv = make_rsrc(vbase + (int64_t)tv * kI8BN * p.v_ss,
                                      (x >= 1 && x <= n) ? tile_bytes<kI8BN>(Sk - tv * kI8BN, (uint32_t)p.v_ss, D) : 0u);
#pragma unroll
            for (int it = 0; it < C::CT; it++) {
                kreg[it] = buffer_load_i4(rk, coff_k[it]);
                vreg[it] = buffer_load_i4(rv, coff_v[it]);
                if constexpr (VTOK) {
                    const int key = tv * kI8BN + 32 * grp + (gtid + it * 256) / C::KCH;
                    vsreg[it] = (x >= 1 && x <= n && key < Sk) ? vtbase[key] : 0.0f;
                }
            }
            if (grp == 0 && gtid < kI8BN && x < n) {
                const int key = tk * kI8BN + gtid;
                ksreg = (ksbase != nullptr && key < Sk) ? ksbase[key] : p.k_scale;
            }
        };
        auto store_pair = [&](int x) {
            int8_t* sK = sKs + (x & 1) * C::TILE_K;
            _Float16* sV = sVs + ((x - 1) & 1) * C::TILE_V;
#pragma unroll
            for (int it = 0; it < C::CT; it++) {
                if (C::HALF_TASK % 256 == 0 || clk[it] >= 0) {
                    if (x < n) {
                        *reinterpret_cast<i4*>(&sK[clk[it]]) = kreg[it];
                    }
                    if (x >= 1 && x <= n) {
                        h8 lo, hi;
                        if constexpr (VTOK) {
                            i8x16_to_h8x2_scaled(vreg[it], vsreg[it], lo, hi);
                        } else {
                            i8x16_to_h8x2(vreg[it], lo, hi);
                        }
                        *reinterpret_cast<h8*>(&sV[clv[it]]) = lo;
                        *reinterpret_cast<h8*>(&sV[clv[it] + 8]) = hi;
                    }
                }
            }
            if (grp == 0 && gtid < kI8BN && x < n) {
                // ks rounded to 22 significant bits (relative change <= 2^-23),
                // so that kI8Bias ks = 3 2^22 ks is exact in fp32 and the
                // dequantisation fma returns S ks rounded once
                const float ks22 = __uint_as_float((__float_as_uint(ksreg) + 2u) & ~3u);
                sks[x & 1][gtid] = ks22;
                sbk[x & 1][gtid] = -kI8Bias * ks22;
            }
        };

        // M(i): S(i)^T = K(i) Q^T (int8 MFMA, i < n) then O^T += V(i-1)^T P(i-1)^T
        // (fp16 MFMA, i >= 1): one stream of MFMAs whose LDS operands are read
        // kI8OpDepth MFMAs ahead through a register ring.  The dequantisation
        // of S(i) rides on the P V MFMAs: 8 groups of 4 scores, group u after
        // P V MFMA 2u + 1, its K scales and biases read at MFMA 2u (at head
        // dim 64, 8 P V MFMAs: group u after MFMA u).  (With the
        // P V MFMAs first it ran after the last Q K^T MFMA, on the phase's
        // critical path.)
        auto mfma_stream = [&](auto do_pv_c, auto do_s_c, int i) {
            constexpr bool DO_PV = decltype(do_pv_c)::value;
            constexpr bool DO_S = decltype(do_s_c)::value;
            constexpr bool DQ = DO_S && !SCORES;
            constexpr int NSK = DO_S ? 2 * C::NS : 0;   // (st, kt)
            constexpr int NPV = DO_PV ? 4 * C::NDT : 0; // (u, dt)
            static_assert(!DO_PV || NPV == 16 || NPV == 8, "8 dequantisation groups over the P V MFMAs");
            constexpr int T = NSK + NPV;
            constexpr int DEPTH = T < kI8OpDepth ? T : kI8OpDepth;
            const int j16 = lane & 15;
            const _Float16* vrow = sVs + ((i - 1) & 1) * C::TILE_V + (4 * g + (j16 >> 2)) * C::LDV +
                                   16 * ((lane >> 4) & 1) + 4 * (j16 & 3);
            const int8_t* krow = sKs + (i & 1) * C::TILE_K + l32 * C::LDK + 16 * g;
            auto op = [&](int j) -> i4 {
                if (j < NSK) {
                    const int st = j >> 1, kt = j & 1;
                    return *reinterpret_cast<const i4*>(krow + kt * 32 * C::LDK + 32 * st);
                }
                const int jp = j - NSK, u = jp / C::NDT, dt = jp % C::NDT;
                const _Float16* base = vrow + (16 * u) * C::LDV + 32 * dt;
                h4 lo = lds_read_tr16(base);
                h4 hi = lds_read_tr16(base + 8 * C::LDV);
                return __builtin_bit_cast(i4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            };
            // SCORES: the raw int32 sums.  Otherwise each chain starts at the bit
            // pattern of kI8Bias, so the int32 result is the fp32 number
            // kI8Bias + S (exact: |S| <= 127^2 D < 2^22, the ulp there is 1)
            const i16x start = SCORES ? i16x{} : bias16;
            i16x acc0 = {}, acc1 = {};
            // dequantisation group u (keys 32 kt + 8 r4 + 4 g .. +3, kt = u / 4,
            // r4 = u % 4), one fma per score: t = (kI8Bias + S) ks - kI8Bias ks,
            // both terms exact (ks has 22 significant bits)
            const float* ksl = sks[i & 1];
            const float* bkl = sbk[i & 1];
            f4 gks = {}, gbk = {};
            auto dq_load = [&](int u) {
                const int o = 32 * (u >> 2) + 8 * (u & 3) + 4 * g;
                gks = *reinterpret_cast<const f4*>(&ksl[o]);
                gbk = *reinterpret_cast<const f4*>(&bkl[o]);
            };
            auto dq_apply = [&](int u) {
                const int kt = u >> 2, r4 = u & 3;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int32_t sv = kt == 0 ? acc0[4 * r4 + e] : acc1[4 * r4 + e];
                    tsc[kt][4 * r4 + e] = fmaf(__int_as_float(sv), gks[e], gbk[e]);
                }
            };
            i4 ring[DEPTH > 0 ? DEPTH : 1];
#pragma unroll
            for (int j = 0; j < DEPTH; j++) {
                ring[j] = op(j);
            }
#pragma unroll
            for (int j = 0; j < T; j++) {
                const i4 a = ring[j % DEPTH];
                if (j + DEPTH < T) {
                    ring[j % DEPTH] = op(j + DEPTH);
                }
                if (j < NSK) {
                    const int st = j >> 1;
                    if (j & 1) {
                        acc1 = mfma_32x32x32_i8(a, qreg[st], st == 0 ? start : acc1);
                    } else {
                        acc0 = mfma_32x32x32_i8(a, qreg[st], st == 0 ? start : acc0);
                    }
                } else {
                    const int jp = j - NSK, u = jp / C::NDT, dt = jp % C::NDT;
                    oacc[dt] = mfma_32x32x16_f16(__builtin_bit_cast(h8, a), pb[u], oacc[dt]);
                    if constexpr (DQ && NPV == 16) {
                        if (jp & 1) {
                            dq_apply(jp >> 1);
                        } else {
                            dq_load(jp >> 1);
                        }
                    } else if constexpr (DQ) {
                        dq_load(jp);
                        dq_apply(jp);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
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
                            srow[k0] = acc0[e];
                        }
                        if (k0 + 32 < Sk) {
                            srow[k0 + 32] = acc1[e];
                        }
                    }
                }
            } else if constexpr (DQ && !DO_PV) {
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    dq_load(u);
                    dq_apply(u);
                }
            }
        };
        auto phase_m = [&](int i) {
            if (!wave_active) {
                return;
            }
            const bool do_pv = !SCORES && i >= 1 && cls_prev != 0;
            const int cls_now = i < n ? tile_class(tcls, t_begin + i) : 0;
            using T_ = std::true_type;
            using F_ = std::false_type;
            if (do_pv && cls_now != 0) {
                mfma_stream(T_{}, T_{}, i);
            } else if (do_pv) {
                mfma_stream(T_{}, F_{}, i);
            } else if (cls_now != 0) {
                mfma_stream(F_{}, T_{}, i);
            }
            cls_prev = cls_now;
        };

        // V(i): exact running max over the 64-key block, P as integers 0..127
        // times the reference factor f; O and l are rescaled only when the
        // reference moves
        auto phase_v = [&](int i) {
            if (SCORES || !wave_active || cls_prev == 0) {
                return;
            }
            f16x (&t)[2] = tsc; // in place: a copy cost 16 moves per tile
            if (!qpos) {
#pragma unroll
                for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        t[kt][e] *= qc;
                    }
                }
            }
            if (cls_prev == 2) {
                const int kt0 = (t_begin + i) * kI8BN;
                const int a = row_lo - kt0 - 4 * g;
                const int bnd = row_hi - kt0 - 4 * g;
#pragma unroll
                for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int off = kt * 32 + 8 * (e >> 2) + (e & 3);
                        t[kt][e] = (off < a || off > bnd) ? -INFINITY : t[kt][e];
                    }
                }
            }
            float mx = t[0][0];
#pragma unroll
            for (int e = 1; e < 16; e++) {
                mx = fmaxf(mx, t[0][e]);
            }
#pragma unroll
            for (int e = 0; e < 16; e++) {
                mx = fmaxf(mx, t[1][e]);
            }
            mx = pair_max(mx) * qeff; // qeff > 0: -inf stays -inf
            m_run = fmaxf(m_run, mx);
            const bool move = m_run > m_ref + kI8RefThreshold; // false while m_run = -inf
            if (wave_any(move)) {
                const float alpha = move ? fast_exp2(m_ref - m_run) : 1.0f; // m_ref = -inf -> 0
                if (move) {
                    m_ref = m_run;
                }
                l_run *= alpha;
#pragma unroll
                for (int dt = 0; dt < C::NDT; dt++) {
                    oacc[dt] *= alpha;
                }
            }
            // m_ref = -inf only while m_run = -inf (no visible key yet: every p is 0)
            const _Float16 f16 = (_Float16)(m_ref == -INFINITY ? 1.0f : fast_exp2(m_run - m_ref));
            const float c0 = int8_exp_offset(m_run);
            const h2 fv = {f16, f16};
            float psum = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                for (int e = 0; e < 16; e += 2) {
                    // y = 127 p (<= 127); h = fp16(1 + y 2^-10) = 1 + round(y) 2^-10
                    // (one v_fma_mix per score: [1, 2) has ulp 2^-10 in fp16),
                    // then h f - f = pq f 2^-10, rounded once (one packed fma)
                    const float y0 = fast_exp2(fmaf(t[kt][e], qeff, c0));
                    const float y1 = fast_exp2(fmaf(t[kt][e + 1], qeff, c0));
                    psum += y0;
                    psum += y1;
                    const h2 hq = {(_Float16)fmaf(y0, kI8PScale, 1.0f), (_Float16)fmaf(y1, kI8PScale, 1.0f)};
                    const h2 pq = hq * fv - fv;
                    pb[kt * 2 + (e >> 3)][e & 7] = pq[0];
                    pb[kt * 2 + (e >> 3)][(e & 7) + 1] = pq[1];
                }
            }
            l_run = fmaf(psum, (float)f16, l_run);
        };

        if (n > 0) {
            load_pair(0);
            store_pair(0);
            load_pair(1);
        }
        __syncthreads();
        if (n > 0) {
            if (grp == 0) {
                for (int i = 0; i < n; i++) {
                    phase_m(i);
                    __syncthreads();
                    store_pair(i + 1);
                    load_pair(i + 2);
                    phase_v(i);
                    __syncthreads();
                }
                phase_m(n);
                __syncthreads();
                __syncthreads();
            } else {
                store_pair(1);
                load_pair(2);
                __syncthreads();
                for (int i = 0; i < n; i++) {
                    phase_m(i);
                    __syncthreads();
                    store_pair(i + 2);
                    load_pair(i + 3);
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
        // O = O^T * v_scale / l (times the per-channel V scales of this kv head
        // when given), through this wave's sO slot
        const float l = pair_sum(l_run);
        const float f = l > 0.0f ? p.v_scale / (l * kI8PScale) : 0.0f;
        const float* vch = p.vch != nullptr ? p.vch + ((int64_t)b * p.Hkv + kvh) * D : nullptr;
        store_o_tile<D, C::LDO>(
            oacc,
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

template <int D, bool VTOK, bool SCORES>
int launch_f16pv(const Int8Params& p, int64_t n_wg, hipStream_t stream, std::string& err) {
    // persistent: as many workgroups as the device holds at once, each
    // walking its share of the n_wg row tiles
    const int64_t resident =
        resident_workgroups(reinterpret_cast<const void*>(&fa_fwd_int8_f16pv<D, VTOK, SCORES>), kI8Threads, err);
    if (resident <= 0) {
        return -1;
    }
    const int64_t grid = std::min(n_wg, resident);
    KernelTimerGuard timer(stream);
    hipLaunchKernelGGL((fa_fwd_int8_f16pv<D, VTOK, SCORES>), dim3((uint32_t)grid), dim3(kI8Threads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

} // namespace

int launch_int8_f16pv(const Int8Params& p, int head_dim, bool scores, int64_t n_wg, hipStream_t stream,
                      std::string& err) {
    const bool vtok = p.vtok != nullptr;
    switch (head_dim) {
    case 64:
        if (vtok && !scores) {
            return launch_f16pv<64, true, false>(p, n_wg, stream, err);
        }
        break;
    case 128:
        if (scores) {
            return launch_f16pv<128, false, true>(p, n_wg, stream, err);
        }
        return vtok ? launch_f16pv<128, true, false>(p, n_wg, stream, err)
                    : launch_f16pv<128, false, false>(p, n_wg, stream, err);
    default: break;
    }
    err = "unsupported head_dim for the fp16 P V int8 kernel";
    return -1;
}

#endif

} // namespace rdna_amd
