// FP16 prefill for head_dim 288..512 on gfx950: the two-group ping-pong of
// the smaller-head kernels (fa_fwd_f16.hip, fa_fwd_f16_kpair.hip), with the
// head dimension of each 32-row tile split between a pair of waves so that two
// waves fit on every SIMD.
//
// One wave holding Q^T (D/4 registers per lane) and O^T (D/2) of 32 rows
// needs 216 (D = 288) to 384 (D = 512) registers, so a one-wave-per-row-tile
// kernel runs one wave per SIMD with its MFMAs and its softmax back to back.  Here waves 2j
// and 2j+1 (a pair, in the same group) own the same 32 query rows, and half
// h = wave & 1 owns the head-dimension range [C0, C0 + W): [0, DA) for half
// 0, [DA, D) for half 1, DA = 32 * ceil(D / 64).  Per 32-key tile each half
// computes the partial S_h^T = K[:, C0:C0+W] Q[:, C0:C0+W]^T (W/16 MFMAs) and
// O_h^T += V[:, C0:C0+W]^T P^T (W/16 MFMAs): 32 MFMAs per phase at D = 512,
// as in the D <= 128 kernel, 20 at D = 288.
//
// The softmax runs once per pair, in half 0; the pair talks through a small
// per-pair LDS area, across the ping-pong's existing barriers:
//
//   M(i): half 1 first reads P(i-1)^T and the rescale factor alpha(i-1) that
//         half 0 left there, and rescales its O^T when alpha != 1; both halves
//         compute S_h(i)^T, then O_h^T += V(i-1)^T P(i-1)^T; half 1 writes its
//         partial S_1(i)^T to the area
//   V(i): half 0 adds S_1(i)^T to its S_0(i)^T, runs the online softmax
//         (lazy max, threshold 2^8), rescales its O^T, and writes P(i)^T and
//         alpha(i) over the partial it has read
//
// Only half 0 keeps the running max and row sum; it hands 1/l to half 1 after
// the loop.  K/V tiles of 32 keys move HBM -> LDS by buffer_load ... lds, one
// DMA instruction per row into padded rows (K at D + 8 halves, V at = 32 mod
// 128 halves: the 16-row ds_read_b128 of K and the 4-row transpose reads of V
// hit distinct banks), double-buffered.  The half-1 waves, whose softmax
// phase is otherwise empty, issue the DMAs there: group B's the K tiles two
// phases before they are read, group A's the V tiles one phase before; with
// the issue split over four waves a tile's DMAs are in flight sooner than
// from two (D 384 +4-5 %, c5b +0.7 %).  Key tiles are walked
// from the aligned start of fa_fwd_f16_kpair.hip, skipped outside the
// causal/window band and masked only at its edges.
#include "fa_common.hpp"
#include "fa_host.hpp"
#include "fa_internal.hpp"
#include "fa_prefill.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace rdna_amd {
namespace {

constexpr int kDPWaves = 8;
constexpr int kDPThreads = 64 * kDPWaves;
constexpr int kDPBN = 32;                  // keys per tile
constexpr float kDPRescaleThreshold = 8.0f; // log2 units
constexpr int kDPWalkBlock = 32;           // row tiles that share a key-tile walk start

template <int D>
struct DPCfg {
    static_assert(D % 32 == 0 && D >= 288 && D <= 512, "head_dim");
    static constexpr int DA = 32 * ((D + 63) / 64); // head-dim range of half 0
    static constexpr int DB = D - DA;               // ... of half 1
    static constexpr int LDK = D + 8;                              // halves
    static constexpr int LDV = D + ((32 - D % 128) + 128) % 128;   // halves, = 32 (mod 128)
    static constexpr int TILE_K = kDPBN * LDK;                     // halves
    static constexpr int TILE_V = kDPBN * LDV;
    static constexpr int KV_BYTES = (2 * TILE_K + 2 * TILE_V) * 2;
    static constexpr int KCH = D / 8; // 16-byte chunks per row = DMA lanes
    // per-pair exchange area: half 1's partial S^T ([4][64 lanes] of 16 bytes),
    // overwritten by half 0's P^T ([2][64 lanes] of 16 bytes); alpha [64 lanes]
    static constexpr int XS_BYTES = 4 * 64 * 16;
    static constexpr int XPAIR_BYTES = XS_BYTES + 64 * 4;
    static constexpr int SMEM_BYTES = KV_BYTES + (kDPWaves / 2) * XPAIR_BYTES;
    // rows of each K and V tile one DMA-issuing wave moves (two such waves)
    static constexpr int DMA_ROWS = kDPBN / 2;
    // MFMA operands in flight: a deeper ring gains 0.3-2 % where it fits the
    // 256 registers, up to D = 448
    static constexpr int OP_DEPTH = D <= 448 ? 4 : 2;
    static_assert(DB % 32 == 0 && DB > 0 && DA >= DB, "halves");
    static_assert(LDV % 128 == 32 && LDV >= D, "V stride");
    static_assert(KCH <= 64, "one DMA instruction per row");
    static_assert(SMEM_BYTES <= 160 * 1024, "LDS");
};

// The work of one half (C0, W) of every pair over one row tile.  Both
// halves of a group pass the same barriers.
template <int D, bool PRE, int C0, int W>
__device__ __forceinline__ void dpair_half(const PrefillParams& p, char* smem, const int wave) {
    using C = DPCfg<D>;
    constexpr int HALF = C0 == 0 ? 0 : 1;
    constexpr int NS = W / 16;  // QK^T reduction steps of this half
    constexpr int NDT = W / 32; // O^T row blocks of this half
    _Float16* const sKs = reinterpret_cast<_Float16*>(smem);
    _Float16* const sVs = sKs + 2 * C::TILE_K;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const int pair = wave >> 1;
    const int grp = wave >> 2; // 0 = group A, 1 = group B
    char* const xpair = smem + C::KV_BYTES + pair * C::XPAIR_BYTES;
    f4* const xs = reinterpret_cast<f4*>(xpair);
    h8* const xp = reinterpret_cast<h8*>(xpair);
    float* const xa = reinterpret_cast<float*>(xpair + C::XS_BYTES);
    // group B's half-1 waves issue the K DMAs, group A's the V DMAs; the group
    // is read from the first lane so that these branches, and the DMA
    // addresses inside them, are scalar
    const int grp_u = __builtin_amdgcn_readfirstlane(grp);
    const bool dma_k = HALF == 1 && grp_u == 1;
    const bool dma_v = HALF == 1 && grp_u == 0;

    const int wg = blockIdx.x;
    int hg, rt;
    wg_tile(wg, p.n_head_groups, p.n_row_tiles, p.hg_chunk, hg, rt);
    const int per_b = p.Hkv * p.groups_per_kv;
    const int b = hg / per_b;
    const int rem = hg - b * per_b;
    const int kvh = rem / p.groups_per_kv;
    const int sub = rem - kvh * p.groups_per_kv;
    // pair j takes head j % G, rows (j / G) * 32 .. +31 of the row tile
    const int h = kvh * p.ratio + sub * p.G + (pair % p.G);
    const int wg_q0 = rt * p.rows_per_wg;
    const int q0 = wg_q0 + (pair / p.G) * 32;
    const int q = q0 + l32;
    const bool wave_active = q0 < p.Sq;
    const int q_hi = min(q0 + 31, p.Sq - 1);

    const _Float16* kbase = p.k + b * p.k_sb + kvh * p.k_sh;
    const _Float16* vbase = p.v + b * p.v_sb + kvh * p.v_sh;

    const int wg_q_hi = min(wg_q0 + p.rows_per_wg, p.Sq) - 1;
    int klo, khi;
    visible_key_range(p.mask, wg_q0, wg_q_hi, klo, khi);
    int t_begin = 0, n = 0;
    if (khi >= klo) {
        t_begin = klo / kDPBN;
        n = khi / kDPBN + 1 - t_begin;
    }
    // Key-tile walk: step x visits tile T(x) = t_begin + (x + off) mod n, with
    // every row tile of a block of kDPWalkBlock starting at the block's highest
    // band start when that lies inside its own band (fa_fwd_f16_kpair.hip), so
    // that the workgroups running together read the same tiles.
    int off = 0;
    {
        const int rt_hi = min(rt | (kDPWalkBlock - 1), p.n_row_tiles - 1);
        const int hi_q0 = rt_hi * p.rows_per_wg;
        int blo, bhi;
        visible_key_range(p.mask, hi_q0, min(hi_q0 + p.rows_per_wg, p.Sq) - 1, blo, bhi);
        const int c = blo / kDPBN;
        if (bhi >= blo && c > t_begin && c < t_begin + n) {
            off = c - t_begin;
        }
    }
    auto walk = [&](int x) { // T(x) for 0 <= x < n
        const int u = x + off;
        return t_begin + (u >= n ? u - n : u);
    };
    int row_lo, row_hi;
    row_key_bounds(p.mask, q, row_lo, row_hi);
    // both halves of a pair share rows, so they share tile classes
    const TileClasses tcls = wave_active ? tile_classes<kDPBN>(p.mask, q0, q_hi) : TileClasses{1, 0, 1, 0};

    // DMAs of a K or V tile: rows dma_r0 .. dma_r0 + 15, lane i moving bytes
    // 16i .. 16i+15 of each row.
    // The row offsets and LDS row addresses are wave-uniform and stepped row by
    // row in scalar registers from an opaque start, so that no per-row value is
    // precomputed and kept across the key-tile loop.
    const uint32_t k_row_b = (uint32_t)(p.k_ss * 2), v_row_b = (uint32_t)(p.v_ss * 2);
    const uint32_t dma_r0 = (uint32_t)__builtin_amdgcn_readfirstlane(((wave >> 1) & 1) * C::DMA_ROWS);
    const uint32_t lane_b = 16u * (uint32_t)lane;
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(smem);
    auto issue_rows = [&](i32x4_t rsrc, uint32_t row_b, uint32_t lds_row0, uint32_t lds_row_b) {
        uint32_t so = dma_r0 * row_b;
        uint32_t m = lds_row0 + dma_r0 * lds_row_b;
        asm volatile("" : "+s"(so), "+s"(m));
        if (lane < C::KCH) {
#pragma unroll
            for (int j = 0; j < C::DMA_ROWS; j++) {
                dma_load16_s(rsrc, lane_b, so, m);
                so += row_b;
                m += lds_row_b;
            }
        }
    };
    auto uniform = [](i32x4_t r) {
        for (int e = 0; e < 4; e++) {
            r[e] = __builtin_amdgcn_readfirstlane(r[e]);
        }
        return r;
    };
    // K(x) into K slot x % 2 (x < n); V(x) into V slot x % 2 (x < n)
    auto issue_k = [&](int x0) {
        const int x = __builtin_amdgcn_readfirstlane(x0);
        const int kt0 = walk(x) * kDPBN;
        const i32x4_t rk = uniform(
            make_rsrc_v(kbase + (int64_t)kt0 * p.k_ss, tile_bytes<kDPBN>(p.mask.sk - kt0, k_row_b, D * 2)));
        issue_rows(rk, k_row_b, lds0 + (uint32_t)((x & 1) * C::TILE_K * 2), C::LDK * 2);
    };
    auto issue_v = [&](int x0) {
        const int x = __builtin_amdgcn_readfirstlane(x0);
        const int vt0 = walk(x) * kDPBN;
        const i32x4_t rv = uniform(
            make_rsrc_v(vbase + (int64_t)vt0 * p.v_ss, tile_bytes<kDPBN>(p.mask.sk - vt0, v_row_b, D * 2)));
        issue_rows(rv, v_row_b, lds0 + (uint32_t)((2 * C::TILE_K + (x & 1) * C::TILE_V) * 2), C::LDV * 2);
    };

    // Q^T operand of d-range [C0, C0 + W): lane holds Q[q][C0 + 16s + 8g .. +7]
    h8 qreg[NS];
    {
        const bool valid = q < p.Sq;
        const int qr = valid ? q : 0;
        const _Float16* qbase = p.q + b * p.q_sb + h * p.q_sh;
        load_q_operand<NS, 8>(qreg, qbase + (int64_t)qr * p.q_ss + C0, p.rot_cos + (int64_t)qr * (D / 2) + C0 / 2,
                              p.rot_sin + (int64_t)qr * (D / 2) + C0 / 2, g, valid, p.rope_q != 0, p.q_sign < 0.0f,
                              PRE ? p.qmul : 0.0f);
    }
    // Q is in registers before the first DMA, so the vmcnt waits below only
    // ever wait for DMAs (which the compiler does not track)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));

    f16x oacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        oacc[dt] = f16x{};
    }
    float m_run = -INFINITY; // half 0 only
    float m_use = 0.0f;      // m_run, or 0 while it is -inf
    f16x minit = f16x{};     // PRE, half 0: the S^T chain starts at -m_use
    float l_run = 0.0f;
    f16x sacc = f16x{};
    h8 pb[2]; // half 0: P^T of the tile whose PV is pending
    pb[0] = h8{};
    pb[1] = h8{};
    int cls_prev = 0; // class of the tile whose P is pending

    // M(i): S_h(i)^T = K(i) Q^T over this half's d-range (i < n), then
    // O_h^T += V(i-1)^T P(i-1)^T (i >= 1), as one stream of MFMAs whose LDS
    // operands are read C::OP_DEPTH MFMAs ahead through a register ring
    auto mfma_stream = [&](auto do_s_c, auto do_pv_c, int i) {
        constexpr bool DO_S = decltype(do_s_c)::value;
        constexpr bool DO_PV = decltype(do_pv_c)::value;
        constexpr int NSK = DO_S ? NS : 0;
        constexpr int NPV = DO_PV ? 2 * NDT : 0; // (u, dt)
        constexpr int T = NSK + NPV;
        constexpr int DEPTH = T < C::OP_DEPTH ? T : C::OP_DEPTH;
        const int j16 = lane & 15;
        const _Float16* krow = sKs + (i & 1) * C::TILE_K + l32 * C::LDK + C0 + 8 * g;
        const _Float16* vrow = sVs + ((i - 1) & 1) * C::TILE_V + (4 * g + (j16 >> 2)) * C::LDV + C0 +
                               16 * ((lane >> 4) & 1) + 4 * (j16 & 3);
        // half 1: P(i-1)^T and alpha(i-1) from half 0
        h8 pop[2];
        float alpha = 1.0f;
        if constexpr (DO_PV && HALF == 1) {
            pop[0] = xp[lane];
            pop[1] = xp[64 + lane];
            alpha = xa[lane];
        }
        auto op = [&](int j) -> h8 {
            if (j < NSK) {
                return *reinterpret_cast<const h8*>(krow + 16 * j);
            }
            const int jv = j - NSK, u = jv / NDT, dt = jv % NDT;
            const _Float16* base = vrow + (16 * u) * C::LDV + 32 * dt;
            h4 lo = lds_read_tr16(base);
            h4 hi = lds_read_tr16(base + 8 * C::LDV);
            return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        };
        f16x acc = {};
        h8 ring[DEPTH > 0 ? DEPTH : 1];
#pragma unroll
        for (int j = 0; j < DEPTH; j++) {
            ring[j] = op(j);
        }
#pragma unroll
        for (int j = 0; j < T; j++) {
            const h8 a = ring[j % DEPTH];
            if (j + DEPTH < T) {
                ring[j % DEPTH] = op(j + DEPTH);
            }
            if constexpr (DO_PV && HALF == 1) {
                if (j == NSK) {
                    // half 0 rescaled its O^T in V(i-1); this half does so before
                    // adding tile i-1 (alpha = 1 on every lane when it did not)
                    if (wave_any(alpha != 1.0f)) {
#pragma unroll
                        for (int dt = 0; dt < NDT; dt++) {
                            oacc[dt] *= alpha;
                        }
                    }
                }
            }
            if (j < NSK) {
                // PRE: only half 0's chain starts at -m_use, so the pair's sum holds it once
                acc = mfma_32x32x16_f16(a, qreg[j], (PRE && HALF == 0 && j == 0) ? minit : acc);
            } else {
                const int jv = j - NSK, u = jv / NDT, dt = jv % NDT;
                oacc[dt] = mfma_32x32x16_f16(a, HALF == 0 ? pb[u] : pop[u], oacc[dt]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (DO_S) {
            if constexpr (HALF == 1) {
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    xs[q4 * 64 + lane] = f4{acc[4 * q4], acc[4 * q4 + 1], acc[4 * q4 + 2], acc[4 * q4 + 3]};
                }
            } else {
                sacc = acc;
            }
        }
    };
    auto phase_m = [&](int i) {
        if (!wave_active) {
            return;
        }
        const bool do_pv = i >= 1 && cls_prev != 0;
        const int cls_now = i < n ? tile_class(tcls, walk(i)) : 0;
        using T_ = std::true_type;
        using F_ = std::false_type;
        if (do_pv && cls_now != 0) {
            mfma_stream(T_{}, T_{}, i);
        } else if (do_pv) {
            mfma_stream(F_{}, T_{}, i);
        } else if (cls_now != 0) {
            mfma_stream(T_{}, F_{}, i);
        }
        cls_prev = cls_now;
    };

    // V(i), half 0: S = S_0 + S_1, the online softmax, P(i)^T and alpha(i) -> LDS
    auto phase_v = [&](int i) {
        if constexpr (HALF == 0) {
            if (!wave_active || cls_prev == 0) {
                return;
            }
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const f4 o = xs[q4 * 64 + lane];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    sacc[4 * q4 + e] += o[e];
                }
            }
            if (cls_prev == 2) {
                // key e of the tile: kt0 + 8 (e / 4) + 4 g + e % 4
                const int kt0 = walk(i) * kDPBN;
                const int a = row_lo - kt0 - 4 * g;
                const int bnd = row_hi - kt0 - 4 * g;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int o8 = 8 * (e >> 2) + (e & 3);
                    sacc[e] = (o8 < a || o8 > bnd) ? -INFINITY : sacc[e];
                }
            }
            float mx = max_tree<16>([&](int e) { return sacc[e]; });
            mx = pair_max(mx);
            // PRE: mx is a max of S c - m_use; otherwise of S (c > 0: -inf stays -inf)
            const float m_new = PRE ? fmaxf(m_run, mx + m_use) : fmaxf(m_run, mx * p.c);
            const bool grow = m_new > m_run + kDPRescaleThreshold;
            float alpha = 1.0f;
            if (wave_any(grow)) {
                alpha = grow ? fast_exp2(m_run - m_new) : 1.0f; // m_run = -inf -> 0
                if (grow) {
                    m_run = m_new;
                }
                l_run *= alpha;
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) {
                    oacc[dt] *= alpha;
                }
                const float m_use_new = (m_run == -INFINITY) ? 0.0f : m_run;
                if constexpr (PRE) {
                    // re-base this tile's exponents and the next tiles' start
                    const float shift = m_use - m_use_new;
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        sacc[e] += shift;
                        minit[e] = -m_use_new;
                    }
                }
                m_use = m_use_new;
            }
#pragma unroll
            for (int e = 0; e < 16; e++) {
                pb[e >> 3][e & 7] = (_Float16)fast_exp2(PRE ? sacc[e] : fmaf(sacc[e], p.c, -m_use));
            }
            l_run += sum_h8(pb[0], 0.0f) + sum_h8(pb[1], 0.0f); // two independent chains
            xp[lane] = pb[0];
            xp[64 + lane] = pb[1];
            xa[lane] = alpha;
        } else {
            (void)i;
        }
    };

    // Prologue: K(0) landed before the first barrier
    if (dma_k && n > 0) {
        issue_k(0);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    }
    __syncthreads();
    // Group A: M(i) in phase 2i, V(i) in phase 2i + 1; group B one phase later.
    // K(i) is read in phases 2i and 2i + 1, V(i) in 2i + 2 and 2i + 3.  K(i + 2)
    // reuses K(i)'s slot: group B's half-1 waves issue it at the start of phase
    // 2i + 2 and wait for it at the end of phase 2i + 3.  V(i) reuses V(i - 2)'s
    // slot: group A's half-1 waves issue it at the start of phase 2i + 1 and
    // wait for it at the end of that phase.  Both groups pass 2n + 2 barriers.
    if (n > 0) {
        if (grp == 0) {
            for (int i = 0; i < n; i++) {
                phase_m(i);
                __syncthreads();
                if (dma_v) {
                    issue_v(i);
                }
                phase_v(i);
                if (dma_v) {
                    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); // V(i) landed
                }
                __syncthreads();
            }
            phase_m(n);
            __syncthreads();
            __syncthreads();
        } else {
            if (dma_k && 1 < n) {
                issue_k(1);
            }
            __syncthreads();
            for (int i = 0; i < n; i++) {
                phase_m(i);
                if (dma_k) {
                    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); // K(i + 1) landed
                }
                __syncthreads();
                if (dma_k && i + 2 < n) {
                    issue_k(i + 2);
                }
                phase_v(i);
                __syncthreads();
            }
            phase_m(n);
            __syncthreads();
        }
    }

    // O = O^T / l: half 0 hands 1/l to half 1 through the pair's area (its
    // address recomputed from an opaque copy of the thread id, so that it is
    // not kept in a register across the key-tile loop)
    int tid_e = tid;
    asm volatile("" : "+v"(tid_e));
    float* const xa_e = reinterpret_cast<float*>(smem + C::KV_BYTES + (tid_e >> 7) * C::XPAIR_BYTES + C::XS_BYTES);
    float inv = 0.0f;
    if constexpr (HALF == 0) {
        const float l = pair_sum(l_run);
        inv = l > 0.0f ? 1.0f / l : 0.0f;
        xa_e[lane] = inv;
    }
    __syncthreads();
    if constexpr (HALF == 1) {
        inv = xa_e[lane];
    }
    if (wave_active && q < p.Sq) {
        _Float16* orow = p.o + b * p.o_sb + h * p.o_sh + (int64_t)q * p.o_ss + C0;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                h4 o4 = {(_Float16)(oacc[dt][4 * qq + 0] * inv), (_Float16)(oacc[dt][4 * qq + 1] * inv),
                         (_Float16)(oacc[dt][4 * qq + 2] * inv), (_Float16)(oacc[dt][4 * qq + 3] * inv)};
                *reinterpret_cast<h4*>(orow + dt * 32 + 8 * qq + 4 * g) = o4;
            }
        }
    }
}

template <int D, bool PRE>
__global__ __launch_bounds__(kDPThreads, 1) void fa_fwd_f16_dpair(PrefillParams p) {
    using C = DPCfg<D>;
    __shared__ __attribute__((aligned(16))) char smem[C::SMEM_BYTES];
    // The branch between the halves must be wave-uniform (both sides pass
    // barriers), so its condition is read from the first lane; the wave index
    // itself stays a vector value.
    const int wave = threadIdx.x >> 6;
    if (__builtin_amdgcn_readfirstlane(wave & 1) == 0) {
        dpair_half<D, PRE, 0, C::DA>(p, smem, wave);
    } else {
        dpair_half<D, PRE, C::DA, C::DB>(p, smem, wave);
    }
}

template <int D>
int launch_dpair_d(const PrefillParams& p, int64_t n_wg, hipStream_t stream, std::string& err) {
    KernelTimerGuard timer(stream);
    // Q pre-scaled into log2 units when |q| c stays representable (c <= 1); not
    // above D = 448, where the 16 registers of half 0's accumulator start do
    // not fit
    constexpr bool kPre = D <= 448;
    if (kPre && p.c <= 1.0f) {
        hipLaunchKernelGGL((fa_fwd_f16_dpair<D, kPre>), dim3((uint32_t)n_wg), dim3(kDPThreads), 0, stream, p);
    } else {
        hipLaunchKernelGGL((fa_fwd_f16_dpair<D, false>), dim3((uint32_t)n_wg), dim3(kDPThreads), 0, stream, p);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

} // namespace

int launch_dpair(const PrefillParams& p, int head_dim, int64_t n_wg, hipStream_t stream, std::string& err) {
    switch (head_dim) {
    case 288: return launch_dpair_d<288>(p, n_wg, stream, err);
    case 320: return launch_dpair_d<320>(p, n_wg, stream, err);
    case 352: return launch_dpair_d<352>(p, n_wg, stream, err);
    case 384: return launch_dpair_d<384>(p, n_wg, stream, err);
    case 416: return launch_dpair_d<416>(p, n_wg, stream, err);
    case 448: return launch_dpair_d<448>(p, n_wg, stream, err);
    case 480: return launch_dpair_d<480>(p, n_wg, stream, err);
    case 512: return launch_dpair_d<512>(p, n_wg, stream, err);
    default: break;
    }
    err = "unsupported head_dim for the head-dimension pair prefill kernel";
    return -1;
}

} // namespace rdna_amd
