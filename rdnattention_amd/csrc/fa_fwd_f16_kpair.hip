// FP16 prefill for head_dim 160..256 on gfx950: the two-group ping-pong of
// the D <= 128 kernel (fa_fwd_f16.hip), with each 32-row tile's work split
// between a pair of waves so that two waves fit on every SIMD.
//
// One wave holding Q^T (D/4 registers per lane) and O^T (D/2) of 32 rows
// needs 192 registers at D = 256 before any score, operand or staging
// register, so the one-wave kernel runs one wave per SIMD, its MFMAs and its
// softmax back to back.  Here waves 2j and 2j+1 (a pair, in the same group)
// own the same 32 query rows, and half h = wave & 1 of the pair
//
//   * computes S^T for keys [32h, 32h + 32) of each 64-key tile, over the
//     full head dimension (Q^T in registers, D/16 MFMAs);
//   * accumulates O^T for d in [C0, C0 + W): [0, DA) for half 0, [DA, D) for
//     half 1, DA = 32 * ceil(D / 64), over all 64 keys (4 W/32 MFMAs).
//
// No work is duplicated.  The pair exchanges three things through LDS, each
// across one of the ping-pong's existing barriers:
//
//   M(i): O^T += V(i-1)^T P(i-1)^T, reading the partner's half of P(i-1) and
//         its row sum; S(i)^T for the own keys; the own tile row max -> LDS
//   V(i): the pair's max = max(own, partner's), the same in both halves, so
//         both make the same rescale decisions; P(i) of the own keys -> LDS
//         together with its row sum
//
// The row sum l adds the two halves' sums in one fixed order, so both halves
// hold the same bits.  Everything else follows fa_fwd_f16_pp: S^T = K Q^T so a
// lane owns one query column, P^T straight from the S accumulator into the
// B operand of O^T = V^T P^T, V^T through transpose reads, the lazy max
// (threshold 2^8), Q pre-scaled into log2 units (PRE), per-row-tile tile
// classes, and (up to D = 192) a persistent grid.
//
// K/V tiles move HBM -> LDS by DMA (buffer_load ... lds), two rows per
// instruction, issued in the softmax phases (K tiles by group B, V tiles by
// group A); the row-pair LDS layout
// (KPCfg) keeps both operand reads free of bank conflicts.  The issuing wave
// waits on each DMA instruction (~70 cycles with four waves issuing), whatever
// its size, so the instruction count sets the cost: one row per DMA cost more
// than the register staging it replaced, and so did DMAs issued between the
// MFMAs of group A's MFMA phase, which they stretched.
#include "fa_common.hpp"
#include "fa_host.hpp"
#include "fa_internal.hpp"
#include "fa_prefill.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace rdna_amd {
namespace {

constexpr int kKPWaves = 8;
constexpr int kKPThreads = 64 * kKPWaves;
constexpr int kKPBN = 64;                  // keys per tile
constexpr float kKPRescaleThreshold = 8.0f; // log2 units
constexpr int kKPWalkBlock = 32;           // row tiles that share a key-tile walk start

template <int D>
struct KPCfg {
    static_assert(D % 32 == 0 && D >= 160 && D <= 256, "head_dim");
    // K/V tiles in LDS as 32 row pairs (rows 2j, 2j + 1), each pair one
    // 1 KB DMA: row 2j's chunk c (16 bytes) at byte 16 c of the pair, row
    // 2j + 1's chunk c at byte 512 + 16 ((c + 8) mod 32).  Pairs lie PSK
    // (PSV) halves apart, 16 (64) bytes more than 1 KB, so that
    //   * the 16-row ds_read_b128 of a K chunk (rows r0 .. r0 + 15, r0 even)
    //     falls on 16 distinct 16-byte bank groups mod 256 B: pair j at
    //     16 j, the odd row a further 16 * 8 = 128 B on;
    //   * the 8-row transpose reads of V (64 bytes per row) fall twice on
    //     each 64-byte quarter of the banks: pair j at 64 j, odd rows +128 B.
    static constexpr int PSK = 520; // halves per K row pair
    static constexpr int PSV = 544; // halves per V row pair
    static constexpr int ODD = 256; // halves from a pair's start to its odd row
    static constexpr int ROT = 64;  // halves of the odd row's chunk rotation (8 chunks)
    static constexpr int TILE_K = (kKPBN / 2) * PSK;
    static constexpr int TILE_V = (kKPBN / 2) * PSV;
    static constexpr int LDK = D + 8; // Q staging rows (halves): the K operand's conflict-free b128 reads
    static constexpr int NS = D / 16;               // Q K^T reduction steps
    static constexpr int DA = 32 * ((D + 63) / 64); // O^T columns of half 0
    static constexpr int DB = D - DA;               // ... of half 1
    static constexpr int KCH = D / 8;               // 16-byte chunks per K/V row
    // Staging: by DMA from D = 224 (wave w of group B moves row pairs 8w ..
    // 8w + 7 of each K tile, of group A of each V tile), below through registers (each group its 32
    // rows, RPI rows per pass, CT passes), which measured faster there: a DMA
    // instruction costs the same however few of its lanes a short row fills
    static constexpr bool DMA = D >= 224;
    static constexpr int DMA_PAIRS = kKPBN / 2 / 4;
    static constexpr int NDMA = 2 * DMA_PAIRS; // DMA instructions of a K and V tile pair per wave
    static constexpr int RPI = (256 / KCH) & ~1;
    static constexpr int CT = (32 + RPI - 1) / RPI;
    static_assert(DMA || RPI * KCH <= 256, "register staging: one chunk per thread and pass");
    // exchange areas: P^T operands [wave][2][64 lanes] of 16 bytes, tile
    // maxima and row sums [wave][64 lanes] of 4 bytes
    static constexpr int KV_BYTES = (2 * TILE_K + 2 * TILE_V) * 2;
    // output staging after the key-tile loop, in the K/V area: [pair][32 rows][LDO]
    static constexpr int LDO = D + 8;
    static_assert(4 * 32 * LDO <= 2 * TILE_K + 2 * TILE_V, "output staging must fit the K/V area");
    // Q staging before the loop: the row tile's 128 rows at the LDK stride, in
    // K slot 1 and the V slots, so that K(0) can land in K slot 0 meanwhile
    static constexpr int Q_STAGE = TILE_K;
    static_assert(4 * 32 * LDK <= TILE_K + 2 * TILE_V, "Q staging must fit K slot 1 and the V slots");
    static_assert(KCH <= 32, "a row fits its 512 bytes of the pair");
    static constexpr int XP_BYTES = kKPWaves * 2 * 64 * 16;
    static constexpr int XS_BYTES = kKPWaves * 64 * 4;
    static constexpr int SMEM_BYTES = KV_BYTES + XP_BYTES + 2 * XS_BYTES;
    // MFMA operands in flight, and a persistent grid up to D = 192: at D = 224
    // and 256 it fits the registers but measured slower, since the static
    // assignment loses the dispatch order that keeps concurrent row tiles on
    // shared key tiles
    static constexpr int OP_DEPTH = 4;
    static constexpr bool PERSIST = D <= 192;
    static_assert(DB % 32 == 0 && DB > 0 && DA >= DB, "halves");
    static_assert(SMEM_BYTES <= 160 * 1024, "LDS");
};

// A group-B wave's DMA operands for one K/V tile pair: the two buffer
// descriptors and the LDS addresses of the wave's first K and V row pairs.
struct DmaPair {
    i32x4_t rk, rv;
    uint32_t mk, mv;
};

// The work of one half (C0, W) of every pair, over the persistent grid's
// row tiles.  Both halves of a group pass the same barriers.
template <int D, bool PRE, int C0, int W>
__device__ __forceinline__ void kpair_half(const PrefillParams& p, char* smem, const int wave) {
    using C = KPCfg<D>;
    constexpr int HALF = C0 == 0 ? 0 : 1;
    constexpr int NDT = W / 32; // O^T row blocks of this half
    _Float16* const sKs = reinterpret_cast<_Float16*>(smem);
    _Float16* const sVs = sKs + 2 * C::TILE_K;
    h8* const xp = reinterpret_cast<h8*>(smem + C::KV_BYTES);
    float* const xmax = reinterpret_cast<float*>(smem + C::KV_BYTES + C::XP_BYTES);
    float* const xsum = xmax + kKPWaves * 64;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const int pair = wave >> 1;
    const int partner = wave ^ 1;
    const int grp = wave >> 2;  // 0 = group A, 1 = group B

    // ---- staging: K/V tiles move HBM -> LDS by DMA (buffer_load ... lds), one
    // instruction per row pair: lane i moves global chunk c of row 2j + i / 32
    // to LDS byte 16 i of the pair, c = i for i < 32 and c = (i - 32 + 24) mod
    // 32 above (the odd row's rotation); lanes whose chunk lies past the row
    // idle.  They are issued in the softmax phases: wave w of group B moves
    // pairs 8w .. 8w + 7 of each K tile, wave w of group A those of each V tile.  The pair's row
    // offset is the instruction's scalar offset, its LDS address M0.
    const uint32_t dma_j0 = (uint32_t)__builtin_amdgcn_readfirstlane((wave & 3) * C::DMA_PAIRS);
    const int dma_c = lane < 32 ? lane : ((lane + 24) & 31);
    const bool dma_lane = dma_c < C::KCH;
    const uint32_t k_row_b = (uint32_t)(p.k_ss * 2), v_row_b = (uint32_t)(p.v_ss * 2);
    const uint32_t dma_vk = (uint32_t)(lane >> 5) * k_row_b + 16u * (uint32_t)dma_c;
    const uint32_t dma_vv = (uint32_t)(lane >> 5) * v_row_b + 16u * (uint32_t)dma_c;
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(smem);
    // Register staging (D <= 192): this group's rows 32 grp .. +31 of K(x)
    // and V(x - 1); thread gtid moves chunk sch of rows r0 + RPI it (RPI even,
    // so every row it moves has r0's parity): one base offset per thread, the
    // pass's row step as the buffer load's scalar offset and as the LDS
    // store's immediate offset.
    const int gtid = tid & 255;
    const int srow = gtid / C::KCH; // < RPI for the busy threads
    const int sch = gtid - srow * C::KCH;
    const bool stager = srow < C::RPI;
    const int r0 = 32 * grp + (stager ? srow : 0);
    const uint32_t coff_k = (uint32_t)(((int64_t)r0 * p.k_ss + 8 * sch) * 2);
    const uint32_t coff_v = (uint32_t)(((int64_t)r0 * p.v_ss + 8 * sch) * 2);
    const int cpos = (r0 & 1) * C::ODD + 8 * ((r0 & 1) ? ((sch + 8) & 31) : sch);
    const int clk = (r0 >> 1) * C::PSK + cpos;
    const int clv = (r0 >> 1) * C::PSV + cpos;
    // pass it moves row r0 + RPI*it, inside the group's 32 rows
    auto stages = [&](int it) { return stager && (32 % C::RPI == 0 || srow + C::RPI * it < 32); };

    auto run_tile = [&](const int wg) {
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
            t_begin = klo / kKPBN;
            n = khi / kKPBN + 1 - t_begin;
        }
        // Key-tile walk: step x visits tile T(x) = t_begin + (x + off) mod n.
        // Under a sliding window the bands of consecutive row tiles start at
        // increasing tiles, and the workgroups running together on an XCD hold
        // consecutive row tiles; each starting at its own band start, they
        // touch that many different tiles per step.  Starting every row tile of
        // a block of kKPWalkBlock at the block's highest band start (when it lies
        // inside the own band) makes them walk the same tiles, at most two
        // distinct ones per step, which then stay in the L2.  Causal bands all
        // start at tile 0: off = 0.
        int off = 0;
        {
            const int rt_hi = min(rt | (kKPWalkBlock - 1), p.n_row_tiles - 1);
            const int hi_q0 = rt_hi * p.rows_per_wg;
            int blo, bhi;
            visible_key_range(p.mask, hi_q0, min(hi_q0 + p.rows_per_wg, p.Sq) - 1, blo, bhi);
            const int c = blo / kKPBN;
            if (bhi >= blo && c > t_begin && c < t_begin + n) {
                off = c - t_begin;
            }
        }
        auto walk = [&](int x) { // T(x) for 0 <= x < n
            const int u = x + off;
            return t_begin + (u >= n ? u - n : u);
        };
        const int Sk = p.mask.sk;
        int row_lo, row_hi;
        row_key_bounds(p.mask, q, row_lo, row_hi);
        // class of key tile T(i) for this pair's rows (0 skip, 1 no mask,
        // 2 masked): both halves of a pair share rows, so they share classes
        const TileClasses tcls = wave_active ? tile_classes<kKPBN>(p.mask, q0, q_hi) : TileClasses{1, 0, 1, 0};

        // Each group sets up pair x = 0, 1, 2, ... in order: K(x) and V(x - 1).
        // The tile addresses advance by one stride per pair and step back n
        // strides where the walk wraps (unsigned arithmetic: tiles past the
        // walk, and V tile -1 of pair 0, are never read; their num_records is
        // 0, so their DMAs write zeros, into slots that no phase reads then).
        const uint64_t k_step = (uint64_t)(kKPBN * p.k_ss * 2), v_step = (uint64_t)(kKPBN * p.v_ss * 2);
        uint64_t k_addr = reinterpret_cast<uint64_t>(kbase) + (uint64_t)((int64_t)(t_begin + off) * kKPBN * p.k_ss * 2);
        uint64_t v_addr = reinterpret_cast<uint64_t>(vbase) + (uint64_t)((int64_t)(t_begin + off - 1) * kKPBN * p.v_ss * 2);
        auto uniform = [](i32x4_t r) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                r[e] = __builtin_amdgcn_readfirstlane(r[e]);
            }
            return r;
        };
        auto dma_pair = [&](int x) {
            const bool k_ok = x < n, v_ok = x >= 1 && x <= n;
            const int tk = k_ok ? walk(x) : 0, tv = v_ok ? walk(x - 1) : 0;
            DmaPair d;
            d.rk = uniform(make_rsrc_v(reinterpret_cast<const void*>(k_addr),
                                       k_ok ? tile_bytes<kKPBN>(Sk - tk * kKPBN, k_row_b, D * 2) : 0u));
            d.rv = uniform(make_rsrc_v(reinterpret_cast<const void*>(v_addr),
                                       v_ok ? tile_bytes<kKPBN>(Sk - tv * kKPBN, v_row_b, D * 2) : 0u));
            d.mk = (uint32_t)__builtin_amdgcn_readfirstlane(
                (int)(lds0 + (uint32_t)(((x & 1) * C::TILE_K + (int)dma_j0 * C::PSK) * 2)));
            d.mv = (uint32_t)__builtin_amdgcn_readfirstlane(
                (int)(lds0 + (uint32_t)((2 * C::TILE_K + ((x - 1) & 1) * C::TILE_V + (int)dma_j0 * C::PSV) * 2)));
            // K(x + 1) is tile t_begin after the wrap at x + 1 + off = n;
            // V(x) likewise after the wrap at x + off = n
            k_addr += k_step - (x + 1 + off == n ? (uint64_t)n * k_step : 0);
            v_addr += v_step - (x + off == n ? (uint64_t)n * v_step : 0);
            return d;
        };
        // DMA k (0 <= k < NDMA) of a tile pair: row pair dma_j0 + k / 2 of
        // the K tile (even k) or of the V tile (odd k)
        auto dma_issue = [&](const DmaPair& d, int k) {
            const uint32_t j = dma_j0 + (uint32_t)(k >> 1);
            const uint32_t so = (uint32_t)__builtin_amdgcn_readfirstlane((int)(2u * j * ((k & 1) ? v_row_b : k_row_b)));
            if (dma_lane) {
                if (k & 1) {
                    dma_load16_s(d.rv, dma_vv, so, d.mv + (uint32_t)((k >> 1) * C::PSV * 2));
                } else {
                    dma_load16_s(d.rk, dma_vk, so, d.mk + (uint32_t)((k >> 1) * C::PSK * 2));
                }
            }
        };
        // the K half (even k, group B) or the V half (odd k, group A) of a tile pair
        auto dma_half = [&](const DmaPair& d, int parity) {
#pragma unroll
            for (int k = 0; k < C::NDMA; k += 2) {
                dma_issue(d, k + parity);
            }
        };

        // Register staging: each group calls load_pair with x = 0, 1, 2, ...
        // in order (the same address stepping) and stores pair x two phases
        // later, whether or not the tiles exist: a missing tile was loaded as
        // zeros into a slot that no phase reads, written on the same schedule
        // as an existing tile (after the last read of the slot's previous
        // contents).
        h8 kreg[C::DMA ? 1 : C::CT], vreg[C::DMA ? 1 : C::CT];
        auto load_pair = [&](int x) {
            const bool k_ok = x < n, v_ok = x >= 1 && x <= n;
            const int tk = k_ok ? walk(x) : 0, tv = v_ok ? walk(x - 1) : 0;
            const auto rk = make_rsrc_uniform(k_addr, k_ok ? tile_bytes<kKPBN>(Sk - tk * kKPBN, k_row_b, D * 2) : 0u);
            const auto rv = make_rsrc_uniform(v_addr, v_ok ? tile_bytes<kKPBN>(Sk - tv * kKPBN, v_row_b, D * 2) : 0u);
            k_addr += k_step - (x + 1 + off == n ? (uint64_t)n * k_step : 0);
            v_addr += v_step - (x + off == n ? (uint64_t)n * v_step : 0);
#pragma unroll
            for (int it = 0; it < C::CT; it++) {
                if (stages(it)) {
                    kreg[it] = buffer_load_h8(rk, coff_k, (uint32_t)(C::RPI * it) * k_row_b);
                    vreg[it] = buffer_load_h8(rv, coff_v, (uint32_t)(C::RPI * it) * v_row_b);
                }
            }
        };
        auto store_pair = [&](int x) {
            _Float16* sK = sKs + (x & 1) * C::TILE_K;
            _Float16* sV = sVs + ((x - 1) & 1) * C::TILE_V;
#pragma unroll
            for (int it = 0; it < C::CT; it++) {
                if (stages(it)) {
                    *reinterpret_cast<h8*>(&sK[clk + (C::RPI / 2) * it * C::PSK]) = kreg[it];
                    *reinterpret_cast<h8*>(&sV[clv + (C::RPI / 2) * it * C::PSV]) = vreg[it];
                }
            }
        };

        // K(0) is in flight while Q^T loads (full head dim, rotated and
        // pre-scaled on the way); V(-1) is not loaded by DMA, its slot holds Q
        const bool dma_wave = __builtin_amdgcn_readfirstlane(grp) == 1;
        if constexpr (C::DMA) {
            if (dma_wave && n > 0) {
                const DmaPair d0 = dma_pair(0);
#pragma unroll
                for (int k = 0; k < C::NDMA; k += 2) {
                    dma_issue(d0, k);
                }
            }
        } else if (n > 0) {
            load_pair(0);
        }
        // Q^T is staged through K slot 1 and the V slots, which are free until
        // the first MFMA phase.  Loaded in the operand layout, each lane would
        // read 16 B of its own row, every load instruction touching 32 rows,
        // and the table loads came in chunks to bound the registers they
        // hold: one round trip per chunk.  Here all 512 threads load the row
        // tile's 128 rows (4 pairs x 32) row-contiguously, KCH lanes per row,
        // with all loads of a thread in flight together, rotate and scale
        // them, and write them at the K rows' stride; each wave then reads
        // its pair's 32 rows with the K operand's conflict-free b128 reads.
        // (These loads are issued after K(0)'s DMAs, so the compiler's waits
        // for them also wait for the DMAs: never too early.)
        h8 qreg[C::NS];
        {
            constexpr int QCT = 4 * 32 * C::KCH / kKPThreads; // chunks per thread
            static_assert(QCT * kKPThreads == 4 * 32 * C::KCH, "Q chunks");
            const int hq0 = kvh * p.ratio + sub * p.G;
            const int gsh = p.G >> 1; // log2 G, G in {1, 2, 4}
            // chunk c of this thread: slot row rj (pair rj / 32), column chunk
            // ch; pair j holds head hq0 + j % G, rows (j / G) * 32 of the tile.
            // Recomputed from an opaque copy of the thread id at each use so
            // that no index stays live across the loads' latency.
            struct Chunk {
                int rj, ch, qr;
            };
            auto chunk = [&](int t, int c) {
                const int idx = t + kKPThreads * c;
                const int rj = idx / C::KCH;
                const int j = rj >> 5;
                return Chunk{rj, idx - rj * C::KCH, wg_q0 + ((j >> gsh) << 5) + (rj & 31)};
            };
            auto head_of = [&](const Chunk& k) { return hq0 + ((k.rj >> 5) & (p.G - 1)); };
            const _Float16* qb = p.q + b * p.q_sb;
            int t = tid;
            asm volatile("" : "+v"(t));
            h8 x[QCT];
#pragma unroll
            for (int c = 0; c < QCT; c++) {
                const Chunk k = chunk(t, c);
                const int src = k.qr < p.Sq ? k.qr : 0;
                x[c] = *reinterpret_cast<const h8*>(qb + head_of(k) * p.q_sh + (int64_t)src * p.q_ss + 8 * k.ch);
            }
            if (p.rope_q) {
                f4 cs[QCT], sn[QCT];
#pragma unroll
                for (int c = 0; c < QCT; c++) {
                    const Chunk k = chunk(t, c);
                    const int64_t off = (int64_t)(k.qr < p.Sq ? k.qr : 0) * (D / 2) + 4 * k.ch;
                    cs[c] = *reinterpret_cast<const f4*>(p.rot_cos + off);
                    sn[c] = *reinterpret_cast<const f4*>(p.rot_sin + off);
                }
#pragma unroll
                for (int c = 0; c < QCT; c++) {
                    x[c] = PRE ? rope8_cs_mul(x[c], cs[c], sn[c], p.qmul) : rope8_cs(x[c], cs[c], sn[c]);
                }
            } else if constexpr (PRE) {
#pragma unroll
                for (int c = 0; c < QCT; c++) {
                    x[c] = scale8(x[c], p.qmul);
                }
            }
            const bool neg = !PRE && p.q_sign < 0.0f; // PRE: the sign is in qmul
            asm volatile("" : "+v"(t));
#pragma unroll
            for (int c = 0; c < QCT; c++) {
                const Chunk k = chunk(t, c);
                *reinterpret_cast<h8*>(&sKs[C::Q_STAGE + k.rj * C::LDK + 8 * k.ch]) =
                    k.qr < p.Sq ? (neg ? -x[c] : x[c]) : h8{};
            }
            __syncthreads();
            const _Float16* src = sKs + C::Q_STAGE + (pair * 32 + l32) * C::LDK + 8 * g;
#pragma unroll
            for (int st = 0; st < C::NS; st++) {
                qreg[st] = *reinterpret_cast<const h8*>(src + 16 * st);
            }
            __syncthreads(); // every wave holds its Q^T before the Q area is overwritten
        }

        f16x oacc[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            oacc[dt] = f16x{};
        }
        float m_run = -INFINITY;
        float m_use = 0.0f; // m_run, or 0 while it is -inf (PRE: the S^T chain starts at -m_use)
        f16x minit = f16x{};
        float l_run = 0.0f;
        f16x sacc = f16x{};
        h8 pb[2]; // P^T operands of the own 16-key groups u = 2 HALF, 2 HALF + 1
        pb[0] = h8{};
        pb[1] = h8{};
        float mx_own = -INFINITY; // own tile row max (of S c - m_use with PRE, else of S)
        float ps_own = 0.0f;      // own row sum of the P held in pb
        int cls_prev = 0;         // class of the tile whose P is held in pb

        // M(i): S(i)^T = K(i) Q^T for the own 32 keys (i < n), then O^T +=
        // V(i-1)^T P(i-1)^T (i >= 1), as one stream of MFMAs whose LDS operands
        // are read C::OP_DEPTH MFMAs ahead through a register ring.  Q K^T first:
        // the partner's P^T, read from LDS as the phase starts, is not needed
        // before the P V MFMAs, and the own scores are done by the phase's end.
        auto mfma_stream = [&](auto do_pv_c, auto do_s_c, int i) {
            constexpr bool DO_PV = decltype(do_pv_c)::value;
            constexpr bool DO_S = decltype(do_s_c)::value;
            constexpr int NPV = DO_PV ? 4 * NDT : 0; // (u, dt)
            constexpr int NSK = DO_S ? C::NS : 0;
            constexpr int T = NPV + NSK;
            constexpr int DEPTH = T < C::OP_DEPTH ? T : C::OP_DEPTH;
            // Operand addresses in the row-pair layout: an odd row's chunk c
            // sits ODD + ROT halves past where the even row's would, or ODD +
            // ROT - 256 for c >= 24 (the rotation wraps).  K: row 32 HALF + l32,
            // chunk 2 st + g, which wraps from st = 12.  V: rows 4 g + j16 / 4
            // (+8, +16 u), columns C0 + 32 dt + 16 x + 4 (j16 % 4), which wrap
            // where C0 + 32 dt >= 192.
            const int j16 = lane & 15;
            const int kodd = (l32 & 1) * 256;
            const int vodd = ((j16 >> 2) & 1) * 256;
            const _Float16* krow = sKs + (i & 1) * C::TILE_K + (16 * HALF + (l32 >> 1)) * C::PSK + 8 * g +
                                   (kodd + (kodd >> 2));
            const _Float16* krow_w = krow - kodd;
            const _Float16* vrow = sVs + ((i - 1) & 1) * C::TILE_V + (2 * g + (j16 >> 3)) * C::PSV + C0 +
                                   16 * ((lane >> 4) & 1) + 4 * (j16 & 3) + (vodd + (vodd >> 2));
            const _Float16* vrow_w = vrow - vodd;
            // the partner's P^T operands (its 16-key groups u = 2 (1 - HALF) + j)
            h8 pop[2];
            if constexpr (DO_PV) {
                pop[0] = xp[(partner * 2 + 0) * 64 + lane];
                pop[1] = xp[(partner * 2 + 1) * 64 + lane];
            }
            auto op = [&](int j) -> h8 {
                if (j < NSK) {
                    return *reinterpret_cast<const h8*>((j < 12 ? krow : krow_w) + 16 * j);
                }
                const int jv = j - NSK, u = jv / NDT, dt = jv % NDT;
                const _Float16* base = (C0 + 32 * dt < 192 ? vrow : vrow_w) + (8 * u) * C::PSV + 32 * dt;
                h4 lo = lds_read_tr16(base);
                h4 hi = lds_read_tr16(base + 4 * C::PSV);
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
                if (j < NSK) {
                    acc = mfma_32x32x16_f16(a, qreg[j], (PRE && j == 0) ? minit : acc);
                } else {
                    const int jv = j - NSK, u = jv / NDT, dt = jv % NDT;
                    const h8 pu = (u >> 1) == HALF ? pb[u & 1] : pop[u & 1];
                    oacc[dt] = mfma_32x32x16_f16(a, pu, oacc[dt]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (DO_S) {
                sacc = acc;
            }
        };
        auto phase_m = [&](int i) {
            if (!wave_active) {
                return;
            }
            const bool do_pv = i >= 1 && cls_prev != 0;
            const int cls_now = i < n ? tile_class(tcls, walk(i)) : 0;
            // the partner's row sum of tile i-1, read now and added after the
            // MFMAs so that the LDS round trip does not hold up the stream
            const float po = do_pv ? xsum[partner * 64 + lane] : 0.0f;
            using T_ = std::true_type;
            using F_ = std::false_type;
            if (do_pv && cls_now != 0) {
                mfma_stream(T_{}, T_{}, i);
            } else if (do_pv) {
                mfma_stream(T_{}, F_{}, i);
            } else if (cls_now != 0) {
                mfma_stream(F_{}, T_{}, i);
            }
            if (do_pv) {
                // the pair's row sum of tile i-1: the same two terms in the same
                // order in both halves
                l_run += HALF == 0 ? ps_own + po : po + ps_own;
            }
            if (cls_now != 0) {
                if (cls_now == 2) {
                    // own key e: kt0 + 32 HALF + 8 (e / 4) + 4 g + e % 4
                    // (4 g from an opaque copy of the lane id: a register
                    // holding it across the row tile is one too many at D = 256)
                    int lane_m = lane;
                    asm volatile("" : "+v"(lane_m));
                    const int kt0 = walk(i) * kKPBN + 32 * HALF + ((lane_m >> 5) << 2);
                    const int a = row_lo - kt0;
                    const int bnd = row_hi - kt0;
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int off = 8 * (e >> 2) + (e & 3);
                        sacc[e] = (off < a || off > bnd) ? -INFINITY : sacc[e];
                    }
                }
                float mx = sacc[0];
#pragma unroll
                for (int e = 1; e < 16; e++) {
                    mx = fmaxf(mx, sacc[e]);
                }
                mx_own = pair_max(mx);
                xmax[wave * 64 + lane] = mx_own;
            }
            cls_prev = cls_now;
        };

        // V(i): the pair's max, rescale, P of the own keys -> pb and LDS
        auto phase_v = [&](int i) {
            (void)i;
            if (!wave_active || cls_prev == 0) {
                return;
            }
            const float mx = fmaxf(mx_own, xmax[partner * 64 + lane]);
            // PRE: mx is a max of S c - m_use; otherwise of S
            const float m_new = PRE ? fmaxf(m_run, mx + m_use) : fmaxf(m_run, mx * p.c);
            const bool grow = m_new > m_run + kKPRescaleThreshold;
            if (wave_any(grow)) {
                const float alpha = grow ? fast_exp2(m_run - m_new) : 1.0f;
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
                    const float shift = m_use - m_use_new;
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        sacc[e] += shift;
                    }
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        minit[e] = -m_use_new;
                    }
                }
                m_use = m_use_new;
            }
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const float x = PRE ? sacc[e] : fmaf(sacc[e], p.c, -m_use);
                pb[e >> 3][e & 7] = (_Float16)fast_exp2(x);
            }
            ps_own = sum_h8(pb[1], sum_h8(pb[0], 0.0f));
            xp[(wave * 2 + 0) * 64 + lane] = pb[0];
            xp[(wave * 2 + 1) * 64 + lane] = pb[1];
            xsum[wave * 64 + lane] = ps_own;
        };

        if constexpr (C::DMA) {
            // K(0) landed (the DMAs are not tracked by the compiler's waits)
            if (dma_wave) {
                __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
            }
        } else if (n > 0) {
            store_pair(0);
            load_pair(1);
        }
        __syncthreads();
        // Group A: M(i) in phase 2i, V(i) in phase 2i + 1; group B one phase
        // later.  K(i) is read in phases 2i and 2i + 1, V(i) in 2i + 2 and
        // 2i + 3.  DMA: group B issues K(i + 2) (K(i)'s slot) at the start of
        // its V(i), in phase 2i + 2, and waits for it at the end of its
        // M(i + 1), phase 2i + 3 (K(1) in phase 0); group A issues V(i)
        // (V(i - 2)'s slot, last read in phase 2i - 1) at the start of its
        // V(i), phase 2i + 1, and waits for it at the end of that phase.  Each
        // softmax side thus carries 8 DMAs per wave per tile, not 0 and 16
        // (two-sided window +-2048 + RoPE, B1 H16 S16384 D256: -1.9 %; D224
        // non-causal -3.8 %).  Registers: each group stores pair i + 1 (A) or i + 2 (B) and
        // loads the next in its V(i).  Both groups pass 2n + 2 barriers after
        // the prologue's.
        if (n > 0) {
            if (grp == 0) {
                if constexpr (C::DMA) {
                    (void)dma_pair(0); // the address stepping starts at pair 0
                }
                for (int i = 0; i < n; i++) {
                    phase_m(i);
                    __syncthreads();
                    if constexpr (!C::DMA) {
                        store_pair(i + 1);
                        load_pair(i + 2);
                    } else {
                        dma_half(dma_pair(i + 1), 1); // V(i)
                    }
                    phase_v(i);
                    if constexpr (C::DMA) {
                        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); // V(i) landed
                    }
                    __syncthreads();
                }
                phase_m(n);
                __syncthreads();
                __syncthreads();
            } else {
                if constexpr (C::DMA) {
                    if (1 < n) {
                        dma_half(dma_pair(1), 0);
                    }
                } else {
                    store_pair(1);
                    load_pair(2);
                }
                __syncthreads();
                for (int i = 0; i < n; i++) {
                    phase_m(i);
                    if constexpr (C::DMA) {
                        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); // K(i + 1) landed
                    }
                    __syncthreads();
                    if constexpr (C::DMA) {
                        if (i + 2 < n) {
                            dma_half(dma_pair(i + 2), 0); // K(i + 2)
                        }
                    } else {
                        store_pair(i + 2);
                        load_pair(i + 3);
                    }
                    phase_v(i);
                    __syncthreads();
                }
                phase_m(n);
                __syncthreads();
            }
        }

        // O = O^T / l.  Every LDS read of the row tile finished before the last
        // barrier, so the K/V area is free: each half writes its columns of the
        // pair's 32 rows into the pair's slot there, and after a barrier each
        // half stores 16 of those rows whole, 16 bytes per lane, non-temporal
        // (O is not read again; streaming it past the L2 keeps the K/V tiles
        // that other row tiles reuse resident).
        _Float16* const oslot = sKs + pair * 32 * C::LDO;
        if (wave_active) {
            const float l = pair_sum(l_run);
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
#pragma unroll
                for (int qq = 0; qq < 4; qq++) {
                    h4 o4 = {(_Float16)(oacc[dt][4 * qq + 0] * inv), (_Float16)(oacc[dt][4 * qq + 1] * inv),
                             (_Float16)(oacc[dt][4 * qq + 2] * inv), (_Float16)(oacc[dt][4 * qq + 3] * inv)};
                    *reinterpret_cast<h4*>(oslot + l32 * C::LDO + C0 + dt * 32 + 8 * qq + 4 * g) = o4;
                }
            }
        }
        __syncthreads(); // both halves' columns are in the slot
        if (wave_active) {
            // 32 lanes per row (D/8 <= 32 of them busy), 2 rows per pass; the
            // indices come from an opaque copy of the lane id so that they are
            // not hoisted above the key-tile loop
            int lane_e = lane;
            asm volatile("" : "+v"(lane_e));
            const int r0 = 16 * HALF + (lane_e >> 5);
            const int ch = lane_e & 31;
            _Float16* const orow0 = p.o + b * p.o_sb + h * p.o_sh + (int64_t)(q0 + r0) * p.o_ss + 8 * ch;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const int r = r0 + 2 * c;
                if (ch < C::KCH && q0 + r < p.Sq) {
                    const h8 o8 = *reinterpret_cast<const h8*>(oslot + r * C::LDO + 8 * ch);
                    __builtin_nontemporal_store(o8, reinterpret_cast<h8*>(orow0 + (int64_t)(2 * c) * p.o_ss));
                }
            }
        }
        if constexpr (C::PERSIST) {
            __syncthreads(); // the next row tile's prologue writes the K/V area
        }
    };
    if constexpr (C::PERSIST) {
        for (int item = 0;; item++) {
            const int wg = persistent_item(blockIdx.x, gridDim.x, item, p.n_items);
            if (wg < 0) {
                break;
            }
            run_tile(wg);
        }
    } else {
        run_tile(blockIdx.x);
    }
}

template <int D, bool PRE>
__global__ __launch_bounds__(kKPThreads, 1) void fa_fwd_f16_kpair(PrefillParams p) {
    using C = KPCfg<D>;
    __shared__ __attribute__((aligned(16))) char smem[C::SMEM_BYTES];
    // The branch between the halves must be wave-uniform (both sides pass
    // barriers), so its condition is read from the first lane; the wave index
    // itself stays a vector value (made uniform, everything derived from it
    // moves to scalar registers and the kernel spills).
    const int wave = threadIdx.x >> 6;
    if (__builtin_amdgcn_readfirstlane(wave & 1) == 0) {
        kpair_half<D, PRE, 0, C::DA>(p, smem, wave);
    } else {
        kpair_half<D, PRE, C::DA, C::DB>(p, smem, wave);
    }
}

template <int D, bool PRE>
int launch_kpair_as(const PrefillParams& p, int64_t n_wg, hipStream_t stream, std::string& err) {
    // persistent: as many workgroups as the device holds at once
    int64_t grid = n_wg;
    if (KPCfg<D>::PERSIST) {
        const int64_t resident =
            resident_workgroups(reinterpret_cast<const void*>(&fa_fwd_f16_kpair<D, PRE>), kKPThreads, err);
        if (resident <= 0) {
            return -1;
        }
        grid = std::min(n_wg, resident);
    }
    KernelTimerGuard timer(stream);
    hipLaunchKernelGGL((fa_fwd_f16_kpair<D, PRE>), dim3((uint32_t)grid), dim3(kKPThreads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

template <int D>
int launch_kpair_d(const PrefillParams& p, int64_t n_wg, hipStream_t stream, std::string& err) {
    // Q pre-scaled into log2 units when |q| c stays representable (c <= 1);
    // not above D = 192, where the 16 registers of the accumulator start
    // would spill inside the key-tile loop
    constexpr bool kPre = D <= 192;
    if (kPre && p.c <= 1.0f) {
        return launch_kpair_as<D, kPre>(p, n_wg, stream, err);
    }
    return launch_kpair_as<D, false>(p, n_wg, stream, err);
}

} // namespace

int launch_kpair(const PrefillParams& p, int head_dim, int64_t n_wg, hipStream_t stream, std::string& err) {
    switch (head_dim) {
    case 160: return launch_kpair_d<160>(p, n_wg, stream, err);
    case 192: return launch_kpair_d<192>(p, n_wg, stream, err);
    case 224: return launch_kpair_d<224>(p, n_wg, stream, err);
    case 256: return launch_kpair_d<256>(p, n_wg, stream, err);
    default: break;
    }
    err = "unsupported head_dim for the wave-pair prefill kernel";
    return -1;
}

} // namespace rdna_amd
