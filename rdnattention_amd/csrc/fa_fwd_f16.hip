// FP16 FlashAttention-2 forward for gfx950 (MI355X): the prefill kernel for
// head_dim <= 128 and the FP16 dispatcher (D 160..256: fa_fwd_f16_kpair.hip,
// D 288..512: fa_fwd_f16_dpair.hip, decode: fa_fwd_decode.hip).
//
// Replaces the reference's forwardKernel / forwardKernelGqa
// (src/rdna/fa2_forward_f16.hip:633-877) with a CDNA4 MFMA design:
//
//   * fa_fwd_f16_pp<D> (D <= 128): 8 waves in two groups that alternate an
//     MFMA phase and a softmax + staging phase (ping-pong, described above
//     the kernel); persistent grid from D = 64 up; Q staged through LDS with
//     row-contiguous loads; output stored through LDS as whole rows,
//     non-temporal
//   * every wave owns 32 query rows of one head and a workgroup holds G query
//     heads of one kv head (G | Hq/Hkv, G <= 4), so each K/V tile staged in
//     LDS serves all of them
//   * S^T = K Q^T on v_mfma_f32_32x32x16_f16: a lane owns one query column,
//     so the row max/sum are lane-local plus one exchange across half-waves
//   * P^T leaves the S^T accumulator in exactly the B-operand layout of the
//     O^T = V^T P^T MFMA, so P never touches LDS; V^T operands come from
//     row-major V tiles through ds_read_b64_tr_b16 transpose reads
//   * key tiles outside the causal/window band are skipped, tiles inside it
//     run a mask-free path, only boundary tiles evaluate the mask
//   * the running max is only raised when it grows by more than 2^8 (the
//     result is the same softmax; P stays <= 256, exact in fp16's range), so
//     the O accumulator is rarely rescaled
//   * RoPE: Q is rotated once when loaded, K once up front (fa_rope.hip)
#include "fa_common.hpp"
#include "fa_host.hpp"
#include "fa_internal.hpp"
#include "fa_prefill.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace rdna_amd {
namespace {

constexpr int kBN = 64;                 // keys per tile
constexpr float kRescaleThreshold = 8.0f; // log2 units

// ---------------------------------------------------------------------------
// Ping-pong prefill (D <= 128): 8 waves in two groups that alternate between
// an MFMA phase and a VALU phase, barrier to barrier, so every SIMD always has
// one wave feeding the matrix core while its partner runs the softmax:
//
//   group A:  M(0) V(0) M(1) V(1) ... M(n-1) V(n-1) M(n)  -
//   group B:  -    M(0) V(0) M(1) ...        M(n-1) V(n-1) M(n)
//
//   M(i): S(i) = K(i) Q^T and O += V(i-1)^T P(i-1)     (32 MFMAs at D=128)
//   V(i): online softmax of S(i) -> P(i), rescale of O, and staging of the
//         group's half of the next K/V tiles (registers -> LDS, HBM -> regs)
//
// K(i) and V(i-1) are read in global phases 2i and 2i+1 and live in LDS slot
// i % 2 and (i - 1) % 2.  Group A stages pair (K(i+1), V(i)) in its V(i)
// (phase 2i+1), group B stages pair (K(i+2), V(i+1)) in its V(i) (phase 2i+2);
// both write slots whose last readers finished before the preceding barrier.
// At D = 128 the tiles move by HBM -> LDS DMA instead (one 1 KB instruction
// per 4-row group): the loads' issue and the LDS stores left the softmax side,
// which is the longer one (0.4 % faster on causal GQA B4 Hq32 Hkv8 S4096 D128
// in same-box A/B runs, 16 fewer registers, 7.7 KB less LDS).  Group B issues
// K(i+2) at the start of its V(i) and awaits it at the end of its M(i+1), two
// phases of latency.  Group A issues V(i) at the start of its own V(i) and
// awaits it at the end of that phase: V(i-2)'s slot was last read in phase
// 2i-1, and V(i) is first read in phase 2i+2.  Each group's softmax side then
// carries four DMAs per wave per tile instead of zero and eight (-0.8 % on the
// causal GQA shape above, -1.1 % on causal GQA B2 Hq32 Hkv8 S8192 D128).
// ---------------------------------------------------------------------------
constexpr int kPPWaves = 8;
constexpr int kOpDepth = 4; // MFMA operands in flight in the MFMA phase
constexpr int kPPThreads = 64 * kPPWaves;

template <int D>
struct PPCfg {
    // LDS row strides (64 banks x 4 B): K rows are read 16 at a time with
    // ds_read_b128 -> a 16 B step mod 256 B keeps them in distinct banks; V rows
    // are read 4 at a time, 64 B each, by the transpose read -> a 64 B step
    static constexpr int LDK = D + 8;
    static constexpr int LDV = D + 32;
    // D = 128: K/V tiles staged by HBM -> LDS DMA, one instruction per 4-row
    // group (1 KB).  Row 4j + b of a tile sits at byte 256 b of group j, its
    // 16-byte chunk c at position c ^ 4b; groups lie PSK (PSV) halves apart,
    // 16 (64) bytes more than 1 KB.  The 16-row b128 K reads then hit 16
    // distinct 16-byte bank groups (group j at 16 j mod 256, row b's chunk
    // moved by 64 b), and the 8-row transpose reads of V fall twice on each
    // 64-byte quarter (group j at 64 j, row b's chunk quad moved by b).
    static constexpr bool DMA = D == 128;
    static constexpr int PSK = 520;
    static constexpr int PSV = 544;
    static constexpr int TILE_K = DMA ? (kBN / 4) * PSK : kBN * LDK;
    static constexpr int TILE_V = DMA ? (kBN / 4) * PSV : kBN * LDV;
    static constexpr int NS = D / 16;
    static constexpr int NDT = D / 32;
    static constexpr int KCH = D / 8;
    static constexpr int HALF_TASK = 32 * KCH;         // one group's chunks of one K (or V) tile
    static constexpr int CT = (HALF_TASK + 255) / 256; // K (and V) chunks per thread
    // Q of the row tile, RoPE applied: [wave][32 rows][LDQ], read like K rows
    static constexpr int LDQ = D + 8;
    static constexpr int TILE_Q = kPPWaves * 32 * LDQ;
    static constexpr int QCT = kPPWaves * 32 * KCH / kPPThreads; // Q chunks per thread (= NS)
    // One resident workgroup per CU from D = 64 up (VGPRs): a persistent grid
    // then saves the workgroup switches and balances the row tiles. At D = 32
    // two workgroups share a CU and hide each other's prologue instead, which
    // the persistent loop's extra registers would prevent.
    static constexpr bool PERSIST = D >= 64;
};

// PRE (used when c = |scale| log2(e) <= 1, which covers 1/sqrt(D) for every
// head dim): Q is staged pre-multiplied by q_sign * c, so the QK^T MFMAs
// produce scores in log2 units, and each S^T accumulator chain starts from
// -m (m the lane's running max, 0 while no key is visible) instead of 0, so
// the MFMA output is the exponent itself: p = 2^acc with no per-score
// multiply-add.  The accumulators are shifted only when the running max
// moves.  Without PRE, Q carries only the sign and p = 2^(acc c - m).
template <int D, bool PRE>
__global__ __launch_bounds__(kPPThreads, 1) void fa_fwd_f16_pp(PrefillParams p) {
    using C = PPCfg<D>;
    // sK[slot], sV[slot], sQ
    __shared__ __attribute__((aligned(16))) _Float16 smem[2 * C::TILE_K + 2 * C::TILE_V + C::TILE_Q];
    _Float16* const sKs = smem;
    _Float16* const sVs = smem + 2 * C::TILE_K;
    _Float16* const sQ = smem + 2 * C::TILE_K + 2 * C::TILE_V;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const int grp = wave >> 2;       // 0 = group A, 1 = group B
    const int gtid = tid & 255;      // thread index inside the group

    // ---- staging: this group's half (rows 32*grp .. +31) of K(x) and V(x-1)
    uint32_t coff_k[C::CT], coff_v[C::CT];
    int clk[C::CT], clv[C::CT]; // LDS element offsets inside a tile, -1 = no chunk
#pragma unroll
    for (int it = 0; it < C::CT; it++) {
        const int e = gtid + it * 256;
        const bool ok = C::HALF_TASK % 256 == 0 || e < C::HALF_TASK;
        const int row = 32 * grp + (ok ? e / C::KCH : 0);
        const int ch = ok ? e - (e / C::KCH) * C::KCH : 0;
        coff_k[it] = (uint32_t)(((int64_t)row * p.k_ss + 8 * ch) * 2);
        coff_v[it] = (uint32_t)(((int64_t)row * p.v_ss + 8 * ch) * 2);
        clk[it] = ok ? row * C::LDK + 8 * ch : -1;
        clv[it] = ok ? row * C::LDV + 8 * ch : -1;
    }
    // DMA staging (PPCfg::DMA): wave w of group B (K) or A (V) moves 4-row
    // groups 4w .. 4w + 3 of each tile, lane i global chunk (i % 16) ^ 4 (i /
    // 16) of row 4j + i / 16 to LDS byte 16 i of group j; the group's row
    // offset is the instruction's scalar offset, its LDS address M0.
    const uint32_t dma_j0 = (uint32_t)__builtin_amdgcn_readfirstlane((wave & 3) * 4);
    const uint32_t dma_c = (uint32_t)((lane & 15) ^ (4 * (lane >> 4)));
    const uint32_t dma_vk = (uint32_t)(lane >> 4) * (uint32_t)(p.k_ss * 2) + 16u * dma_c;
    const uint32_t dma_vv = (uint32_t)(lane >> 4) * (uint32_t)(p.v_ss * 2) + 16u * dma_c;
    const uint32_t lds_k = (uint32_t)reinterpret_cast<uintptr_t>(sKs);
    const uint32_t lds_v = (uint32_t)reinterpret_cast<uintptr_t>(sVs);
    // Persistent (PPCfg::PERSIST): this workgroup walks its share of the row
    // tiles (one per workgroup of a one-tile-per-workgroup grid, see
    // persistent_item). Every group passes the same barriers per item and
    // leaves an item only after its last LDS read, so the next item's
    // prologue may overwrite LDS. Otherwise the grid has one workgroup per
    // row tile.
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

        const _Float16* qbase = p.q + b * p.q_sb + h * p.q_sh;
        const _Float16* kbase = p.k + b * p.k_sb + kvh * p.k_sh;
        const _Float16* vbase = p.v + b * p.v_sb + kvh * p.v_sh;
        _Float16* obase = p.o + b * p.o_sb + h * p.o_sh;

        // Q^T operand (lane holds Q[q][16s + 8g .. +7], RoPE applied), staged
        // through sQ: in the operand layout each lane reads 16 B of its own row,
        // so every load instruction touches 32 rows (cache lines) and the
        // prologue waited on L1 lookups. All threads instead load the tile's Q
        // (and RoPE table) chunks row-contiguously, 16 lanes per 256 B, rotate
        // them and write sQ; after the prologue barrier each wave reads its
        // operand from sQ with conflict-free b128 reads (the K-row layout).
        h8 qreg[C::NS];
        auto stage_q = [&]() {
            const _Float16* qb = p.q + b * p.q_sb + (int64_t)(kvh * p.ratio + sub * p.G) * p.q_sh;
            // chunk c of this thread: (head j, row r, 16-byte column ch), ch
            // fastest; row r of head j is row r % 32 of wave j + G * (r / 32).
            // A tile holds rows_per_wg = 256 / G rows of each of G heads, G in
            // {1, 2, 4}: head and row are a shift and a mask of the slot row
            // (a division by rows_per_wg cost ~30 instructions per chunk).
            // Recomputed from an opaque copy of the thread id at each use so
            // that no index stays live across the loads' latency.
            const uint32_t rsh = 8u - (uint32_t)(p.G >> 1); // log2 rows_per_wg
            struct Chunk {
                uint32_t j, r, ch;
            };
            auto chunk = [&](uint32_t t, int c) {
                const uint32_t idx = t + kPPThreads * c;
                const uint32_t rj = idx / C::KCH;
                return Chunk{rj >> rsh, rj & ((1u << rsh) - 1u), idx - rj * C::KCH};
            };
            auto src_row = [&](const Chunk& k) { return wg_q0 + (int)k.r < p.Sq ? (uint32_t)wg_q0 + k.r : 0u; };
            h8 x[C::QCT];
            f4 cs[C::QCT], sn[C::QCT];
            uint32_t t = tid;
            asm volatile("" : "+v"(t));
            // The table loads are issued first, so that they and the Q loads
            // are in flight together: issued after the Q loads, they waited
            // for all of them (the conversions that both the rotation and the
            // plain scaling start with were hoisted above the branch).
            if (p.rope_q) {
#pragma unroll
                for (int c = 0; c < C::QCT; c++) {
                    const Chunk k = chunk(t, c);
                    const uint64_t off = (uint64_t)src_row(k) * (D / 2) + 4 * k.ch;
                    cs[c] = *reinterpret_cast<const f4*>(p.rot_cos + off);
                    sn[c] = *reinterpret_cast<const f4*>(p.rot_sin + off);
                }
            }
#pragma unroll
            for (int c = 0; c < C::QCT; c++) {
                const Chunk k = chunk(t, c);
                x[c] = *reinterpret_cast<const h8*>(qb + (int64_t)k.j * p.q_sh + (int64_t)src_row(k) * p.q_ss +
                                                    8 * k.ch);
            }
            if (p.rope_q) {
#pragma unroll
                for (int c = 0; c < C::QCT; c++) {
                    x[c] = PRE ? rope8_cs_mul(x[c], cs[c], sn[c], p.qmul) : rope8_cs(x[c], cs[c], sn[c]);
                }
            } else if constexpr (PRE) {
#pragma unroll
                for (int c = 0; c < C::QCT; c++) {
                    x[c] = scale8(x[c], p.qmul);
                }
            }
            const bool neg = !PRE && p.q_sign < 0.0f; // PRE: the sign is in qmul
            asm volatile("" : "+v"(t));
#pragma unroll
            for (int c = 0; c < C::QCT; c++) {
                const Chunk k = chunk(t, c);
                const uint32_t dst = ((k.j + p.G * (k.r >> 5)) * 32 + (k.r & 31)) * C::LDQ + 8 * k.ch;
                *reinterpret_cast<h8*>(&sQ[dst]) = wg_q0 + (int)k.r < p.Sq ? (neg ? -x[c] : x[c]) : h8{};
            }
        };
        auto read_q = [&]() {
            const _Float16* src = sQ + (wave * 32 + l32) * C::LDQ + 8 * g;
#pragma unroll
            for (int st = 0; st < C::NS; st++) {
                qreg[st] = *reinterpret_cast<const h8*>(src + 16 * st);
            }
        };

        const int wg_q_hi = min(wg_q0 + p.rows_per_wg, p.Sq) - 1;
        int klo, khi;
        visible_key_range(p.mask, wg_q0, wg_q_hi, klo, khi);
        int t_begin = 0, n = 0;
        if (khi >= klo) {
            t_begin = klo / kBN;
            n = khi / kBN + 1 - t_begin;
        }
        const int Sk = p.mask.sk;
        const uint32_t k_row_b = (uint32_t)(p.k_ss * 2), v_row_b = (uint32_t)(p.v_ss * 2);
        int row_lo, row_hi;
        row_key_bounds(p.mask, q, row_lo, row_hi);
        // class of key tile t_begin + i for this wave's rows (0 skip, 1 no mask, 2 masked)
        const TileClasses tcls = wave_active ? tile_classes<kBN>(p.mask, q0, q_hi) : TileClasses{1, 0, 1, 0};

        f16x oacc[C::NDT];
#pragma unroll
        for (int dt = 0; dt < C::NDT; dt++) {
            oacc[dt] = f16x{};
        }
        float m_run = -INFINITY;
        float m_use = 0.0f; // m_run, or 0 while it is -inf (PRE: the S^T accumulators start at -m_use)
        f16x minit = f16x{};
        float l_run = 0.0f;
        f16x sacc[2];
        sacc[0] = f16x{};
        sacc[1] = f16x{};
        h8 pb[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            pb[u] = h8{};
        }
        int cls_prev = 0; // classification of the tile whose P is held in pb

        h8 kreg[C::CT], vreg[C::CT];
        // registers <- HBM for pair x (K tile x if x < n, V tile x-1 if 1 <= x <= n);
        // a missing tile gets num_records 0, so its loads return 0 and touch nothing.
        // A tile spans at most kBN rows at a seq stride <= 2^24 elements, so its
        // byte range fits 32 bits (tile_bytes); this keeps the per-tile
        // descriptor set-up to a few scalar instructions.
        // Each group calls load_pair with x = 0, 1, 2, ... in order, so the tile
        // addresses advance by one tile stride per call (unsigned arithmetic:
        // V tile -1 of the first call is never read, its num_records is 0).
        uint64_t k_addr = reinterpret_cast<uint64_t>(kbase) + (uint64_t)((int64_t)t_begin * kBN * p.k_ss * 2);
        uint64_t v_addr = reinterpret_cast<uint64_t>(vbase) + (uint64_t)((int64_t)(t_begin - 1) * kBN * p.v_ss * 2);
        const uint64_t k_step = (uint64_t)(kBN * p.k_ss * 2), v_step = (uint64_t)(kBN * p.v_ss * 2);
        auto load_pair = [&](int x) {
            const int tk = t_begin + x, tv = t_begin + x - 1;
            const auto rk = make_rsrc(reinterpret_cast<const void*>(k_addr),
                                      x < n ? tile_bytes<kBN>(Sk - tk * kBN, k_row_b, D * 2) : 0u);
            const auto rv = make_rsrc(reinterpret_cast<const void*>(v_addr),
                                      (x >= 1 && x <= n) ? tile_bytes<kBN>(Sk - tv * kBN, v_row_b, D * 2) : 0u);
            k_addr += k_step;
            v_addr += v_step;
#pragma unroll
            for (int it = 0; it < C::CT; it++) {
                kreg[it] = buffer_load_h8(rk, coff_k[it], 0);
                vreg[it] = buffer_load_h8(rv, coff_v[it], 0);
            }
        };
        // LDS <- registers for pair x.  Written whether or not the tiles exist:
        // a missing tile was loaded as zeros into a slot that no phase reads
        // (K(x) for x >= n, V(x - 1) for x < 1 or x > n), and every slot is
        // written on the same schedule as for an existing tile, after the last
        // read of its previous contents.  No branches in the VALU phase.
        auto store_pair = [&](int x) {
            _Float16* sK = sKs + (x & 1) * C::TILE_K;
            _Float16* sV = sVs + ((x - 1) & 1) * C::TILE_V;
#pragma unroll
            for (int it = 0; it < C::CT; it++) {
                if (C::HALF_TASK % 256 == 0 || clk[it] >= 0) {
                    *reinterpret_cast<h8*>(&sK[clk[it]]) = kreg[it];
                    *reinterpret_cast<h8*>(&sV[clv[it]]) = vreg[it];
                }
            }
        };

        // DMA staging: each group sets up pair x = 0, 1, 2, ... in order (the
        // same address stepping as load_pair) and issues its half of the 8
        // DMAs: K group dma_j0 + k / 2 for even k (group B), V group dma_j0 +
        // k / 2 for odd k (group A).
        struct DmaPair {
            i32x4_t rk, rv;
            uint32_t mk, mv;
        };
        auto uniform = [](i32x4_t r) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                r[e] = __builtin_amdgcn_readfirstlane(r[e]);
            }
            return r;
        };
        auto dma_pair = [&](int x) {
            const int tk = t_begin + x, tv = t_begin + x - 1;
            DmaPair d;
            d.rk = uniform(make_rsrc_v(reinterpret_cast<const void*>(k_addr),
                                       x < n ? tile_bytes<kBN>(Sk - tk * kBN, k_row_b, D * 2) : 0u));
            d.rv = uniform(make_rsrc_v(reinterpret_cast<const void*>(v_addr),
                                       (x >= 1 && x <= n) ? tile_bytes<kBN>(Sk - tv * kBN, v_row_b, D * 2) : 0u));
            d.mk = (uint32_t)__builtin_amdgcn_readfirstlane(
                (int)(lds_k + (uint32_t)(((x & 1) * C::TILE_K + (int)dma_j0 * C::PSK) * 2)));
            d.mv = (uint32_t)__builtin_amdgcn_readfirstlane(
                (int)(lds_v + (uint32_t)((((x - 1) & 1) * C::TILE_V + (int)dma_j0 * C::PSV) * 2)));
            k_addr += k_step;
            v_addr += v_step;
            return d;
        };
        auto dma_issue = [&](const DmaPair& d, int k) {
            const uint32_t j = dma_j0 + (uint32_t)(k >> 1);
            const uint32_t so = (uint32_t)__builtin_amdgcn_readfirstlane((int)(4u * j * ((k & 1) ? v_row_b : k_row_b)));
            if (k & 1) {
                dma_load16_s(d.rv, dma_vv, so, d.mv + (uint32_t)((k >> 1) * C::PSV * 2));
            } else {
                dma_load16_s(d.rk, dma_vk, so, d.mk + (uint32_t)((k >> 1) * C::PSK * 2));
            }
        };

        // M(i): O += V(i-1)^T P(i-1) (i >= 1) then S(i) = K(i) Q^T (i < n), as one
        // stream of MFMAs whose LDS operands are read kOpDepth MFMAs ahead through
        // a small register ring; sched_barrier stops the compiler from hoisting
        // every read (which would need ~100 more VGPRs).
        auto mfma_stream = [&](auto do_pv_c, auto do_s_c, int i) {
            // The MFMA phase runs at raised wave priority: each SIMD also holds
            // the other group's wave in its softmax phase, whose VALU stream
            // otherwise delays the issue of the next MFMA (-1.2 % on causal GQA
            // B4 Hq32 Hkv8 S4096 D128 with RoPE and on B2 Hq32 Hkv8 S8192 D128 in
            // same-box A/B runs; the INT8 head_dim 128 kernel, whose softmax
            // side is its critical path, measured slower with it)
            __builtin_amdgcn_s_setprio(1);
            constexpr bool DO_PV = decltype(do_pv_c)::value;
            constexpr bool DO_S = decltype(do_s_c)::value;
            constexpr int NPV = DO_PV ? 4 * C::NDT : 0; // (u, dt)
            constexpr int NSK = DO_S ? 2 * C::NS : 0;   // (s, kt)
            constexpr int T = NPV + NSK;
            constexpr int DEPTH = T < kOpDepth ? T : kOpDepth;
            const int j16 = lane & 15;
            const _Float16* vrow = sVs + ((i - 1) & 1) * C::TILE_V + (4 * g + (j16 >> 2)) * C::LDV +
                                   16 * ((lane >> 4) & 1) + 4 * (j16 & 3);
            const _Float16* krow = sKs + (i & 1) * C::TILE_K + l32 * C::LDK + 8 * g;
            // DMA layout: K row l32 (+32 kt) is row b = l32 % 4 of group l32 / 4
            // (+8 kt), its chunk 2 st + g at position 2 (st ^ 2b) + g, i.e. at
            // 16 (st % 2) + 32 ((st / 2) ^ b) halves: one base per st / 2.  V
            // row 16u + 8h + 4g + j16 / 4 is row b = j16 / 4 of group 4u + 2h + g,
            // its columns 32 dt + 16 x + 4 (j16 % 4) at chunk quad dt ^ b: one
            // base per dt.
            const _Float16* kb[C::DMA ? 4 : 1];
            const _Float16* vb[C::DMA ? C::NDT : 1];
            if constexpr (C::DMA) {
                const int bk = l32 & 3, bv = (j16 >> 2) & 3;
                const _Float16* k0 = sKs + (i & 1) * C::TILE_K + (l32 >> 2) * C::PSK + 128 * bk + 8 * g;
                const _Float16* v0 = sVs + ((i - 1) & 1) * C::TILE_V + g * C::PSV + 128 * bv +
                                     16 * ((lane >> 4) & 1) + 4 * (j16 & 3);
#pragma unroll
                for (int s2 = 0; s2 < 4; s2++) {
                    kb[s2] = k0 + 32 * (s2 ^ bk);
                }
#pragma unroll
                for (int dt = 0; dt < C::NDT; dt++) {
                    vb[dt] = v0 + 32 * (dt ^ bv);
                }
            }
            auto op = [&](int j) -> h8 {
                if (j < NPV) {
                    const int u = j / C::NDT, dt = j % C::NDT;
                    if constexpr (C::DMA) {
                        const _Float16* base = vb[dt] + (4 * u) * C::PSV;
                        h4 lo = lds_read_tr16(base);
                        h4 hi = lds_read_tr16(base + 2 * C::PSV);
                        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                    }
                    const _Float16* base = vrow + (16 * u) * C::LDV + 32 * dt;
                    h4 lo = lds_read_tr16(base);
                    h4 hi = lds_read_tr16(base + 8 * C::LDV);
                    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                }
                const int js = j - NPV, st = js >> 1, kt = js & 1;
                if constexpr (C::DMA) {
                    return *reinterpret_cast<const h8*>(kb[st >> 1] + kt * 8 * C::PSK + 16 * (st & 1));
                }
                return *reinterpret_cast<const h8*>(krow + kt * 32 * C::LDK + 16 * st);
            };
            f16x acc0 = {}, acc1 = {};
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
                if (j < NPV) {
                    const int u = j / C::NDT, dt = j % C::NDT;
                    oacc[dt] = mfma_32x32x16_f16(a, pb[u], oacc[dt]);
                } else {
                    const int js = j - NPV, st = js >> 1;
                    if (js & 1) {
                        acc1 = mfma_32x32x16_f16(a, qreg[st], (PRE && st == 0) ? minit : acc1);
                    } else {
                        acc0 = mfma_32x32x16_f16(a, qreg[st], (PRE && st == 0) ? minit : acc0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_s_setprio(0);
            if constexpr (DO_S) {
                sacc[0] = acc0;
                sacc[1] = acc1;
            }
        };
        auto phase_m = [&](int i) {
            if (!wave_active) {
                return;
            }
            const bool do_pv = i >= 1 && cls_prev != 0;
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

        // V(i): softmax of S(i) -> pb, rescale O
        auto phase_v = [&](int i) {
            if (!wave_active || cls_prev == 0) {
                return;
            }
            if (cls_prev == 2) {
                const int kt0 = (t_begin + i) * kBN;
                const int a = row_lo - kt0 - 4 * g;
                const int bnd = row_hi - kt0 - 4 * g;
#pragma unroll
                for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int off = kt * 32 + 8 * (e >> 2) + (e & 3);
                        sacc[kt][e] = (off < a || off > bnd) ? -INFINITY : sacc[kt][e];
                    }
                }
            }
            float mx = max_tree<32>([&](int e) { return sacc[e >> 4][e & 15]; });
            mx = pair_max(mx);
            // PRE: sacc = S c - m_use already; otherwise S
            const float m_new = PRE ? fmaxf(m_run, mx + m_use) : fmaxf(m_run, mx * p.c);
            const bool grow = m_new > m_run + kRescaleThreshold;
            if (wave_any(grow)) {
                const float alpha = grow ? fast_exp2(m_run - m_new) : 1.0f;
                if (grow) {
                    m_run = m_new;
                }
                l_run *= alpha;
#pragma unroll
                for (int dt = 0; dt < C::NDT; dt++) {
                    oacc[dt] *= alpha;
                }
                const float m_use_new = (m_run == -INFINITY) ? 0.0f : m_run;
                if constexpr (PRE) {
                    // re-base this tile's exponents and the next tiles' start
                    const float shift = m_use - m_use_new;
#pragma unroll
                    for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                        for (int e = 0; e < 16; e++) {
                            sacc[kt][e] += shift;
                        }
                    }
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        minit[e] = -m_use_new;
                    }
                }
                m_use = m_use_new;
            }
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const float x = PRE ? sacc[kt][e] : fmaf(sacc[kt][e], p.c, -m_use);
                    pb[kt * 2 + (e >> 3)][e & 7] = (_Float16)fast_exp2(x);
                }
            }
            l_run = sum_h8x4(pb, l_run);
        };

        // ---- prologue: pair 0 in LDS; each group's registers hold its next pair
        // (DMA: group B's K(0) in flight while Q stages)
        const bool dma_wave = __builtin_amdgcn_readfirstlane(grp) == 1;
        if constexpr (C::DMA) {
            if (dma_wave && n > 0) {
                const DmaPair d0 = dma_pair(0);
#pragma unroll
                for (int k = 0; k < 8; k += 2) {
                    dma_issue(d0, k);
                }
            }
        } else if (n > 0) {
            load_pair(0);
        }
        stage_q();
        if constexpr (C::DMA) {
            if (dma_wave) {
                __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); // K(0) landed (not tracked by the compiler)
            }
        } else if (n > 0) {
            store_pair(0);
            load_pair(1);
        }
        __syncthreads();
        read_q();
        // Both groups pass 2n + 2 barriers; group B starts one phase late.
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
                        // V(i) into V(i - 2)'s slot, last read in phase 2i - 1;
                        // first read in phase 2i + 2
                        const DmaPair d = dma_pair(i + 1);
#pragma unroll
                        for (int k = 1; k < 8; k += 2) {
                            dma_issue(d, k);
                        }
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
                // DMA: group B issues K(i + 2) at the start of its V(i) and
                // waits for it at the end of its M(i + 1); K(1) in phase 0
                if constexpr (C::DMA) {
                    if (1 < n) {
                        const DmaPair d1 = dma_pair(1);
#pragma unroll
                        for (int k = 0; k < 8; k += 2) {
                            dma_issue(d1, k);
                        }
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
                            const DmaPair d = dma_pair(i + 2);
#pragma unroll
                            for (int k = 0; k < 8; k += 2) {
                                dma_issue(d, k);
                            }
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

        // O = O^T / l, through this wave's sQ slot (free since read_q)
        if (wave_active) {
            const float l = pair_sum(l_run);
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            store_o_tile<D, C::LDQ>(oacc, [&](int) { return f4{inv, inv, inv, inv}; }, sQ + wave * 32 * C::LDQ,
                                    obase, q0, p.Sq, p.o_ss, lane);
        }
        if constexpr (C::PERSIST) {
            __syncthreads(); // the next row tile's Q staging writes every wave's slot
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
int launch_pp_as(const PrefillParams& p, int64_t n_wg, hipStream_t stream, std::string& err) {
    // persistent: as many workgroups as the device holds at once, each
    // walking its share of the n_wg row tiles
    int64_t grid = n_wg;
    if (PPCfg<D>::PERSIST) {
        const int64_t resident =
            resident_workgroups(reinterpret_cast<const void*>(&fa_fwd_f16_pp<D, PRE>), kPPThreads, err);
        if (resident <= 0) {
            return -1;
        }
        grid = std::min(n_wg, resident);
    }
    KernelTimerGuard timer(stream);
    hipLaunchKernelGGL((fa_fwd_f16_pp<D, PRE>), dim3((uint32_t)grid), dim3(kPPThreads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

// Q pre-scaled into log2 units needs |q| c representable in fp16: c <= 1
// keeps |q c| <= |q|.  Not at D = 32, where the 16 registers of the start
// block would leave room for 3 waves per SIMD, not the 4 that let two
// workgroups share a compute unit.
template <int D>
int launch_pp(const PrefillParams& p, int64_t n_wg, hipStream_t stream, std::string& err) {
    if (D >= 64 && p.c <= 1.0f) {
        return launch_pp_as<D, D >= 64>(p, n_wg, stream, err);
    }
    return launch_pp_as<D, false>(p, n_wg, stream, err);
}

} // namespace

constexpr int64_t kMaxSeqStride = 1 << 24;

int xcd_head_group_chunk(int n_head_groups, int64_t kv_bytes) {
    constexpr int kXcds = 8;
    constexpr int64_t kL2Budget = 3 << 20; // of the 4 MB L2 per XCD
    if (n_head_groups % kXcds != 0 || kv_bytes <= 0) {
        return 0;
    }
    const int per_xcd = n_head_groups / kXcds;
    int c = (int)std::max<int64_t>(1, std::min<int64_t>(per_xcd, kL2Budget / kv_bytes));
    while (per_xcd % c != 0) {
        c--;
    }
    return c;
}

float softmax_log2_scale(float scale) {
    return std::max(std::fabs(scale) * kLog2e, 1e-30f);
}

int fwd_f16_prefill(const AttnArgs& a, bool rope_q, hipStream_t stream, std::string& err) {
    PrefillParams p{};
    p.q = static_cast<const _Float16*>(a.q);
    p.k = static_cast<const _Float16*>(a.k);
    p.v = static_cast<const _Float16*>(a.v);
    p.o = static_cast<_Float16*>(a.o);
    p.rot_cos = a.rot_cos;
    p.rot_sin = a.rot_sin;
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
    p.Sq = a.Sq;
    p.Hkv = a.Hkv;
    p.ratio = a.Hq / a.Hkv;
    const bool kpair = a.D > 128 && a.D <= 256;
    const bool dpair = a.D > 256;
    // every kernel holds G query heads of one kv head (G | Hq/Hkv, G <= 4)
    // and 128 (query, head) rows per workgroup: 8 waves of 32 rows (D <= 128)
    // or 4 pairs of waves of 32 rows (D > 128)
    p.G = (p.ratio % 4 == 0) ? 4 : ((p.ratio % 2 == 0) ? 2 : 1);
    p.rows_per_wg = (kpair ? kKPairRows : dpair ? kDPairRows : 32 * kPPWaves) / p.G;
    p.n_row_tiles = (a.Sq + p.rows_per_wg - 1) / p.rows_per_wg;
    p.groups_per_kv = p.ratio / p.G;
    p.n_head_groups = a.B * a.Hkv * p.groups_per_kv;
    p.hg_chunk = xcd_head_group_chunk(p.n_head_groups, 2 * (int64_t)a.Sk * a.D * (int64_t)sizeof(_Float16));
    p.c = softmax_log2_scale(a.scale);
    p.q_sign = a.scale < 0.0f ? -1.0f : 1.0f;
    p.qmul = p.q_sign * p.c;
    p.mask = MaskSpec{a.Sk, a.Sk - a.Sq, a.causal ? 1 : 0, a.window > 0 ? a.window : 0};
    p.rope_q = rope_q ? 1 : 0;

    const int64_t n_wg = (int64_t)p.n_row_tiles * p.n_head_groups;
    p.n_items = (int32_t)std::min<int64_t>(n_wg, INT32_MAX);
    if (n_wg <= 0) {
        err = "empty launch grid";
        return -1;
    }
    if (n_wg > INT32_MAX) {
        err = "launch grid too large";
        return -1;
    }
    switch (a.D) {
    case 32: return launch_pp<32>(p, n_wg, stream, err);
    case 64: return launch_pp<64>(p, n_wg, stream, err);
    case 96: return launch_pp<96>(p, n_wg, stream, err);
    case 128: return launch_pp<128>(p, n_wg, stream, err);
    default: break;
    }
    if (kpair) {
        return launch_kpair(p, (int)a.D, n_wg, stream, err);
    }
    if (dpair) {
        return launch_dpair(p, (int)a.D, n_wg, stream, err);
    }
    err = "unsupported head_dim (multiples of 32 from 32 to 512)";
    return -1;
}

bool splitk_supported(const AttnArgs& a);

// Auto: few query rows per kv head against a long key sequence -> split-K
// (HBM-bound, parallel over the key axis); everything else -> prefill tiles.
bool prefer_splitk(const AttnArgs& a) {
    return splitk_supported(a) && a.Sk >= 512;
}

int64_t fwd_f16_scratch_bytes(const AttnArgs& a, F16Path path, std::string& err) {
    const bool splitk = path == F16Path::SplitK || (path == F16Path::Auto && prefer_splitk(a));
    size_t bytes = 0;
    if (a.has_rope && a.Sk > 0) {
        bytes += region_bytes((size_t)a.B * a.Hkv * a.Sk * a.D * sizeof(_Float16));
    }
    if (splitk && splitk_supported(a)) {
        int splits = 0, kps = 0;
        if (splitk_plan(a, splits, kps, err) != 0) {
            return -1;
        }
        bytes += region_bytes(splitk_partial_bytes(a, splits));
    }
    return (int64_t)bytes;
}

int fwd_f16(const AttnArgs& in, F16Path path, hipStream_t stream, std::string& err, ScratchRegion* region) {
    AttnArgs a = in;
    // K/V rows are addressed with 32-bit byte offsets inside a 64-key tile
    if (a.ks[2] < 0 || a.vs[2] < 0 || a.ks[2] > kMaxSeqStride || a.vs[2] > kMaxSeqStride) {
        err = "key/value seq strides must be in [0, 2^24] elements";
        return -1;
    }
    const bool splitk = path == F16Path::SplitK || (path == F16Path::Auto && prefer_splitk(a));
    StreamScratch krot(ScratchUse::RotatedK, region);
    if (a.has_rope && a.Sk > 0) {
        const size_t bytes = (size_t)a.B * a.Hkv * a.Sk * a.D * sizeof(_Float16);
        if (krot.alloc(bytes, stream, err) != 0 || rope_rotate_k(a, krot.ptr, stream, err) != 0) {
            return -1;
        }
        a.k = krot.ptr;
        a.ks[0] = (int64_t)a.Hkv * a.Sk * a.D;
        a.ks[1] = (int64_t)a.Sk * a.D;
        a.ks[2] = a.D;
    }
    return splitk ? fwd_f16_splitk(a, a.has_rope != 0, stream, err, region)
                  : fwd_f16_prefill(a, a.has_rope != 0, stream, err);
}

} // namespace rdna_amd
