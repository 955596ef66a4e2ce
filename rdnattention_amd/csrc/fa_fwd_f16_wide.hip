// FP16 prefill for large heads (head_dim 288..352, multiples of 32) on gfx950.
//
// Covers head dims the reference dispatches through its tile planner
// (src/rdna/fa2_forward_f16.hip:1045-1066, chooseTile :923-954) with the same
// results as the smaller-head kernels (fa_fwd_f16.hip); only the data
// movement changes, because such a row tile no longer fits the
// register-staged, 64-key design:
//
//   * one workgroup = 4 waves (one per SIMD); each wave owns 32 query rows of
//     one head, with Q^T in VGPRs (D/4 per lane) and all D columns of O^T in
//     the accumulator registers; G heads of one kv head share the workgroup
//   * K and V tiles of 32 keys go HBM -> LDS with buffer_load ... lds, one DMA
//     instruction per row (D/8 lanes x 16 B), so rows land at a padded stride
//     with no VGPR staging; LDS is double-buffered and tile t+1 is in flight
//     while tile t is computed
//   * K rows at stride D+8 halves and V rows at a stride = 32 (mod 128)
//     halves keep the 16-row ds_read_b128 of K and the 4-row transpose reads
//     of V on distinct banks for every head dim
//   * S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_32x32x16_f16, lane-local
//     softmax rows, P^T straight from the S accumulator, lazy rescale (2^8);
//     one code path for full and boundary tiles (the mask is 16 selects
//     against 64+ MFMAs per tile)
//
// Head dims 384..512 run fa_fwd_f16_dpair.hip, whose wave pairs split the
// head dimension so that two waves fit on every SIMD.
#include "fa_common.hpp"
#include "fa_host.hpp"
#include "fa_internal.hpp"
#include "fa_prefill.hpp"

namespace rdna_amd {
namespace {

constexpr int kWideWaves = 4;
constexpr int kWideThreads = 64 * kWideWaves;
constexpr int kWideBN = 32;                   // keys per tile
constexpr float kWideRescaleThreshold = 8.0f; // log2 units
constexpr int kWideOpDepth = 4;                // MFMA operands in flight

template <int D>
struct WideCfg {
    static_assert(D % 32 == 0 && D >= 32 && D <= 512, "head_dim");
    static constexpr int DV = D;                                   // output columns of a wave
    static constexpr int LDK = D + 8;                              // halves
    static constexpr int LDV = DV + ((32 - DV % 128) + 128) % 128; // halves, = 32 (mod 128)
    static constexpr int TILE_K_BYTES = kWideBN * LDK * 2;
    static constexpr int TILE_V_BYTES = kWideBN * LDV * 2;
    static constexpr int BUF_BYTES = TILE_K_BYTES + TILE_V_BYTES;
    static constexpr int NS = D / 16;   // QK^T reduction steps
    static constexpr int NDT = DV / 32; // O^T row tiles per pass
    static constexpr int KCH = D / 8;   // 16-byte chunks per K row = active DMA lanes
    static constexpr int VCH = DV / 8;  // 16-byte chunks per V row slice
    static constexpr int ROWS_PER_WAVE = kWideBN / kWideWaves;
    static_assert(KCH <= 64, "one DMA instruction per row");
    static_assert(LDV % 128 == 32 && LDV >= DV, "V stride");
    static_assert(2 * BUF_BYTES <= 160 * 1024, "LDS");
};

// Online-softmax bookkeeping shared by the large-head kernels.  PRE: Q holds
// q * scale * log2(e) and each S^T chain started at minit = -m_use (m_run, or
// 0 while it is -inf), so the accumulators are already the exponents; a
// rescale re-bases them and minit.  Returns P^T (fp16) and adds its row sum to
// l_run.
template <bool PRE, int NDT>
__device__ __forceinline__ void wide_softmax(f16x& sacc, f16x (&oacc)[NDT], float& m_run, float& m_use, f16x& minit,
                                             float& l_run, float c, h8 (&pb)[2]) {
    float mx = sacc[0];
#pragma unroll
    for (int i = 1; i < 16; i++) {
        mx = fmaxf(mx, sacc[i]);
    }
    mx = pair_max(mx);
    const float m_new = PRE ? fmaxf(m_run, mx + m_use) : fmaxf(m_run, mx * c); // c > 0: -inf stays -inf
    const bool grow = m_new > m_run + kWideRescaleThreshold;
    if (wave_any(grow)) {
        const float alpha = grow ? fast_exp2(m_run - m_new) : 1.0f; // m_run = -inf -> 0
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
            for (int i = 0; i < 16; i++) {
                sacc[i] += shift;
                minit[i] = -m_use_new;
            }
        }
        m_use = m_use_new;
    }
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        pb[i >> 3][i & 7] = (_Float16)fast_exp2(PRE ? sacc[i] : fmaf(sacc[i], c, -m_use));
    }
    psum = sum_h8(pb[1], sum_h8(pb[0], psum));
    l_run += psum;
}

template <int D, bool PRE>
__device__ __forceinline__ void wide_tile(const char* __restrict__ buf, const h8 (&qreg)[WideCfg<D>::NS],
                                          f16x (&oacc)[WideCfg<D>::NDT], float& m_run, float& m_use, f16x& minit,
                                          float& l_run, int row_lo, int row_hi, int kt0, float c, int lane) {
    using C = WideCfg<D>;
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const _Float16* sK = reinterpret_cast<const _Float16*>(buf);
    const _Float16* sV = reinterpret_cast<const _Float16*>(buf + C::TILE_K_BYTES);

    // S^T[key][query] over the 32-key tile; K operands stream through a
    // small register ring so the scheduler cannot hoist every LDS read
    f16x sacc = PRE ? minit : f16x{};
    const _Float16* krow = sK + l32 * C::LDK + 8 * g;
    {
        constexpr int DEPTH = kWideOpDepth < C::NS ? kWideOpDepth : C::NS;
        h8 ring[DEPTH];
#pragma unroll
        for (int j = 0; j < DEPTH; j++) {
            ring[j] = *reinterpret_cast<const h8*>(krow + 16 * j);
        }
#pragma unroll
        for (int s = 0; s < C::NS; s++) {
            const h8 a = ring[s % DEPTH];
            if (s + DEPTH < C::NS) {
                ring[s % DEPTH] = *reinterpret_cast<const h8*>(krow + 16 * (s + DEPTH));
            }
            sacc = mfma_32x32x16_f16(a, qreg[s], sacc);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    {
        // visible iff row_lo <= key <= row_hi, key = kt0 + 4g + off
        const int a = row_lo - kt0 - 4 * g;
        const int b = row_hi - kt0 - 4 * g;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int off = 8 * (i >> 2) + (i & 3);
            sacc[i] = (off < a || off > b) ? -INFINITY : sacc[i];
        }
    }
    h8 pb[2];
    wide_softmax<PRE>(sacc, oacc, m_run, m_use, minit, l_run, c, pb);

    // O^T += V^T P^T: pb[u] holds keys 16u + 4g + {0..3, 8..11}; the V^T
    // operand rows come from transpose reads of rows 16u + 8hh + 4g + j16/4
    const int j16 = lane & 15;
    const _Float16* vrow = sV + (4 * g + (j16 >> 2)) * C::LDV + 16 * ((lane >> 4) & 1) + 4 * (j16 & 3);
    auto vop = [&](int j) -> h8 {
        const int u = j / C::NDT, dt = j % C::NDT;
        const _Float16* base = vrow + (16 * u) * C::LDV + 32 * dt;
        h4 lo = lds_read_tr16(base);
        h4 hi = lds_read_tr16(base + 8 * C::LDV);
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    {
        constexpr int T = 2 * C::NDT;
        constexpr int DEPTH = kWideOpDepth < T ? kWideOpDepth : T;
        h8 ring[DEPTH];
#pragma unroll
        for (int j = 0; j < DEPTH; j++) {
            ring[j] = vop(j);
        }
#pragma unroll
        for (int j = 0; j < T; j++) {
            const h8 a = ring[j % DEPTH];
            if (j + DEPTH < T) {
                ring[j % DEPTH] = vop(j + DEPTH);
            }
            const int u = j / C::NDT, dt = j % C::NDT;
            oacc[dt] = mfma_32x32x16_f16(a, pb[u], oacc[dt]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

template <int D, bool PRE>
__global__ __launch_bounds__(kWideThreads, 1) void fa_fwd_f16_wide(PrefillParams p) {
    using C = WideCfg<D>;
    __shared__ __attribute__((aligned(16))) char wsm[2 * C::BUF_BYTES];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); // wave-uniform
    const int lane = tid & 63;
    const int l32 = lane & 31;
    const int g = lane >> 5;

    // workgroup -> (head group, row tile), heaviest causal row tiles first,
    // head groups fastest (as in the other prefill kernels)
    const int wg = blockIdx.x;
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

    // Q^T operand in registers: lane holds Q[q][16s + 8g .. +7]
    h8 qreg[C::NS];
    {
        const bool valid = q < p.Sq;
        const int qr = valid ? q : 0;
        const _Float16* qrow = qbase + (int64_t)qr * p.q_ss;
        load_q_operand(qreg, qrow, p.rot_cos + (int64_t)qr * (D / 2), p.rot_sin + (int64_t)qr * (D / 2), g, valid,
                       p.rope_q != 0, p.q_sign < 0.0f, PRE ? p.qmul : 0.0f);
    }
    // Q is in registers before the first DMA, so the per-tile vmcnt waits
    // below only ever wait for DMAs (the compiler does not see those)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));

    const int wg_q_hi = min(wg_q0 + p.rows_per_wg, p.Sq) - 1;
    int klo, khi;
    visible_key_range(p.mask, wg_q0, wg_q_hi, klo, khi);
    int t_begin = 0, t_end = 0;
    if (khi >= klo) {
        t_begin = klo / kWideBN;
        t_end = khi / kWideBN + 1;
    }
    int row_lo, row_hi;
    row_key_bounds(p.mask, q, row_lo, row_hi);

    // this wave's DMA rows of every tile: K rows and V rows wave*8 .. wave*8+7;
    // lane i moves bytes 16i .. 16i+15 of the K row (i < KCH) and of the V
    // row's column slice (i < VCH)
    const int r0 = wave * C::ROWS_PER_WAVE;
    const uint32_t lane_b = 16u * (uint32_t)lane;
    const uint32_t k_row_b = (uint32_t)(p.k_ss * 2);
    const uint32_t v_row_b = (uint32_t)(p.v_ss * 2);
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(wsm);
    auto issue_tile = [&](int t, int slot) {
        const int kt0 = t * kWideBN;
        const int sk_left = p.mask.sk - kt0;
        // one tile's byte range per descriptor (tile_bytes); the descriptor
        // words are wave-uniform (one head per wave), and readfirstlane lets
        // the compiler keep them in the SGPRs the DMA instruction needs
        auto uniform = [](i32x4_t r) {
            for (int e = 0; e < 4; e++) {
                r[e] = __builtin_amdgcn_readfirstlane(r[e]);
            }
            return r;
        };
        const i32x4_t rk =
            uniform(make_rsrc_v(kbase + (int64_t)kt0 * p.k_ss, tile_bytes<kWideBN>(sk_left, k_row_b, D * 2)));
        const i32x4_t rv =
            uniform(make_rsrc_v(vbase + (int64_t)kt0 * p.v_ss, tile_bytes<kWideBN>(sk_left, v_row_b, C::DV * 2)));
        const uint32_t sk = lds0 + slot * C::BUF_BYTES;
        const uint32_t sv = sk + C::TILE_K_BYTES;
        if (lane < C::KCH) {
#pragma unroll
            for (int j = 0; j < C::ROWS_PER_WAVE; j++) {
                const int r = r0 + j;
                dma_load16(rk, lane_b + (uint32_t)r * k_row_b, __builtin_amdgcn_readfirstlane(sk + r * (C::LDK * 2)));
            }
        }
        if (lane < C::VCH) {
#pragma unroll
            for (int j = 0; j < C::ROWS_PER_WAVE; j++) {
                const int r = r0 + j;
                dma_load16(rv, lane_b + (uint32_t)r * v_row_b, __builtin_amdgcn_readfirstlane(sv + r * (C::LDV * 2)));
            }
        }
    };

    f16x oacc[C::NDT];
#pragma unroll
    for (int dt = 0; dt < C::NDT; dt++) {
        oacc[dt] = f16x{};
    }
    float m_run = -INFINITY;
    float m_use = 0.0f;
    f16x minit = f16x{};
    float l_run = 0.0f;

    if (t_begin < t_end) {
        issue_tile(t_begin, 0);
    }
    for (int t = t_begin; t < t_end; t++) {
        const int slot = (t - t_begin) & 1;
        // this wave's rows of tile t have landed; after the barrier every
        // wave's have, and every wave is done reading tile t-1's slot
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        __syncthreads();
        if (t + 1 < t_end) {
            issue_tile(t + 1, slot ^ 1);
        }
        const int kt0 = t * kWideBN;
        // classified per tile: four more live values (tile_classes) would
        // spill at D = 352, where this kernel fills 256 VGPRs + 256 AGPRs
        const int cls = wave_active ? classify_tile(p.mask, q0, q_hi, kt0, kt0 + kWideBN - 1) : 0;
        if (cls != 0) {
            wide_tile<D, PRE>(wsm + slot * C::BUF_BYTES, qreg, oacc, m_run, m_use, minit, l_run, row_lo, row_hi, kt0,
                              p.c, lane);
        }
    }
    // no DMA may still be writing LDS when the workgroup retires
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));

    if (!wave_active) {
        return;
    }
    const float l = pair_sum(l_run);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    if (q < p.Sq) {
        _Float16* orow = obase + (int64_t)q * p.o_ss;
#pragma unroll
        for (int dt = 0; dt < C::NDT; dt++) {
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                h4 o4 = {(_Float16)(oacc[dt][4 * qq + 0] * inv), (_Float16)(oacc[dt][4 * qq + 1] * inv),
                         (_Float16)(oacc[dt][4 * qq + 2] * inv), (_Float16)(oacc[dt][4 * qq + 3] * inv)};
                *reinterpret_cast<h4*>(orow + dt * 32 + 8 * qq + 4 * g) = o4;
            }
        }
    }
}

template <int D>
int launch_wide_d(const PrefillParams& p, int64_t n_wg, hipStream_t stream, std::string& err) {
    KernelTimerGuard timer(stream);
    // Q pre-scaled into log2 units (|q c| <= |q| fits fp16); not at D = 352,
    // where the 16 registers of the start block would spill
    constexpr bool kPre = D <= 320;
    if (kPre && p.c <= 1.0f) {
        hipLaunchKernelGGL((fa_fwd_f16_wide<D, kPre>), dim3((uint32_t)n_wg), dim3(kWideThreads), 0, stream, p);
    } else {
        hipLaunchKernelGGL((fa_fwd_f16_wide<D, false>), dim3((uint32_t)n_wg), dim3(kWideThreads), 0, stream, p);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

} // namespace

int launch_wide(const PrefillParams& p, int head_dim, int64_t n_wg, hipStream_t stream, std::string& err) {
    static_assert(kWideMaxD == 352, "the switch below covers 288..kWideMaxD");
    switch (head_dim) {
    case 288: return launch_wide_d<288>(p, n_wg, stream, err);
    case 320: return launch_wide_d<320>(p, n_wg, stream, err);
    case 352: return launch_wide_d<352>(p, n_wg, stream, err);
    default: break;
    }
    err = "unsupported head_dim for the large-head prefill kernel";
    return -1;
}

} // namespace rdna_amd
