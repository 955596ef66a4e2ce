// FP16 split-K ("flash-decoding") forward for gfx950: few query rows per kv
// head against a long key sequence.  No counterpart in the reference, whose
// decode rows run one workgroup per (batch, head) over the whole cache
// (docs/api.md:203-204); same results, same masking rules.
//
// The shape is HBM-bound (each K/V byte is used by only ratio * Sq query
// rows), so the design goal is bytes in flight, not MFMA rate:
//
//   * grid = (splits, B * Hkv); a workgroup owns one contiguous key range of
//     one kv head and all M = (Hq/Hkv) * Sq query rows of that head group,
//     packed as the 32 columns of one MFMA block (M <= 32)
//   * its 4 waves work independently on interleaved 32-key tiles: each wave
//     streams K and V with buffer_load ... lds (HBM -> LDS, no VGPR staging),
//     non-temporal since every byte is read once, into its own
//     double-buffered LDS slice, two tiles in flight, no workgroup barriers in
//     the loop
//   * LDS rows are stored with an XOR swizzle of their 16-byte chunks so the
//     ds_read_b128 of K (16 rows) and the ds_read_b64_tr_b16 of V (4 rows x
//     32 B) both hit distinct banks although the DMA writes rows unpadded
//   * the waves' (max, sum, O) are merged in LDS; one partial per workgroup
//     goes to a stream-ordered scratch buffer; a combine kernel merges the
//     splits (the same log-sum-exp merge a cross-GPU sequence split would use)
#include "fa_common.hpp"
#include "fa_host.hpp"
#include "fa_internal.hpp"

#include <algorithm>
#include <cmath>

namespace rdna_amd {

float softmax_log2_scale(float scale);

namespace {

constexpr int kDecWaves = 4;
constexpr int kDecThreads = 64 * kDecWaves;
constexpr int kDecTile = 32;              // keys per wave tile
constexpr float kDecRescaleThreshold = 8.0f;

struct DecodeParams {
    const _Float16* q;
    const _Float16* k;
    const _Float16* v;
    const float* rot_cos;
    const float* rot_sin;
    int64_t q_sb, q_sh, q_ss;
    int64_t k_sb, k_sh, k_ss;
    int64_t v_sb, v_sh, v_ss;
    float* part_o;  // [B*Hkv][splits][M][D] unnormalised O
    float* part_ml; // [B*Hkv][splits][M][2]  (m in log2 units, l)
    int32_t Sq, Hkv, ratio, M, splits, keys_per_split;
    float c;
    float q_sign;
    MaskSpec mask;
    int32_t rope_q;
};

template <int D>
struct DecCfg {
    static constexpr int RB = 2 * D;                 // row bytes (unpadded)
    static constexpr int KCH = D / 8;                // 16-byte chunks per row
    static constexpr int TILE_BYTES = kDecTile * RB; // one K (or V) tile
    static constexpr int SLOT_BYTES = 2 * TILE_BYTES;
    static constexpr int WAVE_BYTES = 2 * SLOT_BYTES; // double-buffered
    static constexpr int NS = D / 16;
    static constexpr int NDT = D / 32;
    static constexpr int DMA_PER_TILE = TILE_BYTES / 1024; // 1 KB per wave-wide DMA
    static constexpr int ROWS_PER_DMA = 1024 / RB;
};

// XOR swizzle of the 16-byte chunk index of row r (see the file comment).
template <int D>
__device__ __forceinline__ int dec_swz(int r) {
    if constexpr (D == 32) {
        return (r >> 2) & 3;
    } else if constexpr (D == 64) {
        return (((r >> 1) & 3) << 1) | ((r >> 3) & 1);
    } else {
        return ((r & 7) << 1) | ((r >> 3) & 1);
    }
}

template <int D>
__global__ __launch_bounds__(kDecThreads, 1) void fa_fwd_f16_decode(DecodeParams p) {
    using C = DecCfg<D>;
    __shared__ __attribute__((aligned(16))) char dsm[kDecWaves * C::WAVE_BYTES];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); // wave-uniform
    const int lane = tid & 63;
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const int split = blockIdx.x;
    const int bkv = blockIdx.y;
    const int b = bkv / p.Hkv;
    const int kvh = bkv - b * p.Hkv;

    // column l32 <-> (query head, query row)
    const bool col_valid = l32 < p.M;
    const int hoff = col_valid ? l32 / p.Sq : 0;
    const int q = col_valid ? l32 - hoff * p.Sq : 0;
    const int h = kvh * p.ratio + hoff;

    h8 qreg[C::NS];
    {
        const int qr = q; // 0 for an unused column
        const _Float16* qrow = p.q + b * p.q_sb + h * p.q_sh + (int64_t)qr * p.q_ss;
        load_q_operand(qreg, qrow, p.rot_cos + (int64_t)qr * (D / 2), p.rot_sin + (int64_t)qr * (D / 2), g, col_valid,
                       p.rope_q != 0, p.q_sign < 0.0f);
    }
    // Q is in registers before any DMA is issued, so no later wait for it can
    // drain the DMA queue (the compiler does not see the DMAs)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    int row_lo, row_hi;
    row_key_bounds(p.mask, q, row_lo, row_hi);
    if (!col_valid) {
        row_lo = 1;
        row_hi = 0; // sees nothing
    }

    // this split's key range, restricted to what any of the M rows can see
    const int k_begin = split * p.keys_per_split;
    const int k_end = min(k_begin + p.keys_per_split, p.mask.sk);
    int vis_lo, vis_hi;
    visible_key_range(p.mask, 0, p.Sq - 1, vis_lo, vis_hi);
    const int lo = max(k_begin, vis_lo);
    const int hi = min(k_end - 1, vis_hi);
    int t0 = 0, nt = 0; // tiles of this wave: kt = t0 + wave + 4 * j
    if (hi >= lo) {
        t0 = lo / kDecTile;
        nt = hi / kDecTile + 1 - t0;
    }
    const int my_tiles = nt > wave ? (nt - wave + kDecWaves - 1) / kDecWaves : 0;

    const _Float16* kbase = p.k + b * p.k_sb + kvh * p.k_sh;
    const _Float16* vbase = p.v + b * p.v_sb + kvh * p.v_sh;
    char* wsm = dsm + wave * C::WAVE_BYTES;

    // DMA source offsets: lane i of DMA j writes LDS bytes 1024 j + 16 i of the
    // tile, i.e. row r = j * ROWS_PER_DMA + i / KCH, stored chunk i % KCH,
    // which holds logical chunk (i % KCH) ^ swz(r)
    uint32_t kdo[C::DMA_PER_TILE], vdo[C::DMA_PER_TILE];
#pragma unroll
    for (int j = 0; j < C::DMA_PER_TILE; j++) {
        const int r = j * C::ROWS_PER_DMA + lane / C::KCH;
        const int cs = lane % C::KCH;
        const int cl = cs ^ dec_swz<D>(r);
        kdo[j] = (uint32_t)(((int64_t)r * p.k_ss + 8 * cl) * 2);
        vdo[j] = (uint32_t)(((int64_t)r * p.v_ss + 8 * cl) * 2);
    }
    auto issue_tile = [&](int j_tile, int slot) {
        const int kt0 = (t0 + wave + kDecWaves * j_tile) * kDecTile;
        const i32x4_t rk = make_rsrc_v(kbase + (int64_t)kt0 * p.k_ss, tile_bytes<kDecTile>(p.mask.sk - kt0, (uint32_t)(p.k_ss * 2), D * 2));
        const i32x4_t rv = make_rsrc_v(vbase + (int64_t)kt0 * p.v_ss, tile_bytes<kDecTile>(p.mask.sk - kt0, (uint32_t)(p.v_ss * 2), D * 2));
        const uint32_t sk = (uint32_t)reinterpret_cast<uintptr_t>(wsm + slot * C::SLOT_BYTES);
        const uint32_t sv = sk + C::TILE_BYTES;
#pragma unroll
        for (int j = 0; j < C::DMA_PER_TILE; j++) {
            dma_load16_nt(rk, kdo[j], sk + 1024 * j);
        }
#pragma unroll
        for (int j = 0; j < C::DMA_PER_TILE; j++) {
            dma_load16_nt(rv, vdo[j], sv + 1024 * j);
        }
    };

    f16x oacc[C::NDT];
#pragma unroll
    for (int dt = 0; dt < C::NDT; dt++) {
        oacc[dt] = f16x{};
    }
    float m_run = -INFINITY, l_run = 0.0f;

    if (my_tiles > 0) {
        issue_tile(0, 0);
    }
    if (my_tiles > 1) {
        issue_tile(1, 1);
    }
    for (int j = 0; j < my_tiles; j++) {
        const int slot = j & 1;
        // tile j landed: at most one tile's DMAs (tile j+1) still outstanding
        if (j + 1 < my_tiles) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * C::DMA_PER_TILE));
        } else {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        }
        const int kt0 = (t0 + wave + kDecWaves * j) * kDecTile;
        const char* sk = wsm + slot * C::SLOT_BYTES;
        const char* sv = sk + C::TILE_BYTES;

        // S^T[key][col] = K Q^T over one 32-key tile
        f16x sacc = {};
        {
            const int r = l32;
            const char* krow = sk + r * C::RB;
            const int sw = dec_swz<D>(r);
#pragma unroll
            for (int s = 0; s < C::NS; s++) {
                const int cl = 2 * s + g;
                h8 a = *reinterpret_cast<const h8*>(krow + ((cl ^ sw) << 4));
                sacc = mfma_32x32x16_f16(a, qreg[s], sacc);
            }
        }
        // mask (only where a tile crosses a row's visible range; cheap anyway)
        {
            const int a = row_lo - kt0 - 4 * g;
            const int bnd = row_hi - kt0 - 4 * g;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int off = 8 * (e >> 2) + (e & 3);
                sacc[e] = (off < a || off > bnd) ? -INFINITY : sacc[e];
            }
        }
        float mx = max_tree<16>([&](int e) { return sacc[e]; });
        mx = pair_max(mx);
        const float m_new = fmaxf(m_run, mx * p.c);
        const bool grow = m_new > m_run + kDecRescaleThreshold;
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
        }
        const float m_use = (m_run == -INFINITY) ? 0.0f : m_run;
        h8 pb[2];
        float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f}; // four independent chains
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const float pv = fast_exp2(fmaf(sacc[e], p.c, -m_use));
            ps[e & 3] += pv;
            pb[e >> 3][e & 7] = (_Float16)pv;
        }
        l_run += (ps[0] + ps[1]) + (ps[2] + ps[3]);

        // O^T += V^T P^T; V^T operand through transpose reads
        {
            const int j16 = lane & 15;
#pragma unroll
            for (int u = 0; u < 2; u++) {
#pragma unroll
                for (int dt = 0; dt < C::NDT; dt++) {
                    h4 half4[2];
#pragma unroll
                    for (int hh = 0; hh < 2; hh++) {
                        const int r = 16 * u + 8 * hh + 4 * g + (j16 >> 2);
                        const int d = 32 * dt + 16 * ((lane >> 4) & 1) + 4 * (j16 & 3);
                        const int cl = d >> 3;
                        const char* addr = sv + r * C::RB + ((cl ^ dec_swz<D>(r)) << 4) + ((d & 7) << 1);
                        half4[hh] = lds_read_tr16(reinterpret_cast<const _Float16*>(addr));
                    }
                    h8 a = __builtin_shufflevector(half4[0], half4[1], 0, 1, 2, 3, 4, 5, 6, 7);
                    oacc[dt] = mfma_32x32x16_f16(a, pb[u], oacc[dt]);
                }
            }
        }
        // every LDS read of this slot has returned before the next DMA lands in it
        if (j + 2 < my_tiles) {
            __builtin_amdgcn_s_waitcnt(waitcnt_lgkm(0));
            issue_tile(j + 2, slot);
        }
    }
    __builtin_amdgcn_s_waitcnt(0); // all DMAs and LDS traffic of this wave done
    __syncthreads();

    // ---- merge the 4 waves in LDS (reusing the tile buffers)
    float* sm_ml = reinterpret_cast<float*>(dsm);                 // [4][32][2]
    float* sm_o = reinterpret_cast<float*>(dsm + 4 * 32 * 2 * 4); // [4][D][32]
    const float l_tot = pair_sum(l_run);
    if (g == 0) {
        sm_ml[(wave * 32 + l32) * 2 + 0] = m_run;
        sm_ml[(wave * 32 + l32) * 2 + 1] = l_tot;
    }
    __syncthreads();
    float mref = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecWaves; w++) {
        const float mw = sm_ml[(w * 32 + l32) * 2 + 0];
        if (sm_ml[(w * 32 + l32) * 2 + 1] > 0.0f) {
            mref = fmaxf(mref, mw);
        }
    }
    const float scale_w = (l_tot > 0.0f) ? fast_exp2(m_run - mref) : 0.0f;
#pragma unroll
    for (int dt = 0; dt < C::NDT; dt++) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int d = 32 * dt + 8 * (e >> 2) + 4 * g + (e & 3);
            sm_o[(wave * D + d) * 32 + l32] = oacc[dt][e] * scale_w;
        }
    }
    __syncthreads();
    const int64_t part = (int64_t)bkv * p.splits + split;
    for (int e = tid; e < p.M * D; e += kDecThreads) {
        const int col = e / D;
        const int d = e - col * D;
        float acc = 0.0f;
#pragma unroll
        for (int w = 0; w < kDecWaves; w++) {
            acc += sm_o[(w * D + d) * 32 + col];
        }
        p.part_o[(part * p.M + col) * D + d] = acc;
    }
    if (tid < p.M) {
        float mr = -INFINITY, lsum = 0.0f;
#pragma unroll
        for (int w = 0; w < kDecWaves; w++) {
            if (sm_ml[(w * 32 + tid) * 2 + 1] > 0.0f) {
                mr = fmaxf(mr, sm_ml[(w * 32 + tid) * 2 + 0]);
            }
        }
#pragma unroll
        for (int w = 0; w < kDecWaves; w++) {
            const float lw = sm_ml[(w * 32 + tid) * 2 + 1];
            if (lw > 0.0f) {
                lsum += lw * fast_exp2(sm_ml[(w * 32 + tid) * 2 + 0] - mr);
            }
        }
        p.part_ml[(part * p.M + tid) * 2 + 0] = mr;
        p.part_ml[(part * p.M + tid) * 2 + 1] = lsum;
    }
}

struct CombineParams {
    const float* part_o;
    const float* part_ml;
    _Float16* o;
    int64_t o_sb, o_sh, o_ss;
    int32_t Hkv, ratio, Sq, M, splits, D;
};

// One workgroup per output row (b, kv head, column): log-sum-exp merge of the
// splits, normalise once in fp32, round once to fp16.
__global__ __launch_bounds__(128) void fa_decode_combine(CombineParams p) {
    const int row = blockIdx.x; // (b * Hkv + kvh) * M + col
    const int col = row % p.M;
    const int bkv = row / p.M;
    const int b = bkv / p.Hkv;
    const int kvh = bkv - b * p.Hkv;
    const int h = kvh * p.ratio + col / p.Sq;
    const int q = col % p.Sq;
    float mref = -INFINITY;
    for (int s = 0; s < p.splits; s++) {
        const float* ml = p.part_ml + (((int64_t)bkv * p.splits + s) * p.M + col) * 2;
        if (ml[1] > 0.0f) {
            mref = fmaxf(mref, ml[0]);
        }
    }
    float lsum = 0.0f;
    for (int s = 0; s < p.splits; s++) {
        const float* ml = p.part_ml + (((int64_t)bkv * p.splits + s) * p.M + col) * 2;
        if (ml[1] > 0.0f) {
            lsum += ml[1] * fast_exp2(ml[0] - mref);
        }
    }
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    _Float16* orow = p.o + b * p.o_sb + h * p.o_sh + (int64_t)q * p.o_ss;
    for (int d = threadIdx.x; d < p.D; d += blockDim.x) {
        float acc = 0.0f;
        for (int s = 0; s < p.splits; s++) {
            const int64_t part = (int64_t)bkv * p.splits + s;
            const float* ml = p.part_ml + (part * p.M + col) * 2;
            if (ml[1] > 0.0f) {
                acc += p.part_o[(part * p.M + col) * p.D + d] * fast_exp2(ml[0] - mref);
            }
        }
        orow[d] = (_Float16)(acc * inv);
    }
}

template <int D>
int launch_decode(const DecodeParams& p, int n_bkv, hipStream_t stream, std::string& err) {
    KernelTimerGuard timer(stream);
    hipLaunchKernelGGL(fa_fwd_f16_decode<D>, dim3(p.splits, n_bkv), dim3(kDecThreads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

template <int D>
int64_t decode_resident(std::string& err) {
    return resident_workgroups(reinterpret_cast<const void*>(&fa_fwd_f16_decode<D>), kDecThreads, err);
}

} // namespace

bool splitk_supported(const AttnArgs& a) {
    const int M = (a.Hq / a.Hkv) * a.Sq;
    return (a.D == 32 || a.D == 64 || a.D == 128) && M <= 32;
}

int splitk_plan(const AttnArgs& a, int& splits, int& keys_per_split, std::string& err) {
    // splits: one round of workgroups over the device (as many as it holds at
    // once: one per CU at D = 128, where the LDS ring is 128 KB), each split a
    // whole number of 4-wave tile rounds. Measured on the B=16 Hkv=8
    // Sk=32768 cache: 256 workgroups stream 1-4 % faster than 512 and
    // 4-14 % faster than 1024 or 2048; uneven counts (384, 768) are slower.
    const int n_bkv = a.B * a.Hkv;
    const int round = kDecWaves * kDecTile;
    const int max_splits = std::max(1, (a.Sk + round - 1) / round);
    const int64_t resident = a.D == 32 ? decode_resident<32>(err)
                                       : (a.D == 64 ? decode_resident<64>(err) : decode_resident<128>(err));
    if (resident <= 0) {
        return -1;
    }
    const int n = (int)std::max<int64_t>(1, std::min<int64_t>(max_splits, (resident + n_bkv - 1) / n_bkv));
    int kps = (a.Sk + n - 1) / n;
    kps = std::max(round, (kps + round - 1) / round * round);
    splits = std::max(1, (a.Sk + kps - 1) / kps);
    keys_per_split = kps;
    return 0;
}

size_t splitk_partial_bytes(const AttnArgs& a, int splits) {
    const size_t n_part = (size_t)a.B * a.Hkv * splits * ((a.Hq / a.Hkv) * a.Sq);
    return n_part * (a.D + 2) * sizeof(float);
}

int fwd_f16_splitk(const AttnArgs& a, bool rope_q, hipStream_t stream, std::string& err, ScratchRegion* region) {
    if (!splitk_supported(a)) {
        err = "split-K path needs head_dim in {32, 64, 128} and (num_heads / num_kv_heads) * seq_len <= 32";
        return -1;
    }
    DecodeParams p{};
    p.q = static_cast<const _Float16*>(a.q);
    p.k = static_cast<const _Float16*>(a.k);
    p.v = static_cast<const _Float16*>(a.v);
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
    p.Sq = a.Sq;
    p.Hkv = a.Hkv;
    p.ratio = a.Hq / a.Hkv;
    p.M = p.ratio * a.Sq;
    p.c = softmax_log2_scale(a.scale);
    p.q_sign = a.scale < 0.0f ? -1.0f : 1.0f;
    p.mask = MaskSpec{a.Sk, a.Sk - a.Sq, a.causal ? 1 : 0, a.window > 0 ? a.window : 0};
    p.rope_q = rope_q ? 1 : 0;

    const int n_bkv = a.B * a.Hkv;
    int splits = 0, kps = 0;
    if (splitk_plan(a, splits, kps, err) != 0) {
        return -1;
    }
    p.splits = splits;
    p.keys_per_split = kps;

    // every partial is written by its split's workgroup before the combine
    // reads it, so the buffer needs no clearing
    StreamScratch ws(ScratchUse::SplitKPartials, region);
    const size_t n_part = (size_t)n_bkv * splits * p.M;
    if (ws.alloc(splitk_partial_bytes(a, splits), stream, err) != 0) {
        return -1;
    }
    p.part_o = static_cast<float*>(ws.ptr);
    p.part_ml = p.part_o + n_part * a.D;

    int rc = -1;
    switch (a.D) {
    case 32: rc = launch_decode<32>(p, n_bkv, stream, err); break;
    case 64: rc = launch_decode<64>(p, n_bkv, stream, err); break;
    case 128: rc = launch_decode<128>(p, n_bkv, stream, err); break;
    default: err = "unsupported head_dim"; return -1;
    }
    if (rc != 0) {
        return rc;
    }
    CombineParams cp{};
    cp.part_o = p.part_o;
    cp.part_ml = p.part_ml;
    cp.o = static_cast<_Float16*>(a.o);
    cp.o_sb = a.os[0];
    cp.o_sh = a.os[1];
    cp.o_ss = a.os[2];
    cp.Hkv = a.Hkv;
    cp.ratio = p.ratio;
    cp.Sq = a.Sq;
    cp.M = p.M;
    cp.splits = splits;
    cp.D = a.D;
    hipLaunchKernelGGL(fa_decode_combine, dim3((uint32_t)(n_bkv * p.M)), dim3(128), 0, stream, cp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

} // namespace rdna_amd
