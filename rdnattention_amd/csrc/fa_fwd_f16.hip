// FP16 FlashAttention-2 forward for gfx950 (MI355X): prefill kernel.
//
// Replaces the reference's forwardKernel / forwardKernelGqa
// (src/rdna/fa2_forward_f16.hip:633-877) with a CDNA4 MFMA design:
//
//   * one workgroup = 4 waves; every wave owns 32 query rows of one head;
//     a workgroup holds G query heads of one kv head (G | Hq/Hkv, G <= 4) so
//     each K/V tile staged in LDS serves 128 (query, head) rows
//   * S^T = K Q^T on v_mfma_f32_32x32x16_f16: a lane owns one query column,
//     so the row max/sum are lane-local plus one exchange across half-waves
//   * P^T leaves the S^T accumulator in exactly the B-operand layout of the
//     O^T = V^T P^T MFMA, so P never touches LDS
//   * V is transposed into LDS (sVT[d][key]) with the key quads of every
//     16-key group stored in the order 0,2,1,3 -- the order P^T's rows come
//     out of the accumulator -- so each A operand is one 16-byte LDS read
//   * key tiles outside the causal/window band are skipped per workgroup,
//     tiles fully inside it run without any per-element mask
//   * K/V tiles for step t+1 are loaded from HBM into registers while step
//     t computes; RoPE is applied to Q once and to K while staging it
#include "fa_common.hpp"
#include "fa_host.hpp"

#include <algorithm>

namespace rdna_amd {
namespace {

struct PrefillParams {
    const _Float16* q;
    const _Float16* k;
    const _Float16* v;
    _Float16* o;
    const float* rot_cos;
    const float* rot_sin;
    int64_t q_sb, q_sh, q_ss;
    int64_t k_sb, k_sh, k_ss;
    int64_t v_sb, v_sh, v_ss;
    int64_t o_sb, o_sh, o_ss;
    int32_t Sq, Hkv, ratio;
    int32_t G;             // query heads per workgroup
    int32_t rows_per_wg;   // query rows per head per workgroup (128 / G)
    int32_t n_row_tiles;   // ceil(Sq / rows_per_wg)
    int32_t n_head_groups; // B * Hkv * groups_per_kv
    int32_t groups_per_kv; // ratio / G
    float c;               // |scale| * log2(e)
    float q_sign;          // sign of scale, folded into Q (exact in fp16)
    MaskSpec mask;
    int32_t has_rope;
};

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBN = 64; // keys per tile

template <int D>
struct PrefillCfg {
    static constexpr int K_LD = D + 8;     // sK row stride (halves); +16 B keeps b128 reads conflict-free
    static constexpr int VT_LD = kBN + 8;  // sVT row stride (halves)
    static constexpr int NS = D / 16;      // QK^T reduction steps
    static constexpr int NDT = D / 32;     // O^T row tiles
    static constexpr int KCH = D / 8;      // 16-byte chunks per K/V row
    static constexpr int KTASK = kBN * KCH;
    static constexpr int KT = (KTASK + kThreads - 1) / kThreads;
    static constexpr int VTASK = (kBN / 4) * KCH; // (key quad, chunk) pairs
    static constexpr int VT = (VTASK + kThreads - 1) / kThreads;
    static constexpr int MIN_WG = D <= 128 ? 2 : 1;
};

// Position of the key quad `qd` (0..3) of a 16-key group inside sVT.
__device__ __forceinline__ int vt_quad_pos(int qd) {
    return qd == 1 ? 2 : (qd == 2 ? 1 : qd);
}

template <int D>
__global__ __launch_bounds__(kThreads, PrefillCfg<D>::MIN_WG) void fa_fwd_f16_prefill(PrefillParams p) {
    using C = PrefillCfg<D>;
    __shared__ __attribute__((aligned(16))) _Float16 sK[kBN * C::K_LD];
    __shared__ __attribute__((aligned(16))) _Float16 sVT[D * C::VT_LD];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int l32 = lane & 31;
    const int g = lane >> 5;

    // workgroup -> (head group, row tile); the last (heaviest under a causal
    // mask) row tiles are issued first, head groups fastest so consecutive
    // workgroups -- and therefore one XCD -- keep sharing K/V of a kv head
    const int wg = blockIdx.x;
    const int hg = wg % p.n_head_groups;
    const int rt = p.n_row_tiles - 1 - wg / p.n_head_groups;
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

    // ---- Q^T operand, resident in registers: lane holds Q[q][16s + 8g .. +7]
    h8 qreg[C::NS];
    {
        const bool valid = q < p.Sq;
        const _Float16* qrow = qbase + (int64_t)(valid ? q : 0) * p.q_ss;
#pragma unroll
        for (int s = 0; s < C::NS; s++) {
            h8 x = {};
            if (valid) {
                x = *reinterpret_cast<const h8*>(qrow + 16 * s + 8 * g);
                if (p.has_rope) {
                    x = rope8(x, p.rot_cos + (int64_t)q * (D / 2), p.rot_sin + (int64_t)q * (D / 2), 8 * s + 4 * g);
                }
                if (p.q_sign < 0.0f) {
                    x = -x;
                }
            }
            qreg[s] = x;
        }
    }

    // ---- key tiles this workgroup can see
    const int wg_q_hi = min(wg_q0 + p.rows_per_wg, p.Sq) - 1;
    int klo, khi;
    visible_key_range(p.mask, wg_q0, wg_q_hi, klo, khi);
    int t_begin = 0, t_end = 0;
    if (khi >= klo) {
        t_begin = klo / kBN;
        t_end = khi / kBN + 1;
    }

    f16x oacc[C::NDT];
#pragma unroll
    for (int dt = 0; dt < C::NDT; dt++) {
        oacc[dt] = f16x{};
    }
    float m_run = -INFINITY;
    float l_run = 0.0f;

    h8 kreg[C::KT];
    h8 vreg[C::VT][4];
    const int Sk = p.mask.sk;

    auto load_kv = [&](int t) {
        const int kt0 = t * kBN;
#pragma unroll
        for (int it = 0; it < C::KT; it++) {
            const int e = tid + it * kThreads;
            h8 x = {};
            if (e < C::KTASK) {
                const int row = e / C::KCH;
                const int ch = e - row * C::KCH;
                const int key = kt0 + row;
                if (key < Sk) {
                    x = *reinterpret_cast<const h8*>(kbase + (int64_t)key * p.k_ss + 8 * ch);
                }
            }
            kreg[it] = x;
        }
#pragma unroll
        for (int it = 0; it < C::VT; it++) {
            const int e = tid + it * kThreads;
            const int kq = e & 15;
            const int dc = e >> 4;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                h8 x = {};
                const int key = kt0 + 4 * kq + r;
                if (e < C::VTASK && key < Sk) {
                    x = *reinterpret_cast<const h8*>(vbase + (int64_t)key * p.v_ss + 8 * dc);
                }
                vreg[it][r] = x;
            }
        }
    };

    auto store_kv = [&](int t) {
        const int kt0 = t * kBN;
#pragma unroll
        for (int it = 0; it < C::KT; it++) {
            const int e = tid + it * kThreads;
            if (e < C::KTASK) {
                const int row = e / C::KCH;
                const int ch = e - row * C::KCH;
                const int key = kt0 + row;
                h8 x = kreg[it];
                if (p.has_rope && key < Sk) {
                    x = rope8(x, p.rot_cos + (int64_t)key * (D / 2), p.rot_sin + (int64_t)key * (D / 2), 4 * ch);
                }
                *reinterpret_cast<h8*>(&sK[row * C::K_LD + 8 * ch]) = x;
            }
        }
#pragma unroll
        for (int it = 0; it < C::VT; it++) {
            const int e = tid + it * kThreads;
            if (e < C::VTASK) {
                const int kq = e & 15;
                const int dc = e >> 4;
                const int pos = (kq >> 2) * 16 + vt_quad_pos(kq & 3) * 4;
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    h4 t4 = {vreg[it][0][c], vreg[it][1][c], vreg[it][2][c], vreg[it][3][c]};
                    *reinterpret_cast<h4*>(&sVT[(8 * dc + c) * C::VT_LD + pos]) = t4;
                }
            }
        }
    };

    if (t_begin < t_end) {
        load_kv(t_begin);
    }
    for (int t = t_begin; t < t_end; t++) {
        __syncthreads(); // every wave is done reading the previous tile
        store_kv(t);
        __syncthreads();
        if (t + 1 < t_end) {
            load_kv(t + 1); // in flight while this tile computes
        }
        if (!wave_active) {
            continue;
        }
        const int kt0 = t * kBN;
        const int cls = classify_tile(p.mask, q0, q_hi, kt0, kt0 + kBN - 1);
        if (cls == 0) {
            continue;
        }

        // ---- S^T[key][query] = K Q^T, two 32-key halves
        f16x sacc[2];
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
            f16x acc = {};
#pragma unroll
            for (int s = 0; s < C::NS; s++) {
                h8 a = *reinterpret_cast<const h8*>(&sK[(kt * 32 + l32) * C::K_LD + 16 * s + 8 * g]);
                acc = mfma_32x32x16_f16(a, qreg[s], acc);
            }
            sacc[kt] = acc;
        }

        // ---- online softmax (log2 domain)
        if (cls == 2) {
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int key = kt0 + kt * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
                    if (!key_visible(p.mask, q, key)) {
                        sacc[kt][i] = -INFINITY;
                    }
                }
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                mx = fmaxf(mx, sacc[kt][i]);
            }
        }
        mx = fmaxf(mx, swap_halves(mx));
        const float mt = (mx == -INFINITY) ? -INFINITY : mx * p.c;
        const float m_new = fmaxf(m_run, mt);
        const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
        const float alpha = fast_exp2(m_run - m_use);

        h8 pb[4];
        float psum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float s = sacc[kt][i];
                float pv = fast_exp2(fmaf(s, p.c, -m_use));
                if (cls == 2 && s == -INFINITY) {
                    pv = 0.0f;
                }
                psum += pv;
                pb[kt * 2 + (i >> 3)][i & 7] = (_Float16)pv;
            }
        }
        l_run = l_run * alpha + psum;
        m_run = m_new;
        if (wave_any(alpha != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < C::NDT; dt++) {
                oacc[dt] *= alpha;
            }
        }

        // ---- O^T[d][query] += V^T P^T
#pragma unroll
        for (int dt = 0; dt < C::NDT; dt++) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                h8 a = *reinterpret_cast<const h8*>(&sVT[(dt * 32 + l32) * C::VT_LD + u * 16 + 8 * g]);
                oacc[dt] = mfma_32x32x16_f16(a, pb[u], oacc[dt]);
            }
        }
    }

    if (!wave_active) {
        return;
    }
    // ---- normalise once in fp32, round once to fp16
    const float l = l_run + swap_halves(l_run);
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
int launch_prefill(const PrefillParams& p, int64_t n_wg, hipStream_t stream, std::string& err) {
    hipLaunchKernelGGL(fa_fwd_f16_prefill<D>, dim3((uint32_t)n_wg), dim3(kThreads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

} // namespace

int fwd_f16_prefill(const AttnArgs& a, hipStream_t stream, std::string& err) {
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
    p.G = (p.ratio % 4 == 0) ? 4 : ((p.ratio % 2 == 0) ? 2 : 1);
    p.rows_per_wg = 32 * kWaves / p.G;
    p.n_row_tiles = (a.Sq + p.rows_per_wg - 1) / p.rows_per_wg;
    p.groups_per_kv = p.ratio / p.G;
    p.n_head_groups = a.B * a.Hkv * p.groups_per_kv;
    p.c = std::fabs(a.scale) * kLog2e;
    p.q_sign = a.scale < 0.0f ? -1.0f : 1.0f;
    p.mask = MaskSpec{a.Sk, a.Sk - a.Sq, a.causal ? 1 : 0, a.window > 0 ? a.window : 0};
    p.has_rope = a.has_rope ? 1 : 0;

    const int64_t n_wg = (int64_t)p.n_row_tiles * p.n_head_groups;
    if (n_wg <= 0) {
        err = "empty launch grid";
        return -1;
    }
    if (n_wg > INT32_MAX) {
        err = "launch grid too large";
        return -1;
    }
    switch (a.D) {
    case 32: return launch_prefill<32>(p, n_wg, stream, err);
    case 64: return launch_prefill<64>(p, n_wg, stream, err);
    case 96: return launch_prefill<96>(p, n_wg, stream, err);
    case 128: return launch_prefill<128>(p, n_wg, stream, err);
    case 160: return launch_prefill<160>(p, n_wg, stream, err);
    case 192: return launch_prefill<192>(p, n_wg, stream, err);
    case 224: return launch_prefill<224>(p, n_wg, stream, err);
    case 256: return launch_prefill<256>(p, n_wg, stream, err);
    default: break;
    }
    err = "unsupported head_dim (multiples of 32 from 32 to 512)";
    return -1;
}

} // namespace rdna_amd

namespace rdna_amd {

int fwd_f16_splitk(const AttnArgs& a, hipStream_t stream, std::string& err);

int fwd_f16(const AttnArgs& a, F16Path path, hipStream_t stream, std::string& err) {
    if (path == F16Path::SplitK) {
        return fwd_f16_splitk(a, stream, err);
    }
    return fwd_f16_prefill(a, stream, err);
}

} // namespace rdna_amd
