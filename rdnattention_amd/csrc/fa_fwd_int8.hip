// INT8 FlashAttention forward for gfx950: both GEMMs on int8 MFMA
// (v_mfma_i32_32x32x32_i8, exact int32 accumulation), fp16 output.
//
// Replaces the reference's forwardKernelInt8QK
// (src/rdna/fa2_forward_int8qk.hip:229-495) and keeps its numeric scheme:
//
//   S_ij  = sum_d q_i8 k_i8                          (exact int32)
//   s_ij  = S_ij * qs_i * ks_j * scale * log2(e)      (fp32, log2 domain)
//   per 64-key block, aligned to key 0 (the reference's Bc = 64):
//     m'  = max(m, max_j s_ij);  O *= 2^(m - m'),  l *= 2^(m - m')
//     p   = 2^(s - m'),  l += sum p                  (unquantised p)
//     pq  = min(127, round(p * 127))                 (int8 P)
//     O  += (float)(sum_j pq_j v_j) * (v_scale / 127) (exact int32 GEMM)
//   out = O / l  (0 when no key is visible)
//
// The one deliberate difference: round() here is round-half-to-even
// (v_rndne_f32) where the reference calls lroundf (half away from zero); they
// differ only when p * 127 is exactly k + 0.5.
//
// Kernel structure is the FP16 ping-pong design (fa_fwd_f16.hip): 8 waves in
// two groups alternating MFMA and VALU phases, S^T = K Q^T so a lane owns one
// query column, P^T going from the S accumulator straight into the B operand
// of O^T = V^T P^T, and V^T read with the byte transpose read
// ds_read_b64_tr_b8 (in each 16-lane group, lane i's byte k is byte i % 8 of
// the 8-byte word addressed by lane 2k + i/8).
#include "fa_common.hpp"
#include "fa_host.hpp"
#include "fa_internal.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace rdna_amd {

float softmax_log2_scale(float scale);

namespace {

typedef int8_t i8x8 __attribute__((ext_vector_type(8)));
typedef int i2 __attribute__((ext_vector_type(2)));

constexpr int kI8Waves = 8;
constexpr int kI8Threads = 64 * kI8Waves;
constexpr int kI8BN = 64; // keys per tile = the reference's max-update block

struct Int8Params {
    const int8_t* q;
    const int8_t* k;
    const int8_t* v;
    _Float16* o;
    const float* qsv; // [B, Hq, Sq] or null
    const float* ksv; // [B, Hkv, Sk] or null
    float q_scale, k_scale;
    float pv_scale; // v_scale / 127
    float scale_log2e;
    int64_t q_sb, q_sh, q_ss;
    int64_t k_sb, k_sh, k_ss;
    int64_t v_sb, v_sh, v_ss;
    int64_t o_sb, o_sh, o_ss;
    int32_t Hq, Sq, Hkv, ratio, G, rows_per_wg, n_row_tiles, n_head_groups, groups_per_kv;
    MaskSpec mask;
};

template <int D>
struct I8Cfg {
    static constexpr int LD = D + 16; // LDS row stride in bytes (16 B step mod 256 across rows)
    static constexpr int TILE = kI8BN * LD;
    static constexpr int NS = D / 32;  // QK^T reduction steps (32 int8 per MFMA)
    static constexpr int NDT = D / 32; // O^T row tiles
    static constexpr int KCH = D / 16; // 16-byte chunks per row
    static constexpr int HALF_TASK = 32 * KCH;
    static constexpr int CT = (HALF_TASK + 255) / 256;
};

__device__ __forceinline__ i2 lds_read_tr8(const int8_t* p) {
    typedef __attribute__((address_space(3))) i2 lds_i2;
    const auto* lp = reinterpret_cast<const __attribute__((address_space(3))) char*>(
        (uint32_t)reinterpret_cast<uintptr_t>(p));
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i2*)lp);
}

__device__ __forceinline__ i4 buffer_load_i4(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    u4 x = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
    return __builtin_bit_cast(i4, x);
}

// p in [0, 1] -> round(p * 127) as a byte, packed into byte `sel` of `old`
__device__ __forceinline__ uint32_t quant_p(float p, uint32_t old, int sel) {
    float y = fminf(__builtin_rintf(p * 127.0f), 127.0f);
    return __builtin_amdgcn_cvt_pk_u8_f32(y, sel, old);
}

template <int D>
__global__ __launch_bounds__(kI8Threads, 1) void fa_fwd_int8(Int8Params p) {
    using C = I8Cfg<D>;
    __shared__ __attribute__((aligned(16))) int8_t smem[4 * C::TILE];
    __shared__ __attribute__((aligned(16))) float sks[2][kI8BN];
    int8_t* const sKs = smem;
    int8_t* const sVs = smem + 2 * C::TILE;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const int grp = wave >> 2;
    const int gtid = tid & 255;

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
    const int Sk = p.mask.sk;

    const int8_t* qbase = p.q + b * p.q_sb + h * p.q_sh;
    const int8_t* kbase = p.k + b * p.k_sb + kvh * p.k_sh;
    const int8_t* vbase = p.v + b * p.v_sb + kvh * p.v_sh;
    _Float16* obase = p.o + b * p.o_sb + h * p.o_sh;
    const float* ksbase = p.ksv ? p.ksv + ((int64_t)b * p.Hkv + kvh) * Sk : nullptr;

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
    const float qc = qs * p.scale_log2e;

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

    f16x oacc[C::NDT];
#pragma unroll
    for (int dt = 0; dt < C::NDT; dt++) {
        oacc[dt] = f16x{};
    }
    float m_run = -INFINITY, l_run = 0.0f;
    f16x sf[2]; // scores of the current tile, fp32, log2 domain
    sf[0] = f16x{};
    sf[1] = f16x{};
    i4 pb[2] = {i4{}, i4{}};
    int cls_prev = 0;

    // ---- staging (one group's 32 rows of K and V per pair; ks by group A)
    i4 kreg[C::CT], vreg[C::CT];
    uint32_t coff_k[C::CT], coff_v[C::CT];
    int cl[C::CT];
#pragma unroll
    for (int it = 0; it < C::CT; it++) {
        const int e = gtid + it * 256;
        const bool ok = C::HALF_TASK % 256 == 0 || e < C::HALF_TASK;
        const int row = 32 * grp + (ok ? e / C::KCH : 0);
        const int ch = ok ? e - (e / C::KCH) * C::KCH : 0;
        coff_k[it] = (uint32_t)((int64_t)row * p.k_ss + 16 * ch);
        coff_v[it] = (uint32_t)((int64_t)row * p.v_ss + 16 * ch);
        cl[it] = ok ? row * C::LD + 16 * ch : -1;
    }
    float ksreg = 0.0f;
    auto load_pair = [&](int x) {
        const int tk = t_begin + x, tv = t_begin + x - 1;
        const auto rk = make_rsrc(kbase + (int64_t)tk * kI8BN * p.k_ss,
                                  x < n ? range_bytes(Sk - tk * kI8BN, p.k_ss, D) : 0u);
        const auto rv = make_rsrc(vbase + (int64_t)tv * kI8BN * p.v_ss,
                                  (x >= 1 && x <= n) ? range_bytes(Sk - tv * kI8BN, p.v_ss, D) : 0u);
#pragma unroll
        for (int it = 0; it < C::CT; it++) {
            kreg[it] = buffer_load_i4(rk, coff_k[it]);
            vreg[it] = buffer_load_i4(rv, coff_v[it]);
        }
        if (grp == 0 && gtid < kI8BN && x < n) {
            const int key = tk * kI8BN + gtid;
            ksreg = (ksbase != nullptr && key < Sk) ? ksbase[key] : p.k_scale;
        }
    };
    auto store_pair = [&](int x) {
        int8_t* sK = sKs + (x & 1) * C::TILE;
        int8_t* sV = sVs + ((x - 1) & 1) * C::TILE;
#pragma unroll
        for (int it = 0; it < C::CT; it++) {
            if (C::HALF_TASK % 256 == 0 || cl[it] >= 0) {
                if (x < n) {
                    *reinterpret_cast<i4*>(&sK[cl[it]]) = kreg[it];
                }
                if (x >= 1 && x <= n) {
                    *reinterpret_cast<i4*>(&sV[cl[it]]) = vreg[it];
                }
            }
        }
        if (grp == 0 && gtid < kI8BN && x < n) {
            sks[x & 1][gtid] = ksreg;
        }
    };

    // M(i): O += V(i-1)^T P(i-1) (int32, converted per block) and S(i) = K(i) Q^T
    auto phase_m = [&](int i) {
        if (!wave_active) {
            return;
        }
        int cls_now = 0;
        if (i < n) {
            const int kt0 = (t_begin + i) * kI8BN;
            cls_now = classify_tile(p.mask, q0, q_hi, kt0, kt0 + kI8BN - 1);
        }
        if (i >= 1 && cls_prev != 0) {
            const int8_t* sV = sVs + ((i - 1) & 1) * C::TILE;
            // lane j of each 16-lane group points at key row kr(j/2), bytes
            // 8*(j%2) of the group's 16-column half of the d tile
            const int j16 = lane & 15;
            const int dcol = 16 * ((lane >> 4) & 1) + 8 * (j16 & 1);
            const int kk = j16 >> 1; // slot 0..7 of this read
#pragma unroll
            for (int dt = 0; dt < C::NDT; dt++) {
                i16x acc = {};
#pragma unroll
                for (int kt = 0; kt < 2; kt++) {
                    i2 part[2];
#pragma unroll
                    for (int hh = 0; hh < 2; hh++) {
                        const int slot = 8 * hh + kk; // key = 8*(slot/4) + 4g + slot%4
                        const int row = 32 * kt + 8 * (slot >> 2) + 4 * g + (slot & 3);
                        part[hh] = lds_read_tr8(sV + row * C::LD + 32 * dt + dcol);
                    }
                    i4 a = {part[0][0], part[0][1], part[1][0], part[1][1]};
                    acc = mfma_32x32x32_i8(a, pb[kt], acc);
                }
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    oacc[dt][e] = fmaf((float)acc[e], p.pv_scale, oacc[dt][e]);
                }
            }
        }
        if (cls_now != 0) {
            const int8_t* sK = sKs + (i & 1) * C::TILE;
            const float* ksl = sks[i & 1];
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                i16x acc = {};
#pragma unroll
                for (int s = 0; s < C::NS; s++) {
                    i4 a = *reinterpret_cast<const i4*>(&sK[(kt * 32 + l32) * C::LD + 32 * s + 16 * g]);
                    acc = mfma_32x32x32_i8(a, qreg[s], acc);
                }
                // s = S * qs * ks * scale * log2e
#pragma unroll
                for (int r4 = 0; r4 < 4; r4++) {
                    const f4 ks4 = *reinterpret_cast<const f4*>(&ksl[kt * 32 + 8 * r4 + 4 * g]);
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        sf[kt][4 * r4 + e] = ((float)acc[4 * r4 + e] * ks4[e]) * qc;
                    }
                }
            }
        }
        cls_prev = cls_now;
    };

    // V(i): exact running max over the 64-key block, P quantised to int8
    auto phase_v = [&](int i) {
        if (!wave_active || cls_prev == 0) {
            return;
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
                    sf[kt][e] = (off < a || off > bnd) ? -INFINITY : sf[kt][e];
                }
            }
        }
        float mx = sf[0][0];
#pragma unroll
        for (int e = 1; e < 16; e++) {
            mx = fmaxf(mx, sf[0][e]);
        }
#pragma unroll
        for (int e = 0; e < 16; e++) {
            mx = fmaxf(mx, sf[1][e]);
        }
        mx = pair_max(mx);
        const float m_new = fmaxf(m_run, mx);
        const bool grow = m_new > m_run;
        if (wave_any(grow)) {
            const float alpha = grow ? fast_exp2(m_run - m_new) : 1.0f;
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < C::NDT; dt++) {
                oacc[dt] *= alpha;
            }
        }
        const float m_use = (m_run == -INFINITY) ? 0.0f : m_run;
        float psum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
            uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const float pv = fast_exp2(sf[kt][e] - m_use);
                psum += pv;
                w[e >> 2] = quant_p(pv, w[e >> 2], e & 3);
            }
            pb[kt] = i4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        }
        l_run += psum;
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

// Exact int32 S = Q K^T on the same MFMA tiles as the attention kernel's
// first GEMM; one wave per (32 queries, 32 keys, b*h) tile.
template <int D>
__global__ __launch_bounds__(64) void int8_scores_kernel(const int8_t* __restrict__ qp, const int8_t* __restrict__ kp,
                                                        int32_t* __restrict__ out, int64_t q_sb, int64_t q_sh,
                                                        int64_t q_ss, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                                                        int32_t Hq, int32_t Hkv, int32_t Sq, int32_t Sk) {
    const int lane = threadIdx.x;
    const int l32 = lane & 31, g = lane >> 5;
    const int q0 = blockIdx.x * 32, k0 = blockIdx.y * 32;
    const int bh = blockIdx.z;
    const int b = bh / Hq, h = bh - b * Hq;
    const int kvh = h / (Hq / Hkv);
    const int q = q0 + l32, key = k0 + l32;
    i16x acc = {};
#pragma unroll
    for (int s = 0; s < D / 32; s++) {
        i4 a = key < Sk ? *reinterpret_cast<const i4*>(kp + b * k_sb + kvh * k_sh + (int64_t)key * k_ss + 32 * s + 16 * g)
                        : i4{};
        i4 bq = q < Sq ? *reinterpret_cast<const i4*>(qp + b * q_sb + h * q_sh + (int64_t)q * q_ss + 32 * s + 16 * g)
                       : i4{};
        acc = mfma_32x32x32_i8(a, bq, acc);
    }
    if (q < Sq) {
        int32_t* orow = out + ((int64_t)bh * Sq + q) * Sk;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int kk = k0 + 8 * (e >> 2) + 4 * g + (e & 3);
            if (kk < Sk) {
                orow[kk] = acc[e];
            }
        }
    }
}

template <int D>
int launch_int8(const Int8Params& p, int64_t n_wg, hipStream_t stream, std::string& err) {
    KernelTimerGuard timer(stream);
    hipLaunchKernelGGL(fa_fwd_int8<D>, dim3((uint32_t)n_wg), dim3(kI8Threads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

} // namespace

int fwd_int8(const AttnArgs& a, hipStream_t stream, std::string& err) {
    if (a.ks[2] < 0 || a.vs[2] < 0 || a.ks[2] > (1 << 24) || a.vs[2] > (1 << 24)) {
        err = "key/value seq strides must be in [0, 2^24] elements";
        return -1;
    }
    Int8Params p{};
    p.q = static_cast<const int8_t*>(a.q);
    p.k = static_cast<const int8_t*>(a.k);
    p.v = static_cast<const int8_t*>(a.v);
    p.o = static_cast<_Float16*>(a.o);
    p.qsv = a.q_scale_vec;
    p.ksv = a.k_scale_vec;
    p.q_scale = a.q_scale;
    p.k_scale = a.k_scale;
    p.pv_scale = (1.0f / 127.0f) * a.v_scale;
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
    p.mask = MaskSpec{a.Sk, a.Sk - a.Sq, a.causal ? 1 : 0, a.window > 0 ? a.window : 0};
    const int64_t n_wg = (int64_t)p.n_row_tiles * p.n_head_groups;
    if (n_wg <= 0 || n_wg > INT32_MAX) {
        err = "launch grid out of range";
        return -1;
    }
    switch (a.D) {
    case 64: return launch_int8<64>(p, n_wg, stream, err);
    case 128: return launch_int8<128>(p, n_wg, stream, err);
    default: break;
    }
    err = "unsupported head_dim (only 64 and 128 are compiled in for the int8 kernel)";
    return -1;
}

int int8_scores(const AttnArgs& a, int32_t* scores, hipStream_t stream, std::string& err) {
    dim3 grid((uint32_t)((a.Sq + 31) / 32), (uint32_t)((a.Sk + 31) / 32), (uint32_t)(a.B * a.Hq));
    if (a.D == 64) {
        hipLaunchKernelGGL(int8_scores_kernel<64>, grid, dim3(64), 0, stream, static_cast<const int8_t*>(a.q),
                           static_cast<const int8_t*>(a.k), scores, a.qs[0], a.qs[1], a.qs[2], a.ks[0], a.ks[1],
                           a.ks[2], a.Hq, a.Hkv, a.Sq, a.Sk);
    } else {
        hipLaunchKernelGGL(int8_scores_kernel<128>, grid, dim3(64), 0, stream, static_cast<const int8_t*>(a.q),
                           static_cast<const int8_t*>(a.k), scores, a.qs[0], a.qs[1], a.qs[2], a.ks[0], a.ks[1],
                           a.ks[2], a.Hq, a.Hkv, a.Sq, a.Sk);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

} // namespace rdna_amd
