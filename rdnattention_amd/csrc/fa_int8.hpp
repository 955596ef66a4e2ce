// Parameter block and launch helpers shared by the INT8 attention kernels
// (fa_fwd_int8.hip: head_dim 64 with both GEMMs on int8 MFMA;
// fa_fwd_int8_f16pv.hip: head_dim 128 and the per-token V scale extension,
// with P V on fp16 MFMA).
#pragma once

#include "fa_common.hpp"
#include "fa_host.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace rdna_amd {

constexpr int kI8Waves = 8;
constexpr int kI8Threads = 64 * kI8Waves;
constexpr int kI8BN = 64; // keys per tile = the reference's max-update block (Bc)

constexpr float kLog2Of127 = 6.98868468677f; // log2(127)

// c0 of the scheme's y = 127 p = 2^(s - m + log2 127), evaluated as
// fma(t, qeff, c0) with c0 = log2(127) - m (m = the running max, 0 while it
// is -inf).  The reference clamps pq = min(127, lroundf(127 p))
// (src/rdna/fa2_forward_int8qk.hip:335-339); here the bound comes from c0.
// The block maximum gives y <= 127 * 2^(e), e the rounding of m (from its
// product) and of c0, each within ulp(m): below |m| = 2^15, e <= 2^-8 and
// y <= 127.35 rounds to 127.  Above, c0 is lowered by |m| 2^-21 (at least
// four ulp(m)), so y < 127 there too; those rows' scores carry less than 8
// fractional bits in fp32 anyway.
__device__ __forceinline__ float int8_exp_offset(float m) {
    const float mc = m == -INFINITY ? 0.0f : m;
    const float a = fabsf(mc);
    return (kLog2Of127 - mc) - (a >= 32768.0f ? a * 0x1p-21f : 0.0f);
}

struct Int8Params {
    const int8_t* q;
    const int8_t* k;
    const int8_t* v;
    _Float16* o;
    const float* qsv;  // [B, Hq, Sq] or null
    const float* ksv;  // [B, Hkv, Sk] or null
    const float* vch;  // [B, Hkv, D] per-channel V scale or null
    const float* vtok; // [B, Hkv, Sk] per-token V scale (the per-token kernel) or null
    int32_t* scores;   // [B, Hq, Sq, Sk] int32 (the score-export instantiations only)
    float q_scale, k_scale;
    float v_scale;
    float scale_log2e;
    int64_t q_sb, q_sh, q_ss;
    int64_t k_sb, k_sh, k_ss;
    int64_t v_sb, v_sh, v_ss;
    int64_t o_sb, o_sh, o_ss;
    int32_t Hq, Sq, Hkv, ratio, G, rows_per_wg, n_row_tiles, n_head_groups, groups_per_kv;
    int32_t hg_chunk; // head groups per XCD at a time (0 = head groups fastest)
    int32_t n_items;  // n_row_tiles * n_head_groups
    MaskSpec mask;
};

// Kernel parameters and grid size of an INT8 launch.  Returns the number of
// row tiles (workgroups of a one-tile-per-workgroup grid), or -1 with `err`.
int64_t int8_params(const AttnArgs& a, Int8Params& p, std::string& err);

// The kernel with P V on fp16 MFMA (fa_fwd_int8_f16pv.hip): head_dim 128
// (forward and, with `scores`, the score export) and the per-token V scale at
// head_dim 64 or 128.
int launch_int8_f16pv(const Int8Params& p, int head_dim, bool scores, int64_t n_wg, hipStream_t stream,
                      std::string& err);

} // namespace rdna_amd
