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
