// Parameter block of the FP16 prefill kernels (device-side headers only).
#pragma once

#include "fa_common.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace rdna_amd {

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
    int32_t rows_per_wg;   // query rows per head per workgroup (32 * waves / G)
    int32_t n_row_tiles;   // ceil(Sq / rows_per_wg)
    int32_t n_head_groups; // B * Hkv * groups_per_kv
    int32_t groups_per_kv; // ratio / G
    int32_t hg_chunk;      // head groups per XCD at a time (0 = head groups fastest)
    int32_t n_items;       // n_row_tiles * n_head_groups (persistent kernels)
    float c;               // max(|scale| * log2(e), 1e-30)
    float q_sign;          // sign of scale, folded into Q (exact in fp16)
    float qmul;            // q_sign * c: Q pre-scaled into log2 units (kernels that do so, when c <= 1)
    MaskSpec mask;
    int32_t rope_q;        // rotate Q with rot_cos / rot_sin while loading it
};

// Head groups an XCD should work through at a time so that their K/V
// (kv_bytes each) fit its L2; 0 when the grid cannot be dealt evenly.
int xcd_head_group_chunk(int n_head_groups, int64_t kv_bytes);

// Prefill for head_dim 160..256 (fa_fwd_f16_kpair.hip): 8 waves, each pair of
// waves 32 rows of one head, so a workgroup holds kKPairRows / G rows of G
// heads (the launcher's PrefillParams must be set up that way).
constexpr int kKPairRows = 128;
int launch_kpair(const PrefillParams& p, int head_dim, int64_t n_wg, hipStream_t stream, std::string& err);

// Prefill for head_dim 288..512 (fa_fwd_f16_dpair.hip): 8 waves, each pair of
// waves 32 rows of one head with the head dimension split between them, so a
// workgroup holds kDPairRows / G rows of G heads (the launcher's
// PrefillParams must be set up that way).
constexpr int kDPairRows = 128;
int launch_dpair(const PrefillParams& p, int head_dim, int64_t n_wg, hipStream_t stream, std::string& err);

} // namespace rdna_amd
