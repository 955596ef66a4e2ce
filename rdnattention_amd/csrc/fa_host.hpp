// Host-side argument block shared by the C ABI (c_api.cpp) and the kernel
// launchers.  Arguments arrive here already validated; launchers only pick a
// kernel, size the grid and enqueue on the caller's stream.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace rdna_amd {

struct AttnArgs {
    const void* q = nullptr;
    const void* k = nullptr;
    const void* v = nullptr;
    void* o = nullptr;
    const float* rot_cos = nullptr;
    const float* rot_sin = nullptr;
    // element strides (batch, head, seq); the head_dim stride is 1
    int64_t qs[3] = {0, 0, 0};
    int64_t ks[3] = {0, 0, 0};
    int64_t vs[3] = {0, 0, 0};
    int64_t os[3] = {0, 0, 0};
    int32_t B = 0, Hq = 0, Hkv = 0, Sq = 0, Sk = 0, D = 0;
    float scale = 1.0f;
    int32_t causal = 0;
    int32_t has_rope = 0;
    int32_t window = 0; // > 0 enables the sliding window
    // INT8 only
    float q_scale = 1.0f, k_scale = 1.0f, v_scale = 1.0f;
    const float* q_scale_vec = nullptr;
    const float* k_scale_vec = nullptr;
    // per-channel V scale [B, Hkv, D] (contiguous) multiplied into the output,
    // or null
    const float* v_channel = nullptr;
    // per-token V scale [B, Hkv, Sk] (contiguous) applied to each V row as it
    // is staged, or null
    const float* v_token = nullptr;
};

// INT8 quantiser arguments: x fp16 or fp32 [B, H, S, D] (element strides
// b, h, s; unit stride along D) -> q int8 [B, H, S, D] contiguous and fp32
// scales, [B, H, S] per token or [B, H, D] per channel.
struct QuantArgs {
    const void* x = nullptr;
    int32_t x_fp32 = 0;
    int64_t xs[3] = {0, 0, 0};
    int32_t B = 0, H = 0, S = 0, D = 0;
    int32_t per_channel = 0;
    const float* rot_cos = nullptr; // per token only: RoPE tables [>= S, D/2] fp32, or null
    const float* rot_sin = nullptr;
    void* q = nullptr;
    float* scale = nullptr;
};

// Kernel paths the FP16 dispatcher can take.
enum class F16Path : int32_t { Auto = 0, Prefill = 1, SplitK = 2 };

struct ScratchRegion;

// FP16 forward (prefill tiles or split-K decode).  Returns 0 or sets `err`.
// With `region`, every scratch buffer (the RoPE-rotated K copy, the split-K
// partials) is carved from it and nothing is allocated; the caller first
// checks fwd_f16_scratch_bytes against its size.
int fwd_f16(const AttnArgs& a, F16Path path, hipStream_t stream, std::string& err, ScratchRegion* region = nullptr);

// Scratch bytes fwd_f16 takes for these arguments (each buffer 256-byte
// aligned), or -1 with `err`.
int64_t fwd_f16_scratch_bytes(const AttnArgs& a, F16Path path, std::string& err);

// INT8 forward (Q K^T on int8 MFMA, P V on fp16 MFMA).  Returns 0 or sets `err`.
int fwd_int8(const AttnArgs& a, hipStream_t stream, std::string& err);

// INT8 quantisation on the GPU (fa_quant.hip).  Returns 0 or sets `err`.
int quantize_int8(const QuantArgs& a, hipStream_t stream, std::string& err);

// Test export: exact int32 S = Q_i8 K_i8^T into `scores` [B,Hq,Sq,Sk] (contiguous).
int int8_scores(const AttnArgs& a, int32_t* scores, hipStream_t stream, std::string& err);

} // namespace rdna_amd
