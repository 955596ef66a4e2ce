// C ABI and C++ launch API of librdnattention.so.
//
// Mirrors the reference's boundary (src/c_api.cpp:15-195, src/c_api.hpp:16-87,
// src/rdna/fa2_forward_f16.hpp, src/rdna/fa2_forward_int8qk.hpp): the same
// exported names and argument lists, return codes 0 / -3 / -4, and a
// thread-local 512-byte error buffer set only on failure, with the messages
// "Attention (fp16) failed: %s" and "Attention (int8qk) failed: %s".
//
// Unlike the reference, every argument the kernels depend on is checked here,
// before any HIP call: head_dim, the GQA ratio, empty grids, null pointers,
// 16-byte alignment of pointers and strides (the reference's 128-bit loads
// assumed it silently), RoPE tables, and int32 index ranges.
#include "rdnattention.h"
#include "rdnattention.hpp"
#include "rdnattention_ext.h"
#include "fa_host.hpp"
#include "fa_internal.hpp"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>

using rdna_amd::AttnArgs;
using rdna_amd::F16Path;

namespace {

thread_local char g_error[512] = {0};
thread_local char g_last_f16[256] = {0};
thread_local char g_last_i8[256] = {0};

void set_error(const char* fmt, const std::string& detail) {
    std::snprintf(g_error, sizeof(g_error), fmt, detail.empty() ? "unknown error" : detail.c_str());
}

bool aligned(const void* p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

bool stride_ok(const int64_t s[3], int64_t mult) {
    return s[0] % mult == 0 && s[1] % mult == 0 && s[2] % mult == 0;
}

constexpr uint32_t kMaxSeq = 1u << 30;

#if defined(RDNATTENTION_NO_INT8)
// the reference's FP16-only build text (src/c_api.cpp:151-153)
constexpr const char* kNoInt8 = "this library was built without the INT8 kernel - use rdna_attention_forward() instead";
#endif

// Shared checks.  Returns "" when the arguments are acceptable.
std::string check_common(const AttnArgs& a, uint32_t B, uint32_t Hq, uint32_t Hkv, uint32_t Sq, uint32_t Sk,
                         int64_t in_mult) {
    if (Hkv == 0 || Hq % Hkv != 0) {
        return "numHeads must be a positive multiple of numKvHeads";
    }
    if (B == 0 || Hq == 0 || Sq == 0) {
        return "empty launch grid (batch_size, num_heads and seq_len must be non-zero)";
    }
    if (Sq > kMaxSeq || Sk > kMaxSeq || (uint64_t)B * Hq > (uint64_t)INT32_MAX) {
        return "tensor dimensions exceed the supported range (seq_len, key_seq_len <= 2^30)";
    }
    if (a.q == nullptr || a.o == nullptr || (Sk > 0 && (a.k == nullptr || a.v == nullptr))) {
        return "null tensor pointer";
    }
    if (!aligned(a.q, 16) || !aligned(a.k, 16) || !aligned(a.v, 16) || !aligned(a.o, 16)) {
        return "tensor base pointers must be 16-byte aligned";
    }
    if (!stride_ok(a.qs, in_mult) || !stride_ok(a.ks, in_mult) || !stride_ok(a.vs, in_mult) || !stride_ok(a.os, 8)) {
        return "batch/head/seq strides must be multiples of 16 bytes (8 fp16 or 16 int8 elements)";
    }
    return "";
}

bool head_dim_f16_ok(uint32_t d) {
    return d >= 32 && d <= 512 && d % 32 == 0;
}

int32_t forward_f16_impl(const void* q, const void* k, const void* v, void* output, const void* rot_cos,
                         const void* rot_sin, int64_t qsb, int64_t qsh, int64_t qss, int64_t ksb, int64_t ksh,
                         int64_t kss, int64_t vsb, int64_t vsh, int64_t vss, int64_t osb, int64_t osh, int64_t oss,
                         uint32_t B, uint32_t Hq, uint32_t Hkv, uint32_t Sq, uint32_t Sk, uint32_t D, float scale,
                         int32_t causal, int32_t has_rope, int32_t window, F16Path path, void* stream,
                         std::string& err, bool noalloc = false) {
    if (!head_dim_f16_ok(D)) {
        err = "unsupported head_dim (multiples of 32 from 32 to 512)";
        return -1;
    }
    AttnArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = output;
    a.rot_cos = static_cast<const float*>(rot_cos);
    a.rot_sin = static_cast<const float*>(rot_sin);
    a.qs[0] = qsb, a.qs[1] = qsh, a.qs[2] = qss;
    a.ks[0] = ksb, a.ks[1] = ksh, a.ks[2] = kss;
    a.vs[0] = vsb, a.vs[1] = vsh, a.vs[2] = vss;
    a.os[0] = osb, a.os[1] = osh, a.os[2] = oss;
    err = check_common(a, B, Hq, Hkv, Sq, Sk, 8);
    if (!err.empty()) {
        return -1;
    }
    if (has_rope != 0 && (rot_cos == nullptr || rot_sin == nullptr)) {
        err = "has_rope is set but rot_cos/rot_sin is null";
        return -1;
    }
    if (has_rope != 0 && (!aligned(rot_cos, 16) || !aligned(rot_sin, 16))) {
        err = "rot_cos/rot_sin must be 16-byte aligned";
        return -1;
    }
    if (path != F16Path::Auto && path != F16Path::Prefill && path != F16Path::SplitK) {
        err = "unknown kernel path";
        return -1;
    }
    a.B = (int32_t)B;
    a.Hq = (int32_t)Hq;
    a.Hkv = (int32_t)Hkv;
    a.Sq = (int32_t)Sq;
    a.Sk = (int32_t)Sk;
    a.D = (int32_t)D;
    a.scale = scale;
    a.causal = causal != 0 ? 1 : 0;
    a.has_rope = has_rope != 0 ? 1 : 0;
    a.window = window > 0 ? window : 0;
    if (!noalloc) {
        return rdna_amd::fwd_f16(a, path, static_cast<hipStream_t>(stream), err);
    }
    // every scratch buffer from the static array; sized before any launch
    const int64_t need = rdna_amd::fwd_f16_scratch_bytes(a, path, err);
    if (need < 0) {
        return -1;
    }
    if ((uint64_t)need > rdna_amd::kNoAllocBytes) {
        err = "this call needs " + std::to_string(need) +
              " bytes of scratch (RoPE-rotated K copy and/or split-K partials); the no-allocation entry point "
              "provides " +
              std::to_string(rdna_amd::kNoAllocBytes) + " bytes per device";
        return -1;
    }
    rdna_amd::ScratchRegion region;
    if (rdna_amd::noalloc_region(region, err) != 0) {
        return -1;
    }
    return rdna_amd::fwd_f16(a, path, static_cast<hipStream_t>(stream), err, &region);
}

int32_t forward_i8_impl(const void* q, const void* k, const void* v, void* output, int64_t qsb, int64_t qsh,
                        int64_t qss, int64_t ksb, int64_t ksh, int64_t kss, int64_t vsb, int64_t vsh, int64_t vss,
                        int64_t osb, int64_t osh, int64_t oss, uint32_t B, uint32_t Hq, uint32_t Hkv, uint32_t Sq,
                        uint32_t Sk, uint32_t D, float scale, float q_scale, float k_scale, float v_scale,
                        const void* q_scale_vec, const void* k_scale_vec, const void* v_channel_vec,
                        const void* v_token_vec, int32_t causal, int32_t window, void* stream, std::string& err) {
    // order of the reference's checks: ratio, then head_dim (fa2_forward_int8qk.hip:570-589)
    if (Hkv == 0 || Hq % Hkv != 0) {
        err = "numHeads must be a positive multiple of numKvHeads";
        return -1;
    }
    if (D != 64 && D != 128) {
        err = "unsupported head_dim (only 64 and 128 are compiled in for the int8 kernel)";
        return -1;
    }
    AttnArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = output;
    a.qs[0] = qsb, a.qs[1] = qsh, a.qs[2] = qss;
    a.ks[0] = ksb, a.ks[1] = ksh, a.ks[2] = kss;
    a.vs[0] = vsb, a.vs[1] = vsh, a.vs[2] = vss;
    a.os[0] = osb, a.os[1] = osh, a.os[2] = oss;
    err = check_common(a, B, Hq, Hkv, Sq, Sk, 16);
    if (!err.empty()) {
        return -1;
    }
    if (!aligned(q_scale_vec, 4) || !aligned(k_scale_vec, 4)) {
        err = "q_scale_vec/k_scale_vec must be 4-byte aligned float arrays";
        return -1;
    }
    if (!aligned(v_channel_vec, 16)) {
        err = "v_channel_vec must be a 16-byte aligned float array";
        return -1;
    }
    if (!aligned(v_token_vec, 4)) {
        err = "v_token_vec must be a 4-byte aligned float array";
        return -1;
    }
    if (v_channel_vec != nullptr && v_token_vec != nullptr) {
        err = "v_channel_vec and v_token_vec are exclusive";
        return -1;
    }
    a.B = (int32_t)B;
    a.Hq = (int32_t)Hq;
    a.Hkv = (int32_t)Hkv;
    a.Sq = (int32_t)Sq;
    a.Sk = (int32_t)Sk;
    a.D = (int32_t)D;
    a.scale = scale;
    a.causal = causal != 0 ? 1 : 0;
    a.window = window > 0 ? window : 0;
    a.q_scale = q_scale;
    a.k_scale = k_scale;
    a.v_scale = v_scale;
    a.q_scale_vec = static_cast<const float*>(q_scale_vec);
    a.k_scale_vec = static_cast<const float*>(k_scale_vec);
    a.v_channel = static_cast<const float*>(v_channel_vec);
    a.v_token = static_cast<const float*>(v_token_vec);
    return rdna_amd::fwd_int8(a, static_cast<hipStream_t>(stream), err);
}

} // namespace

RDNA_API int32_t rdna_has_device(void) {
    return rdna::hasDevice() ? 1 : 0;
}

RDNA_API const char* rdna_get_error(void) {
    return g_error;
}

RDNA_API const char* rdna_version(void) {
    return "0.1.0-gfx950";
}

RDNA_API int32_t rdna_attention_forward(const void* q, const void* k, const void* v, void* output,
                                        const void* rot_cos, const void* rot_sin, int64_t q_stride_b,
                                        int64_t q_stride_h, int64_t q_stride_s, int64_t k_stride_b,
                                        int64_t k_stride_h, int64_t k_stride_s, int64_t v_stride_b,
                                        int64_t v_stride_h, int64_t v_stride_s, int64_t o_stride_b,
                                        int64_t o_stride_h, int64_t o_stride_s, uint32_t batch_size,
                                        uint32_t num_heads, uint32_t num_kv_heads, uint32_t seq_len,
                                        uint32_t key_seq_len, uint32_t head_dim, float scale, int32_t causal,
                                        int32_t has_rope, int32_t window_size, void* hip_stream) {
    std::string err;
    int rc = forward_f16_impl(q, k, v, output, rot_cos, rot_sin, q_stride_b, q_stride_h, q_stride_s, k_stride_b,
                              k_stride_h, k_stride_s, v_stride_b, v_stride_h, v_stride_s, o_stride_b, o_stride_h,
                              o_stride_s, batch_size, num_heads, num_kv_heads, seq_len, key_seq_len, head_dim,
                              scale, causal, has_rope, window_size, F16Path::Auto, hip_stream, err);
    if (rc != 0) {
        set_error("Attention (fp16) failed: %s", err);
        return -3;
    }
    return 0;
}

RDNA_API int32_t rdna_attention_forward_noalloc(const void* q, const void* k, const void* v, void* output,
                                                const void* rot_cos, const void* rot_sin, int64_t q_stride_b,
                                                int64_t q_stride_h, int64_t q_stride_s, int64_t k_stride_b,
                                                int64_t k_stride_h, int64_t k_stride_s, int64_t v_stride_b,
                                                int64_t v_stride_h, int64_t v_stride_s, int64_t o_stride_b,
                                                int64_t o_stride_h, int64_t o_stride_s, uint32_t batch_size,
                                                uint32_t num_heads, uint32_t num_kv_heads, uint32_t seq_len,
                                                uint32_t key_seq_len, uint32_t head_dim, float scale, int32_t causal,
                                                int32_t has_rope, int32_t window_size, void* hip_stream) {
    std::string err;
    int rc = forward_f16_impl(q, k, v, output, rot_cos, rot_sin, q_stride_b, q_stride_h, q_stride_s, k_stride_b,
                              k_stride_h, k_stride_s, v_stride_b, v_stride_h, v_stride_s, o_stride_b, o_stride_h,
                              o_stride_s, batch_size, num_heads, num_kv_heads, seq_len, key_seq_len, head_dim,
                              scale, causal, has_rope, window_size, F16Path::Auto, hip_stream, err, true);
    if (rc != 0) {
        set_error("Attention (fp16) failed: %s", err);
        return -3;
    }
    return 0;
}

RDNA_API int32_t rdna_scratch_trim(void) {
    std::string err;
    if (rdna_amd::scratch_trim(err) != 0) {
        set_error("Scratch trim failed: %s", err);
        return -3;
    }
    return 0;
}

RDNA_API int32_t rdna_scratch_stats(int32_t device, uint64_t* cached_bytes, int64_t* entries,
                                    int64_t* allocations) {
    if (cached_bytes == nullptr || entries == nullptr || allocations == nullptr) {
        set_error("Scratch stats failed: %s", std::string("null output pointer"));
        return -3;
    }
    return rdna_amd::scratch_stats(device, *cached_bytes, *entries, *allocations);
}

RDNA_API int32_t rdna_attention_forward_path(const void* q, const void* k, const void* v, void* output,
                                             const void* rot_cos, const void* rot_sin, int64_t q_stride_b,
                                             int64_t q_stride_h, int64_t q_stride_s, int64_t k_stride_b,
                                             int64_t k_stride_h, int64_t k_stride_s, int64_t v_stride_b,
                                             int64_t v_stride_h, int64_t v_stride_s, int64_t o_stride_b,
                                             int64_t o_stride_h, int64_t o_stride_s, uint32_t batch_size,
                                             uint32_t num_heads, uint32_t num_kv_heads, uint32_t seq_len,
                                             uint32_t key_seq_len, uint32_t head_dim, float scale, int32_t causal,
                                             int32_t has_rope, int32_t window_size, int32_t path,
                                             void* hip_stream) {
    std::string err;
    int rc = forward_f16_impl(q, k, v, output, rot_cos, rot_sin, q_stride_b, q_stride_h, q_stride_s, k_stride_b,
                              k_stride_h, k_stride_s, v_stride_b, v_stride_h, v_stride_s, o_stride_b, o_stride_h,
                              o_stride_s, batch_size, num_heads, num_kv_heads, seq_len, key_seq_len, head_dim,
                              scale, causal, has_rope, window_size, static_cast<F16Path>(path), hip_stream, err);
    if (rc != 0) {
        set_error("Attention (fp16) failed: %s", err);
        return -3;
    }
    return 0;
}

RDNA_API int32_t rdna_attention_forward_int8qk(const void* q, const void* k, const void* v, void* output,
                                               int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
                                               int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s,
                                               int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s,
                                               int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_s,
                                               uint32_t batch_size, uint32_t num_heads, uint32_t num_kv_heads,
                                               uint32_t seq_len, uint32_t key_seq_len, uint32_t head_dim,
                                               float scale, float q_scale, float k_scale, float v_scale,
                                               const void* q_scale_vec, const void* k_scale_vec, int32_t causal,
                                               int32_t window_size, void* hip_stream) {
#if defined(RDNATTENTION_NO_INT8)
    (void)q, (void)k, (void)v, (void)output, (void)q_stride_b, (void)q_stride_h, (void)q_stride_s;
    (void)k_stride_b, (void)k_stride_h, (void)k_stride_s, (void)v_stride_b, (void)v_stride_h, (void)v_stride_s;
    (void)o_stride_b, (void)o_stride_h, (void)o_stride_s, (void)batch_size, (void)num_heads, (void)num_kv_heads;
    (void)seq_len, (void)key_seq_len, (void)head_dim, (void)scale, (void)q_scale, (void)k_scale, (void)v_scale;
    (void)q_scale_vec, (void)k_scale_vec, (void)causal, (void)window_size, (void)hip_stream;
    set_error("Attention (int8qk) unavailable: %s", kNoInt8);
    return -4;
#else
    std::string err;
    int rc = forward_i8_impl(q, k, v, output, q_stride_b, q_stride_h, q_stride_s, k_stride_b, k_stride_h, k_stride_s,
                             v_stride_b, v_stride_h, v_stride_s, o_stride_b, o_stride_h, o_stride_s, batch_size,
                             num_heads, num_kv_heads, seq_len, key_seq_len, head_dim, scale, q_scale, k_scale,
                             v_scale, q_scale_vec, k_scale_vec, nullptr, nullptr, causal, window_size, hip_stream, err);
    if (rc != 0) {
        set_error("Attention (int8qk) failed: %s", err);
        return -3;
    }
    return 0;
#endif
}

RDNA_API int32_t rdna_attention_forward_int8qk_vchannel(
    const void* q, const void* k, const void* v, void* output, int64_t q_stride_b, int64_t q_stride_h,
    int64_t q_stride_s, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s, int64_t v_stride_b,
    int64_t v_stride_h, int64_t v_stride_s, int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_s,
    uint32_t batch_size, uint32_t num_heads, uint32_t num_kv_heads, uint32_t seq_len, uint32_t key_seq_len,
    uint32_t head_dim, float scale, float q_scale, float k_scale, float v_scale, const void* q_scale_vec,
    const void* k_scale_vec, const void* v_channel_vec, int32_t causal, int32_t window_size, void* hip_stream) {
#if defined(RDNATTENTION_NO_INT8)
    (void)q, (void)k, (void)v, (void)output, (void)q_stride_b, (void)q_stride_h, (void)q_stride_s;
    (void)k_stride_b, (void)k_stride_h, (void)k_stride_s, (void)v_stride_b, (void)v_stride_h, (void)v_stride_s;
    (void)o_stride_b, (void)o_stride_h, (void)o_stride_s, (void)batch_size, (void)num_heads, (void)num_kv_heads;
    (void)seq_len, (void)key_seq_len, (void)head_dim, (void)scale, (void)q_scale, (void)k_scale, (void)v_scale;
    (void)q_scale_vec, (void)k_scale_vec, (void)v_channel_vec, (void)causal, (void)window_size, (void)hip_stream;
    set_error("Attention (int8qk) unavailable: %s", kNoInt8);
    return -4;
#else
    std::string err;
    int rc = forward_i8_impl(q, k, v, output, q_stride_b, q_stride_h, q_stride_s, k_stride_b, k_stride_h, k_stride_s,
                             v_stride_b, v_stride_h, v_stride_s, o_stride_b, o_stride_h, o_stride_s, batch_size,
                             num_heads, num_kv_heads, seq_len, key_seq_len, head_dim, scale, q_scale, k_scale,
                             v_scale, q_scale_vec, k_scale_vec, v_channel_vec, nullptr, causal, window_size,
                             hip_stream, err);
    if (rc != 0) {
        set_error("Attention (int8qk) failed: %s", err);
        return -3;
    }
    return 0;
#endif
}

RDNA_API int32_t rdna_attention_forward_int8qk_vtoken(
    const void* q, const void* k, const void* v, void* output, int64_t q_stride_b, int64_t q_stride_h,
    int64_t q_stride_s, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s, int64_t v_stride_b,
    int64_t v_stride_h, int64_t v_stride_s, int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_s,
    uint32_t batch_size, uint32_t num_heads, uint32_t num_kv_heads, uint32_t seq_len, uint32_t key_seq_len,
    uint32_t head_dim, float scale, float q_scale, float k_scale, float v_scale, const void* q_scale_vec,
    const void* k_scale_vec, const void* v_token_vec, int32_t causal, int32_t window_size, void* hip_stream) {
#if defined(RDNATTENTION_NO_INT8)
    (void)q, (void)k, (void)v, (void)output, (void)q_stride_b, (void)q_stride_h, (void)q_stride_s;
    (void)k_stride_b, (void)k_stride_h, (void)k_stride_s, (void)v_stride_b, (void)v_stride_h, (void)v_stride_s;
    (void)o_stride_b, (void)o_stride_h, (void)o_stride_s, (void)batch_size, (void)num_heads, (void)num_kv_heads;
    (void)seq_len, (void)key_seq_len, (void)head_dim, (void)scale, (void)q_scale, (void)k_scale, (void)v_scale;
    (void)q_scale_vec, (void)k_scale_vec, (void)v_token_vec, (void)causal, (void)window_size, (void)hip_stream;
    set_error("Attention (int8qk) unavailable: %s", kNoInt8);
    return -4;
#else
    if (v_token_vec == nullptr) {
        set_error("Attention (int8qk) failed: %s", std::string("v_token_vec is null"));
        return -3;
    }
    std::string err;
    int rc = forward_i8_impl(q, k, v, output, q_stride_b, q_stride_h, q_stride_s, k_stride_b, k_stride_h, k_stride_s,
                             v_stride_b, v_stride_h, v_stride_s, o_stride_b, o_stride_h, o_stride_s, batch_size,
                             num_heads, num_kv_heads, seq_len, key_seq_len, head_dim, scale, q_scale, k_scale,
                             v_scale, q_scale_vec, k_scale_vec, nullptr, v_token_vec, causal, window_size,
                             hip_stream, err);
    if (rc != 0) {
        set_error("Attention (int8qk) failed: %s", err);
        return -3;
    }
    return 0;
#endif
}

RDNA_API int32_t rdna_quantize_int8(const void* x, int32_t x_dtype, int64_t x_stride_b, int64_t x_stride_h,
                                    int64_t x_stride_s, uint32_t batch_size, uint32_t num_heads, uint32_t seq_len,
                                    uint32_t head_dim, int32_t per_channel, const void* rot_cos,
                                    const void* rot_sin, void* q_out, void* scale_out, void* hip_stream) {
    std::string err;
    const int64_t mult = x_dtype == 1 ? 4 : 8; // elements per 16 bytes
    if (x_dtype != 0 && x_dtype != 1) {
        err = "x_dtype must be 0 (fp16) or 1 (fp32)";
    } else if (head_dim < 8 || head_dim > 512 || head_dim % 8 != 0) {
        err = "head_dim must be a multiple of 8 from 8 to 512";
    } else if (batch_size == 0 || num_heads == 0 || seq_len == 0) {
        err = "empty tensor (batch_size, num_heads and seq_len must be non-zero)";
    } else if (seq_len > kMaxSeq || (uint64_t)batch_size * num_heads > (uint64_t)INT32_MAX / 2) {
        err = "tensor dimensions exceed the supported range";
    } else if (x == nullptr || q_out == nullptr || scale_out == nullptr) {
        err = "null tensor pointer";
    } else if (!aligned(x, 16) || !aligned(q_out, 16) || !aligned(scale_out, 4)) {
        err = "x and q_out must be 16-byte aligned, scale_out 4-byte aligned";
    } else if (x_stride_b % mult != 0 || x_stride_h % mult != 0 || x_stride_s % mult != 0) {
        err = "batch/head/seq strides of x must be multiples of 16 bytes";
    } else if ((rot_cos == nullptr) != (rot_sin == nullptr)) {
        err = "pass both rot_cos and rot_sin, or neither";
    } else if (rot_cos != nullptr && per_channel != 0) {
        err = "RoPE applies to the per-token scheme only";
    } else if (!aligned(rot_cos, 16) || !aligned(rot_sin, 16)) {
        err = "rot_cos and rot_sin must be 16-byte aligned";
    } else {
        rdna_amd::QuantArgs a;
        a.x = x;
        a.x_fp32 = x_dtype == 1 ? 1 : 0;
        a.xs[0] = x_stride_b, a.xs[1] = x_stride_h, a.xs[2] = x_stride_s;
        a.B = (int32_t)batch_size;
        a.H = (int32_t)num_heads;
        a.S = (int32_t)seq_len;
        a.D = (int32_t)head_dim;
        a.per_channel = per_channel != 0 ? 1 : 0;
        a.rot_cos = static_cast<const float*>(rot_cos);
        a.rot_sin = static_cast<const float*>(rot_sin);
        a.q = q_out;
        a.scale = static_cast<float*>(scale_out);
        if (rdna_amd::quantize_int8(a, static_cast<hipStream_t>(hip_stream), err) == 0) {
            return 0;
        }
    }
    set_error("Quantize (int8) failed: %s", err);
    return -3;
}

RDNA_API int32_t rdna_int8_qk_scores(const void* q, const void* k, int32_t* scores, int64_t q_stride_b,
                                     int64_t q_stride_h, int64_t q_stride_s, int64_t k_stride_b, int64_t k_stride_h,
                                     int64_t k_stride_s, uint32_t batch_size, uint32_t num_heads,
                                     uint32_t num_kv_heads, uint32_t seq_len, uint32_t key_seq_len,
                                     uint32_t head_dim, void* hip_stream) {
#if defined(RDNATTENTION_NO_INT8)
    (void)q, (void)k, (void)scores, (void)q_stride_b, (void)q_stride_h, (void)q_stride_s, (void)k_stride_b;
    (void)k_stride_h, (void)k_stride_s, (void)batch_size, (void)num_heads, (void)num_kv_heads, (void)seq_len;
    (void)key_seq_len, (void)head_dim, (void)hip_stream;
    set_error("Attention (int8qk) unavailable: %s", kNoInt8);
    return -4;
#else
    std::string err;
    AttnArgs a;
    a.q = q;
    a.k = k;
    a.v = k;
    a.o = scores;
    a.qs[0] = q_stride_b, a.qs[1] = q_stride_h, a.qs[2] = q_stride_s;
    a.ks[0] = k_stride_b, a.ks[1] = k_stride_h, a.ks[2] = k_stride_s;
    a.vs[0] = k_stride_b, a.vs[1] = k_stride_h, a.vs[2] = k_stride_s;
    if (num_kv_heads == 0 || num_heads % num_kv_heads != 0) {
        err = "numHeads must be a positive multiple of numKvHeads";
    } else if (head_dim != 64 && head_dim != 128) {
        err = "unsupported head_dim (only 64 and 128 are compiled in for the int8 kernel)";
    } else {
        err = check_common(a, batch_size, num_heads, num_kv_heads, seq_len, key_seq_len, 16);
    }
    if (err.empty() && key_seq_len == 0) {
        err = "key_seq_len must be non-zero";
    }
    if (err.empty()) {
        a.B = (int32_t)batch_size;
        a.Hq = (int32_t)num_heads;
        a.Hkv = (int32_t)num_kv_heads;
        a.Sq = (int32_t)seq_len;
        a.Sk = (int32_t)key_seq_len;
        a.D = (int32_t)head_dim;
        if (rdna_amd::int8_scores(a, scores, static_cast<hipStream_t>(hip_stream), err) == 0) {
            return 0;
        }
    }
    set_error("Attention (int8qk) failed: %s", err);
    return -3;
#endif
}

// ---------------------------------------------------------------------------
// C++ launch API (reference: src/rdna/fa2_forward_f16.hpp, fa2_forward_int8qk.hpp)
// ---------------------------------------------------------------------------
namespace rdna {

int forwardF16(const ForwardParams& p, void* stream) {
    std::string err;
    int rc = forward_f16_impl(p.q, p.k, p.v, p.o, p.rot_cos, p.rot_sin, p.qStrideB, p.qStrideH, p.qStrideS,
                              p.kStrideB, p.kStrideH, p.kStrideS, p.vStrideB, p.vStrideH, p.vStrideS, p.oStrideB,
                              p.oStrideH, p.oStrideS, p.batchSize, p.numHeads, p.numKvHeads, p.seqLen, p.keySeqLen,
                              p.headDim, p.scale, (int32_t)p.causal, (int32_t)p.hasRope, p.windowSize, F16Path::Auto,
                              stream, err);
    if (rc != 0) {
        std::snprintf(g_last_f16, sizeof(g_last_f16), "%s", err.c_str());
        return -1;
    }
    return 0;
}

const char* lastError() {
    return g_last_f16[0] != '\0' ? g_last_f16 : nullptr;
}

bool hasDevice() {
    int count = 0;
    return hipGetDeviceCount(&count) == hipSuccess && count > 0;
}

int forwardInt8QK(const ForwardParamsInt8QK& p, void* stream) {
    std::string err;
    int rc = forward_i8_impl(p.q, p.k, p.v, p.o, p.qStrideB, p.qStrideH, p.qStrideS, p.kStrideB, p.kStrideH,
                             p.kStrideS, p.vStrideB, p.vStrideH, p.vStrideS, p.oStrideB, p.oStrideH, p.oStrideS,
                             p.batchSize, p.numHeads, p.numKvHeads, p.seqLen, p.keySeqLen, p.headDim, p.scale,
                             p.qScale, p.kScale, p.vScale, p.qScaleVec, p.kScaleVec, nullptr, nullptr,
                             (int32_t)p.causal, p.windowSize, stream, err);
    if (rc != 0) {
        std::snprintf(g_last_i8, sizeof(g_last_i8), "%s", err.c_str());
        return -1;
    }
    return 0;
}

const char* lastErrorInt8QK() {
    return g_last_i8[0] != '\0' ? g_last_i8 : nullptr;
}

} // namespace rdna
