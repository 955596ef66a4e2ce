/*
 * rdnattention.h -- C ABI of librdnattention.so (gfx950 / MI355X build).
 *
 * Drop-in for the reference's C ABI (dmonkman/RDNAttention src/c_api.hpp):
 * the same four symbols, argument lists, return codes and thread-local error
 * string.  Every function works on caller-owned HIP device memory (a torch
 * tensor's data_ptr(), a hipMalloc'd buffer); launches are asynchronous on
 * the caller's stream.
 *
 * Return codes: 0 = success; -3 = rejected arguments or launch failure
 * (detail in rdna_get_error()); -4 = INT8 entry point in a library built
 * without the INT8 kernel.  All argument checks run before any HIP call, so
 * every error path is reachable without a GPU.
 */
#ifndef RDNATTENTION_H
#define RDNATTENTION_H

#include <stdint.h>

#ifdef __cplusplus
#define RDNA_EXTERN_C extern "C"
#else
#define RDNA_EXTERN_C
#endif
#define RDNA_API RDNA_EXTERN_C __attribute__((visibility("default")))

/* 1 if a HIP device is visible, else 0.
 * Replaces src/c_api.hpp:16 (rdna_has_device). */
RDNA_API int32_t rdna_has_device(void);

/* Reason the most recent failing call on this thread failed, or "" if none
 * ever did.  Never cleared by a successful call.
 * Replaces src/c_api.hpp:18-19 (rdna_get_error). */
RDNA_API const char* rdna_get_error(void);

/* FP16 forward attention: O = softmax(scale * Q K^T + mask) V.
 * Q/K/V/output: _Float16, head_dim contiguous; *_stride_b/h/s are strides in
 * ELEMENTS for the batch/head/seq axes.  head_dim is any multiple of 32 from
 * 32 to 512.  num_kv_heads must divide num_heads (GQA/MQA when smaller).
 * rot_cos/rot_sin (has_rope != 0): contiguous float [max(seq_len,
 * key_seq_len), head_dim/2], shared across batch and heads, row = position
 * within the tensor; channels 2i and 2i+1 rotate by column i.
 * causal: key k visible to query q iff k <= q + (key_seq_len - seq_len).
 * window_size > 0: causal -> the window_size keys ending at q + delta;
 * non-causal -> |q + delta - k| <= window_size / 2.  <= 0 disables it.
 * Rows that see no key are written as 0.
 * This build additionally requires 16-byte aligned base pointers and strides
 * that are multiples of 8 elements (the reference assumed this silently).
 * hip_stream: hipStream_t as void*, NULL = the null stream.
 * Replaces src/c_api.hpp:36-57 (rdna_attention_forward). */
RDNA_API int32_t rdna_attention_forward(
    const void* q, const void* k, const void* v, void* output,
    const void* rot_cos, const void* rot_sin,
    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
    int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s,
    int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s,
    int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_s,
    uint32_t batch_size, uint32_t num_heads, uint32_t num_kv_heads,
    uint32_t seq_len, uint32_t key_seq_len, uint32_t head_dim,
    float scale, int32_t causal, int32_t has_rope, int32_t window_size,
    void* hip_stream);

/* INT8 forward attention, both GEMMs in int8 (int32 accumulation), fp16 out.
 * Q/K/V: int8, head_dim 64 or 128, strides in elements (multiples of 16 in
 * this build).  Dequant: value = int8 * scale.  q_scale_vec (optional) is a
 * contiguous float [batch, num_heads, seq_len] of per-token Q scales,
 * k_scale_vec (optional) [batch, num_kv_heads, key_seq_len]; NULL selects
 * the scalar q_scale / k_scale.  v_scale is per tensor.  P is quantised per
 * 64-key block against the running row max: min(127, lround(p * 127)); the
 * softmax denominator uses the unquantised p.  No RoPE.
 * Replaces src/c_api.hpp:64-87 (rdna_attention_forward_int8qk). */
RDNA_API int32_t rdna_attention_forward_int8qk(
    const void* q, const void* k, const void* v, void* output,
    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
    int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s,
    int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s,
    int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_s,
    uint32_t batch_size, uint32_t num_heads, uint32_t num_kv_heads,
    uint32_t seq_len, uint32_t key_seq_len, uint32_t head_dim,
    float scale, float q_scale, float k_scale, float v_scale,
    const void* q_scale_vec, const void* k_scale_vec,
    int32_t causal, int32_t window_size, void* hip_stream);

#endif /* RDNATTENTION_H */
