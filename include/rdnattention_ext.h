/*
 * rdnattention_ext.h -- entry points of librdnattention.so that have no
 * counterpart in the reference's C ABI.  They exist for testing and
 * measurement; the four drop-in symbols in rdnattention.h do not depend on
 * them.  Same return-code and error-string conventions as rdnattention.h.
 */
#ifndef RDNATTENTION_EXT_H
#define RDNATTENTION_EXT_H

#include "rdnattention.h"

/* Kernel path for rdna_attention_forward_path(). */
#define RDNA_PATH_AUTO 0    /* what rdna_attention_forward() picks */
#define RDNA_PATH_PREFILL 1 /* tiled prefill kernel */
#define RDNA_PATH_SPLITK 2  /* split-K decode kernel + combine */

/* rdna_attention_forward() with the kernel path forced, so tests can run the
 * prefill and split-K kernels on the same input.  No reference counterpart:
 * for parity tests and benchmarks. */
RDNA_API int32_t rdna_attention_forward_path(
    const void* q, const void* k, const void* v, void* output,
    const void* rot_cos, const void* rot_sin,
    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
    int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s,
    int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s,
    int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_s,
    uint32_t batch_size, uint32_t num_heads, uint32_t num_kv_heads,
    uint32_t seq_len, uint32_t key_seq_len, uint32_t head_dim,
    float scale, int32_t causal, int32_t has_rope, int32_t window_size,
    int32_t path, void* hip_stream);

/* Releases the device memory the library keeps for reuse: the scratch
 * buffers (RoPE-rotated K copies, split-K partials, quantiser partials) it
 * caches per (device, stream, use), grown to the largest call so far (at most
 * 256 MiB each, at most 1 GiB per device over all streams and uses), and the
 * free blocks of the devices' default memory pools.  A call never frees or
 * allocates scratch on the host's time: a cached buffer large enough is
 * reused with no allocator call; growth and eviction are stream-ordered
 * (hipFreeAsync / hipMallocAsync).  This trim is the one synchronising path:
 * it waits for each buffer's last use and for its device; a buffer a call is
 * using at that moment is kept.  No reference counterpart (the reference
 * allocates nothing).  Returns 0, or -3 with rdna_get_error() set. */
RDNA_API int32_t rdna_scratch_trim(void);

/* The scratch cache of HIP device `device`: bytes it holds, buffers it holds,
 * and the allocator calls (hipMallocAsync) the library has made for that
 * device's scratch since it was loaded.  For tests and monitoring; no
 * reference counterpart.  Returns 0, or -3 if an output pointer is null. */
RDNA_API int32_t rdna_scratch_stats(int32_t device, uint64_t* cached_bytes, int64_t* entries,
                                    int64_t* allocations);

/* rdna_attention_forward() for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No reference counterpart: the reference needs no scratch.
 * Same arguments, results and return codes as rdna_attention_forward(); the
 * scratch that path takes -- the RoPE-rotated K copy (B*Hkv*Sk*D fp16) and
 * the split-K decode partials -- comes from a static 64 MiB device array the
 * library holds on each GPU it runs on, so the call makes no hipMalloc,
 * hipFree or pool allocation.  A call needing more than 64 MiB of scratch
 * returns -3 ("... bytes of scratch ...") before launching anything.  Every
 * call on one GPU shares that GPU's array: calls that overlap on a GPU
 * (different streams, not ordered) race. */
RDNA_API int32_t rdna_attention_forward_noalloc(
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

/* Exact int32 scores S = Q_i8 K_i8^T (GQA head map kv = h / (Hq/Hkv)),
 * written to `scores`, a contiguous int32 [batch, num_heads, seq_len,
 * key_seq_len] device buffer.  Runs the INT8 attention kernel itself (its
 * score-export instantiation: the same K tile staging, LDS layout, operand
 * ring and v_mfma_i32_32x32x32_i8 sequence as rdna_attention_forward_int8qk's
 * first GEMM) and writes its accumulators; softmax, P V and output are
 * compiled out.  Key and query strides as for the forward (seq strides
 * <= 2^24 elements).  No reference counterpart: it exposes the production
 * kernel's scores so tests can check them bit for bit. */
RDNA_API int32_t rdna_int8_qk_scores(
    const void* q, const void* k, int32_t* scores,
    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
    int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s,
    uint32_t batch_size, uint32_t num_heads, uint32_t num_kv_heads,
    uint32_t seq_len, uint32_t key_seq_len, uint32_t head_dim,
    void* hip_stream);

/* rdna_attention_forward_int8qk() with a per-channel V scale applied inside
 * the kernel: output = softmax-weighted sum of v_i8 * v_scale *
 * v_channel_vec[b, kv_head, d], where v_channel_vec is a contiguous fp32
 * [batch, num_kv_heads, head_dim] device array (16-byte aligned), or null for
 * the plain per-tensor v_scale.  No reference counterpart: the reference's
 * flash_attn_int8qk_quantized (rdnattention/__init__.py:346-357) multiplies
 * the kernel's fp16 output by v_channel in a separate torch pass; here that
 * product is part of the kernel's epilogue. */
RDNA_API int32_t rdna_attention_forward_int8qk_vchannel(
    const void* q, const void* k, const void* v, void* output,
    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
    int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s,
    int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s,
    int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_s,
    uint32_t batch_size, uint32_t num_heads, uint32_t num_kv_heads,
    uint32_t seq_len, uint32_t key_seq_len, uint32_t head_dim,
    float scale, float q_scale, float k_scale, float v_scale,
    const void* q_scale_vec, const void* k_scale_vec, const void* v_channel_vec,
    int32_t causal, int32_t window_size, void* hip_stream);

/* rdna_attention_forward_int8qk() with a per-token V scale: V row j of each
 * (batch, kv head) is dequantised by v_token_vec[b, kv_head, j] while the
 * kernel stages it, v'_j = fp16(sat(v_i8[j] * v_token_vec[...])) (the product
 * in fp32, saturated to +-65504, rounded once to fp16), and the
 * quantised P (the reference's pq = min(127, round(127 p))) multiplies these
 * fp16 rows: output = sum_j pq_j v'_j * v_scale / (127 l).  v_token_vec is a
 * contiguous fp32 [batch, num_kv_heads, key_seq_len] device array (4-byte
 * aligned, required).  No reference counterpart: the reference lists a
 * per-token V scale as missing (FEATURES.md:191, :201-202); this is the extension
 * that fills it, with the per-token V quantiser of
 * quantize_int8_qk_pertoken's formula. */
RDNA_API int32_t rdna_attention_forward_int8qk_vtoken(
    const void* q, const void* k, const void* v, void* output,
    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
    int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s,
    int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s,
    int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_s,
    uint32_t batch_size, uint32_t num_heads, uint32_t num_kv_heads,
    uint32_t seq_len, uint32_t key_seq_len, uint32_t head_dim,
    float scale, float q_scale, float k_scale, float v_scale,
    const void* q_scale_vec, const void* k_scale_vec, const void* v_token_vec,
    int32_t causal, int32_t window_size, void* hip_stream);

/* INT8 quantisation on the GPU, bit-identical to the reference wrapper's
 * torch ops (rdnattention/__init__.py:303-343):
 *   per_channel == 0 (per token): scale[b,h,s] = max_d |x| / 127 (0 -> 1)
 *   per_channel != 0 (per channel): scale[b,h,d] = max_s |x| / 127 (0 -> 1)
 *   q = clamp(round_half_even(x / scale), -127, 127)
 * x: fp16 (x_dtype 0) or fp32 (x_dtype 1) [batch, num_heads, seq_len,
 * head_dim] with element strides (b, h, s) and unit stride along head_dim;
 * 16-byte aligned, strides multiples of 16 bytes; head_dim a multiple of 8
 * up to 512.  q_out: int8 [batch, num_heads, seq_len, head_dim] contiguous;
 * scale_out: fp32, [batch, num_heads, seq_len] or [batch, num_heads,
 * head_dim], contiguous.
 * rot_cos / rot_sin (per token only; both or neither, nullptr = none): fp32
 * RoPE tables [>= seq_len, head_dim / 2], contiguous, 16-byte aligned, as
 * for rdna_attention_forward.  Each row (position s) is rotated first, with
 * the FP16 attention path's arithmetic (pairs rotated in fp32, rounded to
 * fp16 for fp16 input), and the rotated row is quantised: INT8 attention
 * with RoPE, which the reference does not offer.
 * Returns 0, or -3 with "Quantize (int8) failed: ...".
 * No reference counterpart (the reference quantises with torch ops). */
RDNA_API int32_t rdna_quantize_int8(
    const void* x, int32_t x_dtype,
    int64_t x_stride_b, int64_t x_stride_h, int64_t x_stride_s,
    uint32_t batch_size, uint32_t num_heads, uint32_t seq_len, uint32_t head_dim,
    int32_t per_channel, const void* rot_cos, const void* rot_sin,
    void* q_out, void* scale_out, void* hip_stream);

/* Kernel timer.  While enabled, each launch of a main attention kernel
 * (prefill, split-K, int8; not the RoPE pre-rotation or split-K combine
 * kernels) is bracketed by a HIP event pair recorded on its stream.
 * rdna_kernel_timer_enable(on) discards what was recorded and switches the
 * timer on (on != 0) or off.  rdna_kernel_timer_read waits for the recorded
 * events, stores the summed kernel time in *total_ms and the number of timed
 * launches in *launches, and clears the record; returns -3 if an event could
 * not be created, recorded or read.  Process-wide; no reference counterpart:
 * benchmarks use it to divide a kernel's FLOPs or bytes by its own time. */
RDNA_API int32_t rdna_kernel_timer_enable(int32_t on);
RDNA_API int32_t rdna_kernel_timer_read(double* total_ms, int64_t* launches);

/* Library version string ("0.1.0-gfx950"). */
RDNA_API const char* rdna_version(void);

#endif /* RDNATTENTION_EXT_H */
