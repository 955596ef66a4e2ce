// INT8 quantisers on the GPU: the two schemes of the reference's Python
// wrapper (rdnattention/__init__.py:303-343), computed with the fp32
// arithmetic of torch's GPU kernels so the results are bit-identical:
//
//   per token (rows):       s = amax_d |x| / 127 (0 -> 1), q = clamp(rne(x / s), -127, 127)
//   per channel (columns):  s_d = amax_seq |x_d| / 127 (0 -> 1), q = clamp(rne(x / s_d), -127, 127)
//
// x is fp16 or fp32 [B, H, S, D] with element strides (b, h, s) and unit
// stride along D; q is int8 [B, H, S, D] contiguous; scales are fp32,
// [B, H, S] (rows) or [B, H, D] (columns), contiguous.
//
// Bit-exactness follows torch's GPU kernels: amax / 127.0 (a tensor divided
// by a Python scalar) is computed as amax * fp32(1/127), one rounding each,
// while x / s (tensor by tensor) is an IEEE fp32 division; rounding is
// round-half-to-even like torch.round.  (torch on the CPU divides amax by 127
// instead, which can differ in the last bit of the scale.)
//
// The per-token scheme can rotate the rows first (RoPE with the attention
// kernels' tables and arithmetic: interleaved pairs rotated in fp32 and, for
// fp16 input, rounded to fp16 exactly as the FP16 path rotates Q and K), so
// that INT8 attention with RoPE quantises the rotated Q and K in one pass.
// The reference has no INT8 RoPE.
//
// These kernels are HBM-bound streaming passes (read x once, write q once; the
// per-channel scheme reads x twice: column maxima, then quantisation).
#include "fa_common.hpp"
#include "fa_host.hpp"
#include "fa_internal.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace rdna_amd {
namespace {

constexpr int kQThreads = 256;
constexpr float kInv127 = 1.0f / 127.0f; // torch: scalar divisor -> reciprocal multiply

// 8 consecutive elements of x as fp32
template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
    if constexpr (sizeof(T) == 2) {
        const h8 x = *reinterpret_cast<const h8*>(p);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            v[e] = (float)x[e];
        }
    } else {
        typedef float f4 __attribute__((ext_vector_type(4)));
        const f4 a = *reinterpret_cast<const f4*>(p);
        const f4 b = *reinterpret_cast<const f4*>(p + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[e] = a[e];
            v[4 + e] = b[e];
        }
    }
}

__device__ __forceinline__ int8_t quant1(float x, float s) {
    const float r = rintf(x / s);
    return (int8_t)fminf(fmaxf(r, -127.0f), 127.0f);
}

__device__ __forceinline__ void store8(int8_t* p, const float (&v)[8], float s) {
    typedef int8_t i8x8_t __attribute__((ext_vector_type(8)));
    i8x8_t o;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        o[e] = quant1(v[e], s);
    }
    *reinterpret_cast<i8x8_t*>(p) = o;
}

// RoPE of the 8-element chunk `sub` of a row at position s (tables
// [positions, D/2] fp32): the pairs rotated in fp32 (rope8_cs, the FP16
// kernels' arithmetic), rounded to fp16 for fp16 input.
template <typename T>
__device__ __forceinline__ void rope_chunk(float (&v)[8], const float* cos_t, const float* sin_t, int s, int D,
                                           int sub) {
    const f4 c = *reinterpret_cast<const f4*>(cos_t + (int64_t)s * (D / 2) + 4 * sub);
    const f4 sn = *reinterpret_cast<const f4*>(sin_t + (int64_t)s * (D / 2) + 4 * sub);
    if constexpr (sizeof(T) == 2) {
        h8 x;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            x[e] = (_Float16)v[e]; // exact: v holds fp16 values
        }
        const h8 y = rope8_cs(x, c, sn);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            v[e] = (float)y[e];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float a = v[2 * i];
            const float b = v[2 * i + 1];
            v[2 * i] = a * c[i] - b * sn[i];
            v[2 * i + 1] = a * sn[i] + b * c[i];
        }
    }
}

// Per-token: LPR lanes (a power of two >= D/8) per row, each holding one
// 8-element chunk; 256 / LPR rows per block iteration, grid-stride over rows.
// With rot_cos (and rot_sin) the rows are rotated by RoPE before quantisation.
template <typename T, int LPR>
__global__ __launch_bounds__(kQThreads) void quant_rows_kernel(const T* __restrict__ x, int8_t* __restrict__ q,
                                                               float* __restrict__ scale,
                                                               const float* __restrict__ rot_cos,
                                                               const float* __restrict__ rot_sin, int64_t sb,
                                                               int64_t sh, int64_t ss, int32_t H, int32_t S,
                                                               int32_t D, int64_t n_rows) {
    constexpr int RPB = kQThreads / LPR; // rows per block iteration
    const int tid = threadIdx.x;
    const int sub = tid % LPR;
    const int ch = D / 8;
    for (int64_t row = (int64_t)blockIdx.x * RPB + tid / LPR; row - tid / LPR < n_rows;
         row += (int64_t)gridDim.x * RPB) {
        const bool row_ok = row < n_rows;
        const bool active = row_ok && sub < ch;
        float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (active) {
            const int64_t bh = row / S;
            const int s = (int)(row - bh * S);
            const int64_t b = bh / H;
            const int h = (int)(bh - b * H);
            load8(x + b * sb + h * sh + (int64_t)s * ss + 8 * sub, v);
            if (rot_cos != nullptr) {
                rope_chunk<T>(v, rot_cos, rot_sin, s, D, sub);
            }
        }
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            m = fmaxf(m, fabsf(v[e]));
        }
#pragma unroll
        for (int off = LPR / 2; off > 0; off >>= 1) {
            m = fmaxf(m, __shfl_xor(m, off, LPR));
        }
        float s = m * kInv127;
        s = (s == 0.0f) ? 1.0f : s;
        if (active) {
            store8(q + row * D + 8 * sub, v, s);
        }
        if (row_ok && sub == 0) {
            scale[row] = s;
        }
    }
}

// Per-channel, pass 1: column maxima of one chunk of rows of one (b, h):
// thread (c, r) covers chunk c of the row and rows r, r + RL, ...; partial
// maxima go to part[bh][chunk][D].
template <typename T>
__global__ __launch_bounds__(kQThreads) void col_max_kernel(const T* __restrict__ x, float* __restrict__ part,
                                                            int64_t sb, int64_t sh, int64_t ss, int32_t H,
                                                            int32_t S, int32_t D, int32_t rows_per_chunk) {
    __shared__ float red[kQThreads * 8];
    const int tid = threadIdx.x;
    const int ch = D / 8;
    const int rl = kQThreads / ch; // row lanes (D/8 divides 256 for D in {8, 16, ..., 256}; else a remainder idles)
    const int c = tid % ch;
    const int r = tid / ch;
    const int chunk = blockIdx.x;
    const int bh = blockIdx.y;
    const int b = bh / H, h = bh - b * H;
    const int s0 = chunk * rows_per_chunk;
    const int s1 = min(s0 + rows_per_chunk, S);
    float m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (r < rl) {
        const T* base = x + (int64_t)b * sb + (int64_t)h * sh + 8 * c;
        for (int s = s0 + r; s < s1; s += rl) {
            float v[8];
            load8(base + (int64_t)s * ss, v);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                m[e] = fmaxf(m[e], fabsf(v[e]));
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 8; e++) {
        red[tid * 8 + e] = m[e];
    }
    __syncthreads();
    // column d = 8 c + e: max over the row lanes
    for (int d = tid; d < D; d += kQThreads) {
        const int cc = d >> 3, e = d & 7;
        float mm = 0.0f;
        for (int rr = 0; rr < rl; rr++) {
            mm = fmaxf(mm, red[(rr * ch + cc) * 8 + e]);
        }
        part[((int64_t)bh * gridDim.x + chunk) * D + d] = mm;
    }
}

// Per-channel, pass 2: channel scales from the partial maxima (written once
// per (b, h) by chunk 0), then quantisation of this chunk's rows.
template <typename T>
__global__ __launch_bounds__(kQThreads) void quant_cols_kernel(const T* __restrict__ x, const float* __restrict__ part,
                                                               int8_t* __restrict__ q, float* __restrict__ cscale,
                                                               int64_t sb, int64_t sh, int64_t ss, int32_t H,
                                                               int32_t S, int32_t D, int32_t rows_per_chunk,
                                                               int32_t n_chunks) {
    __shared__ float sc[512];
    const int tid = threadIdx.x;
    const int chunk = blockIdx.x;
    const int bh = blockIdx.y;
    const int b = bh / H, h = bh - b * H;
    for (int d = tid; d < D; d += kQThreads) {
        float mm = 0.0f;
        for (int k = 0; k < n_chunks; k++) {
            mm = fmaxf(mm, part[((int64_t)bh * n_chunks + k) * D + d]);
        }
        float s = mm * kInv127;
        s = (s == 0.0f) ? 1.0f : s;
        sc[d] = s;
        if (chunk == 0) {
            cscale[(int64_t)bh * D + d] = s;
        }
    }
    __syncthreads();
    const int ch = D / 8;
    const int s0 = chunk * rows_per_chunk;
    const int s1 = min(s0 + rows_per_chunk, S);
    const int64_t n = (int64_t)(s1 - s0) * ch;
    const T* base = x + (int64_t)b * sb + (int64_t)h * sh;
    int8_t* qbase = q + (int64_t)bh * S * D;
    for (int64_t e = tid; e < n; e += kQThreads) {
        const int rr = (int)(e / ch);
        const int c = (int)(e - (int64_t)rr * ch);
        const int s = s0 + rr;
        float v[8];
        load8(base + (int64_t)s * ss + 8 * c, v);
        typedef int8_t i8x8_t __attribute__((ext_vector_type(8)));
        i8x8_t o;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            o[k] = quant1(v[k], sc[8 * c + k]);
        }
        *reinterpret_cast<i8x8_t*>(qbase + (int64_t)s * D + 8 * c) = o;
    }
}

template <typename T>
int launch_rows(const QuantArgs& a, hipStream_t stream) {
    const int ch = a.D / 8;
    const int64_t n_rows = (int64_t)a.B * a.H * a.S;
    auto go = [&](auto lpr_c) {
        constexpr int LPR = decltype(lpr_c)::value;
        constexpr int RPB = kQThreads / LPR;
        const int64_t blocks = std::min<int64_t>((n_rows + RPB - 1) / RPB, 65536);
        hipLaunchKernelGGL((quant_rows_kernel<T, LPR>), dim3((uint32_t)blocks), dim3(kQThreads), 0, stream,
                           static_cast<const T*>(a.x), static_cast<int8_t*>(a.q), a.scale, a.rot_cos, a.rot_sin,
                           a.xs[0], a.xs[1], a.xs[2], a.H, a.S, a.D, n_rows);
    };
    if (ch <= 4) {
        go(std::integral_constant<int, 4>{});
    } else if (ch <= 8) {
        go(std::integral_constant<int, 8>{});
    } else if (ch <= 16) {
        go(std::integral_constant<int, 16>{});
    } else if (ch <= 32) {
        go(std::integral_constant<int, 32>{});
    } else {
        go(std::integral_constant<int, 64>{});
    }
    return 0;
}

template <typename T>
int launch_cols(const QuantArgs& a, hipStream_t stream, std::string& err) {
    const int64_t n_bh = (int64_t)a.B * a.H;
    // about 4 chunks of rows per CU in total, at least 64 rows per chunk
    const int64_t want = std::max<int64_t>(1, 1024 / std::max<int64_t>(1, n_bh));
    int rows_per_chunk = (int)std::max<int64_t>(64, ((int64_t)a.S + want - 1) / want);
    const int n_chunks = (a.S + rows_per_chunk - 1) / rows_per_chunk;
    StreamScratch part(ScratchUse::QuantPartials);
    if (part.alloc((size_t)n_bh * n_chunks * a.D * sizeof(float), stream, err) != 0) {
        return -1;
    }
    const dim3 grid((uint32_t)n_chunks, (uint32_t)n_bh);
    hipLaunchKernelGGL(col_max_kernel<T>, grid, dim3(kQThreads), 0, stream, static_cast<const T*>(a.x),
                       static_cast<float*>(part.ptr), a.xs[0], a.xs[1], a.xs[2], a.H, a.S, a.D, rows_per_chunk);
    hipLaunchKernelGGL(quant_cols_kernel<T>, grid, dim3(kQThreads), 0, stream, static_cast<const T*>(a.x),
                       static_cast<const float*>(part.ptr), static_cast<int8_t*>(a.q), a.scale, a.xs[0], a.xs[1],
                       a.xs[2], a.H, a.S, a.D, rows_per_chunk, n_chunks);
    return 0;
}

} // namespace

int quantize_int8(const QuantArgs& a, hipStream_t stream, std::string& err) {
    int rc;
    if (a.per_channel && a.rot_cos != nullptr) {
        err = "RoPE applies to the per-token scheme only";
        return -1;
    }
    if (a.per_channel) {
        rc = a.x_fp32 ? launch_cols<float>(a, stream, err) : launch_cols<_Float16>(a, stream, err);
    } else {
        rc = a.x_fp32 ? launch_rows<float>(a, stream) : launch_rows<_Float16>(a, stream);
    }
    if (rc != 0) {
        return rc;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

} // namespace rdna_amd
