// RoPE pre-rotation of K.
//
// The reference rotates every K tile inside the attention loop
// (src/rdna/fa2_forward_f16.hip:256), i.e. once per query row tile that
// reads it.  Here K is rotated exactly once, by a streaming kernel, into a
// contiguous [B, Hkv, Sk, D] scratch tensor with the same arithmetic (fp32
// rotation of interleaved pairs, rounded to fp16), and the attention kernels
// read the rotated copy: the result is identical and the inner loop carries no
// table loads.
#include "fa_common.hpp"
#include "fa_host.hpp"
#include "fa_internal.hpp"

#include <cstdint>

namespace rdna_amd {
namespace {

__global__ __launch_bounds__(256) void rope_rotate_rows(const _Float16* __restrict__ src, _Float16* __restrict__ dst,
                                                        const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t, int64_t sb, int64_t sh,
                                                        int64_t ss, int32_t H, int32_t S, int32_t D,
                                                        int64_t n_chunks) {
    const int chunks_per_row = D / 8;
    const int half = D / 2;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n_chunks;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = e / chunks_per_row;
        const int ch = (int)(e - row * chunks_per_row);
        const int64_t bh = row / S;
        const int s = (int)(row - bh * S);
        const int64_t b = bh / H;
        const int h = (int)(bh - b * H);
        h8 x = *reinterpret_cast<const h8*>(src + b * sb + h * sh + s * ss + 8 * ch);
        x = rope8(x, cos_t + (int64_t)s * half, sin_t + (int64_t)s * half, 4 * ch);
        *reinterpret_cast<h8*>(dst + row * D + 8 * ch) = x;
    }
}

} // namespace

int rope_rotate_k(const AttnArgs& a, void* dst, hipStream_t stream, std::string& err) {
    const int64_t n_chunks = (int64_t)a.B * a.Hkv * a.Sk * (a.D / 8);
    if (n_chunks == 0) {
        return 0;
    }
    const int64_t blocks64 = (n_chunks + 255) / 256;
    const uint32_t blocks = (uint32_t)(blocks64 < 65536 ? blocks64 : 65536);
    hipLaunchKernelGGL(rope_rotate_rows, dim3(blocks), dim3(256), 0, stream, static_cast<const _Float16*>(a.k),
                       static_cast<_Float16*>(dst), a.rot_cos, a.rot_sin, a.ks[0], a.ks[1], a.ks[2], a.Hkv, a.Sk, a.D,
                       n_chunks);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

} // namespace rdna_amd
