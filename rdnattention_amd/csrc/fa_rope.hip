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

// Grid (row blocks, heads): block x is a run of kRopeRows rows, block y walks
// the (b, h) pairs y, y + gridDim.y, ...; each thread rotates the 16-byte
// chunks of one column (D / 8 threads per row), row after row, with no
// division per chunk.  A flat index with three 64-bit divisions per chunk ran
// at 5.8 TB/s.
constexpr int kRopeThreads = 256;
constexpr int kRopeRows = 64;

__global__ __launch_bounds__(kRopeThreads) void rope_rotate_rows(const _Float16* __restrict__ src,
                                                                 _Float16* __restrict__ dst,
                                                                 const float* __restrict__ cos_t,
                                                                 const float* __restrict__ sin_t, int64_t sb,
                                                                 int64_t sh, int64_t ss, int32_t H, int32_t S,
                                                                 int32_t D, int64_t heads) {
    const int cpr = D / 8;                 // chunks per row
    const int rpp = kRopeThreads / cpr;    // rows per pass (D <= 512: cpr <= 64)
    const int ch = threadIdx.x % cpr;
    const int r0 = threadIdx.x / cpr;
    if (r0 >= rpp) {
        return; // D / 8 does not divide the block (D = 96, 160, ...)
    }
    const int half = D / 2;
    const int row_end = min(S, (int)(blockIdx.x + 1) * kRopeRows);
    for (int64_t bh = blockIdx.y; bh < heads; bh += gridDim.y) {
        const int64_t b = bh / H, h = bh - (bh / H) * H;
        const _Float16* sp = src + b * sb + h * sh + 8 * ch;
        _Float16* dp = dst + bh * S * D + 8 * ch;
        for (int s = (int)blockIdx.x * kRopeRows + r0; s < row_end; s += rpp) {
            h8 x = *reinterpret_cast<const h8*>(sp + (int64_t)s * ss);
            x = rope8(x, cos_t + (int64_t)s * half, sin_t + (int64_t)s * half, 4 * ch);
            __builtin_nontemporal_store(x, reinterpret_cast<h8*>(dp + (int64_t)s * D));
        }
    }
}

} // namespace

int rope_rotate_k(const AttnArgs& a, void* dst, hipStream_t stream, std::string& err) {
    const int64_t heads = (int64_t)a.B * a.Hkv;
    if (heads == 0 || a.Sk == 0) {
        return 0;
    }
    const uint32_t row_blocks = (uint32_t)((a.Sk + kRopeRows - 1) / kRopeRows);
    const uint32_t head_blocks = (uint32_t)(heads < 65535 ? heads : 65535);
    hipLaunchKernelGGL(rope_rotate_rows, dim3(row_blocks, head_blocks), dim3(kRopeThreads), 0, stream,
                       static_cast<const _Float16*>(a.k), static_cast<_Float16*>(dst), a.rot_cos, a.rot_sin,
                       a.ks[0], a.ks[1], a.ks[2], a.Hkv, a.Sk, a.D, heads);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

} // namespace rdna_amd
