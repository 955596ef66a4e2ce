// A C++ caller of the rdna:: launch API (include/rdnattention.hpp), written the
// way the reference's own C++ callers use it: fill rdna::ForwardParams /
// rdna::ForwardParamsInt8QK field by field, call rdna::forwardF16 /
// rdna::forwardInt8QK, and read rdna::lastError*() on failure (reference:
// tests/hip_forward_gate.hip:196-228, tests/hip_forward_int8qk_gate.hip:196-232).
// The tests load this file's library with ctypes and compare its results with
// the C ABI's; nothing in the shipped library uses it.
#include "rdnattention.hpp"

#include <cstdint>
#include <cstring>

namespace {

void copy_error(const char* msg, char* err, int errlen) {
    if (err == nullptr || errlen <= 0) {
        return;
    }
    std::strncpy(err, msg != nullptr ? msg : "", (size_t)errlen - 1);
    err[errlen - 1] = '\0';
}

} // namespace

extern "C" {

// strides: q, k, v, o x (b, h, s), in elements; dims: B, Hq, Hkv, Sq, Sk, D
int cxx_forward_f16(const void* q, const void* k, const void* v, void* o, const void* rot_cos, const void* rot_sin,
                    const int64_t* strides, const uint32_t* dims, float scale, uint32_t causal, uint32_t has_rope,
                    int32_t window, void* stream, char* err, int errlen) {
    rdna::ForwardParams p{};
    p.q = q;
    p.k = k;
    p.v = v;
    p.o = o;
    p.rot_cos = rot_cos;
    p.rot_sin = rot_sin;
    p.qStrideB = strides[0];
    p.qStrideH = strides[1];
    p.qStrideS = strides[2];
    p.kStrideB = strides[3];
    p.kStrideH = strides[4];
    p.kStrideS = strides[5];
    p.vStrideB = strides[6];
    p.vStrideH = strides[7];
    p.vStrideS = strides[8];
    p.oStrideB = strides[9];
    p.oStrideH = strides[10];
    p.oStrideS = strides[11];
    p.batchSize = dims[0];
    p.numHeads = dims[1];
    p.numKvHeads = dims[2];
    p.seqLen = dims[3];
    p.keySeqLen = dims[4];
    p.headDim = dims[5];
    p.scale = scale;
    p.causal = causal;
    p.hasRope = has_rope;
    p.windowSize = window;
    const int rc = rdna::forwardF16(p, stream);
    copy_error(rc != 0 ? rdna::lastError() : nullptr, err, errlen);
    return rc;
}

int cxx_forward_int8qk(const void* q, const void* k, const void* v, void* o, const int64_t* strides,
                       const uint32_t* dims, float scale, float q_scale, float k_scale, float v_scale,
                       const void* q_scale_vec, const void* k_scale_vec, uint32_t causal, int32_t window, void* stream,
                       char* err, int errlen) {
    rdna::ForwardParamsInt8QK p{};
    p.q = q;
    p.k = k;
    p.v = v;
    p.o = o;
    p.qStrideB = strides[0];
    p.qStrideH = strides[1];
    p.qStrideS = strides[2];
    p.kStrideB = strides[3];
    p.kStrideH = strides[4];
    p.kStrideS = strides[5];
    p.vStrideB = strides[6];
    p.vStrideH = strides[7];
    p.vStrideS = strides[8];
    p.oStrideB = strides[9];
    p.oStrideH = strides[10];
    p.oStrideS = strides[11];
    p.batchSize = dims[0];
    p.numHeads = dims[1];
    p.numKvHeads = dims[2];
    p.seqLen = dims[3];
    p.keySeqLen = dims[4];
    p.headDim = dims[5];
    p.scale = scale;
    p.qScale = q_scale;
    p.kScale = k_scale;
    p.vScale = v_scale;
    p.causal = causal;
    p.windowSize = window;
    p.qScaleVec = q_scale_vec;
    p.kScaleVec = k_scale_vec;
    const int rc = rdna::forwardInt8QK(p, stream);
    copy_error(rc != 0 ? rdna::lastErrorInt8QK() : nullptr, err, errlen);
    return rc;
}

int cxx_has_device() { return rdna::hasDevice() ? 1 : 0; }

} // extern "C"
