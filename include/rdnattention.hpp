// rdnattention.hpp -- C++ launch API of librdnattention.so.
//
// Same types and functions as the reference's C++ layer
// (dmonkman/RDNAttention src/rdna/fa2_forward_f16.hpp:12-44 and
// src/rdna/fa2_forward_int8qk.hpp:10-46), so C++ callers of rdna::forwardF16
// and rdna::forwardInt8QK (the reference's own gates and benchmarks call
// them directly) link against this library unchanged.  Both functions
// validate exactly like the C ABI in rdnattention.h and return 0 or -1.
#pragma once

#include <cstdint>

namespace rdna {

struct ForwardParams {
    const void* q = nullptr;
    const void* k = nullptr;
    const void* v = nullptr;
    void* o = nullptr;
    const void* rot_cos = nullptr;
    const void* rot_sin = nullptr;

    // Strides in elements (not bytes).
    int64_t qStrideB = 0, qStrideH = 0, qStrideS = 0;
    int64_t kStrideB = 0, kStrideH = 0, kStrideS = 0;
    int64_t vStrideB = 0, vStrideH = 0, vStrideS = 0;
    int64_t oStrideB = 0, oStrideH = 0, oStrideS = 0;

    uint32_t batchSize = 0;
    uint32_t numHeads = 0;
    uint32_t numKvHeads = 0;
    uint32_t seqLen = 0;
    uint32_t keySeqLen = 0;
    uint32_t headDim = 0; // multiple of 32 up to 512
    float scale = 1.0f;
    uint32_t causal = 0;
    uint32_t hasRope = 0;
    int32_t windowSize = -1; // <= 0 = full attention
};

/// Launches the FP16 forward on `stream` (hipStream_t). Non-blocking. 0 on success.
int forwardF16(const ForwardParams& params, void* stream);

/// Reason the most recent forwardF16() call on this thread failed, or nullptr.
const char* lastError();

bool hasDevice();

struct ForwardParamsInt8QK {
    const void* q = nullptr; // int8_t
    const void* k = nullptr; // int8_t
    const void* v = nullptr; // int8_t
    void* o = nullptr;       // _Float16

    int64_t qStrideB = 0, qStrideH = 0, qStrideS = 0;
    int64_t kStrideB = 0, kStrideH = 0, kStrideS = 0;
    int64_t vStrideB = 0, vStrideH = 0, vStrideS = 0;
    int64_t oStrideB = 0, oStrideH = 0, oStrideS = 0;

    uint32_t batchSize = 0;
    uint32_t numHeads = 0;
    uint32_t numKvHeads = 0;
    uint32_t seqLen = 0;
    uint32_t keySeqLen = 0;
    uint32_t headDim = 0;    // 64 or 128
    float scale = 1.0f;      // softmax scale, applied after dequantisation
    float qScale = 1.0f;     // per-tensor Q scale (if qScaleVec is null)
    float kScale = 1.0f;     // per-tensor K scale (if kScaleVec is null)
    float vScale = 1.0f;     // per-tensor V scale
    uint32_t causal = 0;
    int32_t windowSize = -1; // <= 0 = full attention

    const void* qScaleVec = nullptr; // const float*, (batchSize, numHeads, seqLen)
    const void* kScaleVec = nullptr; // const float*, (batchSize, numKvHeads, keySeqLen)
};

/// Launches the INT8 forward on `stream`. Non-blocking. 0 on success.
int forwardInt8QK(const ForwardParamsInt8QK& params, void* stream);

/// Reason the most recent forwardInt8QK() call on this thread failed, or nullptr.
const char* lastErrorInt8QK();

} // namespace rdna
