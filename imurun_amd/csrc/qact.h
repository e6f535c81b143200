// Device arithmetic of FISH's activation quantizer (quantize_acts_scalar /
// quantize_acts_k_scalar, quant.cpp:400-434), shared by the quantize kernel
// and the GEMV that quantizes its own input, so both produce the same bytes:
//   d = amax / 127 (IEEE f32 division), id = d > 0 ? 1 / d : 0,
//   q = clamp(rint(x * id), -127, 127) with round-half-to-even, x * id one
//   rounding (no contraction). Lanes 8j..8j+7 hold one 32-value block.
#pragma once

#include "common.h"

namespace fishhip {

__device__ __forceinline__ float wave_max8(float v) {
    v = fmaxf(v, __shfl_xor(v, 1));
    v = fmaxf(v, __shfl_xor(v, 2));
    v = fmaxf(v, __shfl_xor(v, 4));
    return v;
}

__device__ __forceinline__ float wave_max64(float v) {
    for (int off = 1; off < 64; off <<= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ int wave_sum8(int v) {
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    return v;
}

__device__ __forceinline__ int code(float x, float id) {
    const float p = __fmul_rn(x, id);
    const int q = static_cast<int>(__builtin_rintf(p));
    return q < -127 ? -127 : (q > 127 ? 127 : q);
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t(a) & 0xFF) | ((uint32_t(b) & 0xFF) << 8) | ((uint32_t(c) & 0xFF) << 16) | (uint32_t(d) << 24);
}

// d and 1/d of a block with absolute maximum amax
__device__ __forceinline__ float block_d(float amax) { return amax / 127.0f; }
__device__ __forceinline__ float block_id(float d) { return d > 0.0f ? 1.0f / d : 0.0f; }

}  // namespace fishhip
