// Device arithmetic of FISH's activation quantizer (quantize_acts_scalar /
// quantize_acts_k_scalar, quant.cpp:400-434), shared by the quantize kernel
// and the GEMV that quantizes its own input, so both produce the same bytes:
//   d = amax / 127 (IEEE f32 division), id = d > 0 ? 1 / d : 0,
//   q = clamp(rint(x * id), -127, 127) with round-half-to-even, x * id one
//   rounding (no contraction). Lanes 8j..8j+7 hold one 32-value block.
#pragma once

#include "common.h"

namespace fishhip {

// Cross-lane reductions on DPP lane swizzles (register-to-register, a few
// cycles) rather than ds_bpermute (an LDS round trip each). The caller's
// wavefront must have every lane active. Max and integer sums do not depend
// on the order of their operands, so the results equal any other reduction's.
//   quad_perm [1,0,3,2] = lane ^ 1, [2,3,0,1] = lane ^ 2,
//   row_half_mirror: lane i of each 8-lane half row <- lane 7 - i (after a quad
//     reduction, the other quad of the 8 lanes),
//   row_mirror: lane i of each 16-lane row <- lane 15 - i (after an 8-lane
//     reduction, the other 8 lanes of the row).
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}

// max over each aligned group of 8 lanes, in all 8
__device__ __forceinline__ float wave_max8(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    return fmaxf(v, dpp_f<kDppHalfMirror>(v));
}

// max over each 16-lane row, in all 16
__device__ __forceinline__ float wave_max16(float v) {
    v = wave_max8(v);
    return fmaxf(v, dpp_f<kDppMirror>(v));
}

// max over the wavefront, in all lanes (the four row maxima through scalar registers)
__device__ __forceinline__ float wave_max64(float v) {
    v = wave_max16(v);
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// sum over each aligned group of 4 lanes, in all 4
__device__ __forceinline__ int wave_sum4(int v) {
    v += dpp_i<kDppXor1>(v);
    return v + dpp_i<kDppXor2>(v);
}

// sum over each aligned group of 8 lanes, in all 8
__device__ __forceinline__ int wave_sum8(int v) {
    v = wave_sum4(v);
    return v + dpp_i<kDppHalfMirror>(v);
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

// One token's activations quantized by a workgroup into LDS, in the layout
// the decode kernels read: codes [2][maxg] 16-byte pieces (piece h of group
// g = elements 16 h .. 16 h + 15), and per group either Q8Act (d, sum) or,
// for K-quants, the super-block's Q8ActK d (at [g >> 3]) and the group's two
// per-16 sums packed as int16 pairs.
struct LdsAct {
    uint4* codes;
    float* d;
    int* s;
    int maxg;
};

// Quantizes n_in values held as float4 chunks j = tid + TH i (i < XV) of
// the calling thread; the caller synchronises before reading. Whole 32-value
// (K-quants: 256-value) blocks are in one wavefront, so the reductions are
// wavefront shuffles, and inactive chunks switch whole blocks off together.
template <bool KQ, int XV, int TH>
__device__ __forceinline__ void quantize_to_lds(const float4 (&xv)[XV], int n_in, int tid, const LdsAct& L) {
    const int lane = tid & 63;
    uint8_t* codes = reinterpret_cast<uint8_t*>(L.codes);
#pragma unroll
    for (int i = 0; i < XV; ++i) {
        const int k0 = 4 * (tid + TH * i);
        const bool active = k0 < n_in;
        const float4 v = xv[i];
        const float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        const int g = k0 >> 5, o = k0 & 31;
        uint8_t* dst = codes + (size_t((o >> 4) * L.maxg + g) * 16) + (o & 15);
        if constexpr (!KQ) {
            const float d = block_d(wave_max8(a)), id = block_id(d);
            const int q0 = code(v.x, id), q1 = code(v.y, id), q2 = code(v.z, id), q3 = code(v.w, id);
            const int sum = wave_sum8(q0 + q1 + q2 + q3);
            if (active) {
                *reinterpret_cast<uint32_t*>(dst) = pack4(q0, q1, q2, q3);
                if ((lane & 7) == 0) {
                    L.d[g] = d;
                    L.s[g] = sum;
                }
            }
        } else {
            const float d = block_d(wave_max64(a)), id = block_id(d);
            const int q0 = code(v.x, id), q1 = code(v.y, id), q2 = code(v.z, id), q3 = code(v.w, id);
            const int g16 = wave_sum4(q0 + q1 + q2 + q3);
            const int g16b = dpp_i<kDppHalfMirror>(g16);  // the other 16 values of the 32-value group
            if (active) {
                *reinterpret_cast<uint32_t*>(dst) = pack4(q0, q1, q2, q3);
                if (lane == 0) L.d[k0 >> 8] = d;
                if ((lane & 7) == 0) L.s[g] = (g16 & 0xFFFF) | (g16b << 16);
            }
        }
    }
}

// silu(g) * u in FISH's float order: g / (1 + exp(-g)), then times u
// (silu_inplace, ops.cpp:25-30; model.cpp:1504-1508).
__device__ __forceinline__ float silu_mul(float g, float u) {
    const float s = g / __fadd_rn(1.0f, expf(-g));
    return __fmul_rn(s, u);
}

// act(g) * u in FISH's float steps, each one rounding whatever the file's
// contraction setting: SiLU as silu_mul, or the tanh GELU
// 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3))) (gelu_inplace, ops.cpp:32-38),
// then times u (model.cpp:1504-1508).
__device__ __forceinline__ float act_mul(float g, float u, bool gelu) {
    if (!gelu) return silu_mul(g, u);
    const float c = __fmul_rn(__fmul_rn(__fmul_rn(0.044715f, g), g), g);
    const float t = tanhf(__fmul_rn(0.7978845608028654f, __fadd_rn(g, c)));
    return __fmul_rn(__fmul_rn(__fmul_rn(0.5f, g), __fadd_rn(1.0f, t)), u);
}

}  // namespace fishhip
