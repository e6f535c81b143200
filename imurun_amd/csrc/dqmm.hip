// matmul_batch for the weight types FISH multiplies in f32 (ops.cpp:219-250):
// Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, MXFP4 and plain F32 / F16 / BF16
// rows. FISH has no int8 kernel for them (quant.cpp:475-481): it
// dequantises each weight row to f32 and dots it with the f32 activations.
//
// Here the weights stay in their GGUF bytes on the device. A wavefront owns
// one output row; lane l takes the row's 32-value sub-blocks l, l + 64, ...,
// decodes each one into 32 f32 values with FISH's own float expressions (so
// the dequantised weights are bit-identical to dequant_row), then multiplies
// it into the accumulators of up to NT tokens with fused multiply-adds; the
// lanes are added by a xor butterfly. Results agree with FISH's to f32
// rounding (FISH sums in another order). Compiled without contraction so that
// each dequantisation rounds like FISH's, step by step.
#include "common.h"
#include "kernels.h"

namespace fishhip {

namespace {

constexpr int kDqWaves = 4;
constexpr int kDqTokens = 8;  // tokens per grid row

__device__ __forceinline__ uint16_t ld16(const uint8_t* p) {
    return uint16_t(p[0] | (uint16_t(p[1]) << 8));
}
__device__ __forceinline__ uint32_t ld32(const uint8_t* p) {
    return uint32_t(p[0]) | (uint32_t(p[1]) << 8) | (uint32_t(p[2]) << 16) | (uint32_t(p[3]) << 24);
}

__constant__ int8_t kCodebookNL[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
__constant__ float kE2M1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

// Values 32 j .. 32 j + 31 of the block (or row chunk) at p, in FISH's float
// order (quant.cpp:92-126, :218-331; F16 / BF16: exact widening).
template <uint32_t T>
__device__ __forceinline__ void dq32(const uint8_t* p, int j, float (&w)[32]) {
    if constexpr (T == kF32) {
        const float* f = reinterpret_cast<const float*>(p) + 32 * j;
#pragma unroll
        for (int k = 0; k < 32; ++k) w[k] = f[k];
    } else if constexpr (T == kF16 || T == kBF16) {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(p) + 32 * j;
#pragma unroll
        for (int k = 0; k < 32; ++k)
            w[k] = T == kF16 ? f16_bits_to_f32(h[k]) : __builtin_bit_cast(float, uint32_t(h[k]) << 16);
    } else if constexpr (T == kQ4_1 || T == kQ5_1) {
        const float d = f16_bits_to_f32(ld16(p)), m = f16_bits_to_f32(ld16(p + 2));
        const uint32_t qh = T == kQ5_1 ? ld32(p + 4) : 0u;
        const uint8_t* qs = p + (T == kQ5_1 ? 8 : 4);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int lo = (qs[k] & 15) | int(((qh >> k) & 1) << 4), hi = (qs[k] >> 4) | int(((qh >> (k + 16)) & 1) << 4);
            w[k] = d * float(lo) + m;
            w[k + 16] = d * float(hi) + m;
        }
    } else if constexpr (T == kQ5_0) {
        const float d = f16_bits_to_f32(ld16(p));
        const uint32_t qh = ld32(p + 2);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int lo = (p[6 + k] & 15) | int(((qh >> k) & 1) << 4), hi = (p[6 + k] >> 4) | int(((qh >> (k + 16)) & 1) << 4);
            w[k] = d * float(lo - 16);
            w[k + 16] = d * float(hi - 16);
        }
    } else if constexpr (T == kQ2_K) {
        // value 32 j + 16 h + l: scale byte 8 n + 2 jj + h, bits 2 jj of qs[32 n + 16 h + l]
        // (n = j / 4, jj = j % 4); (d * sc) * q - dmin * m
        const float d = f16_bits_to_f32(ld16(p + 80)), dmin = f16_bits_to_f32(ld16(p + 82));
        const int n = j >> 2, jj = j & 3;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int sc = p[8 * n + 2 * jj + h];
            const float dl = d * float(sc & 15), ml = dmin * float(sc >> 4);
#pragma unroll
            for (int l = 0; l < 16; ++l) w[16 * h + l] = dl * float((p[16 + 32 * n + 16 * h + l] >> (2 * jj)) & 3) - ml;
        }
    } else if constexpr (T == kQ3_K) {
        // 6-bit signed scales (low 4 bits in bytes 96..103, high 2 in 104..107), 2-bit
        // codes minus 4 where the hmask bit 4 n + jj is clear
        const float dall = f16_bits_to_f32(ld16(p + 108));
        const int n = j >> 2, jj = j & 3;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int i = 8 * n + 2 * jj + h;
            const int lo = i < 8 ? (p[96 + i] & 15) : (p[96 + i - 8] >> 4);
            const int hi = (p[104 + (i & 3)] >> (2 * (i >> 2))) & 3;
            const float dl = dall * float((lo | (hi << 4)) - 32);
#pragma unroll
            for (int l = 0; l < 16; ++l) {
                const int idx = 16 * h + l;
                const int q2 = (p[32 + 32 * n + idx] >> (2 * jj)) & 3;
                const int hm = (p[idx] >> (4 * n + jj)) & 1;
                w[idx] = dl * float(q2 - (hm ? 0 : 4));
            }
        }
    } else if constexpr (T == kIQ4_NL) {
        const float d = f16_bits_to_f32(ld16(p));
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            w[k] = d * float(kCodebookNL[p[2 + k] & 15]);
            w[k + 16] = d * float(kCodebookNL[p[2 + k] >> 4]);
        }
    } else {  // MXFP4: 2^(e - 127) times signed e2m1 codes
        const float d = ldexpf(1.0f, int(p[0]) - 127);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int lo = p[1 + k] & 15, hi = p[1 + k] >> 4;
            w[k] = d * ((lo & 8) ? -kE2M1[lo & 7] : kE2M1[lo & 7]);
            w[k + 16] = d * ((hi & 8) ? -kE2M1[hi & 7] : kE2M1[hi & 7]);
        }
    }
}

template <uint32_t T>
struct DqShape {
    // elements and bytes of one block (row chunks of 32 for the plain float types)
    static constexpr int elems = (T == kQ2_K || T == kQ3_K) ? 256 : 32;
    static constexpr int bytes = T == kF32 ? 128 : (T == kF16 || T == kBF16) ? 64 : T == kQ4_1 ? 20 : T == kQ5_0 ? 22
                                 : T == kQ5_1 ? 24 : T == kQ2_K ? 84 : T == kQ3_K ? 110 : T == kIQ4_NL ? 18 : 17;
};

template <uint32_t T, int NT>
__global__ __launch_bounds__(64 * kDqWaves) void dq_matmul_kernel(const uint8_t* __restrict__ w,
                                                                  const float* __restrict__ x, int n_tok, int n_in,
                                                                  int n_out, float* __restrict__ y) {
    using S = DqShape<T>;
    const int row = int(blockIdx.x) * kDqWaves + int(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= n_out) return;  // uniform over the wavefront
    const int t0 = int(blockIdx.y) * NT, nt = min(NT, n_tok - t0);
    const size_t row_bytes = size_t(n_in / S::elems) * S::bytes;
    const uint8_t* wr = w + size_t(row) * row_bytes;
    constexpr int per_block = S::elems / 32;
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    for (int sb = lane; sb < n_in / 32; sb += 64) {
        float v[32];
        dq32<T>(wr + size_t(sb / per_block) * S::bytes, sb % per_block, v);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t >= nt) break;
            const float4* xt = reinterpret_cast<const float4*>(x + size_t(t0 + t) * n_in + 32 * sb);
            float a = acc[t];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 xv = xt[q];
                a = fmaf(v[4 * q], xv.x, a);
                a = fmaf(v[4 * q + 1], xv.y, a);
                a = fmaf(v[4 * q + 2], xv.z, a);
                a = fmaf(v[4 * q + 3], xv.w, a);
            }
            acc[t] = a;
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float a = acc[t];
        for (int off = 32; off > 0; off >>= 1) a += __shfl_xor(a, off);
        if (lane == 0 && t < nt) y[size_t(t0 + t) * n_out + row] = a;
    }
}

template <uint32_t T>
hipError_t dq_launch(const void* w, const float* x, int n_tok, int n_in, int n_out, float* y, hipStream_t s) {
    if (n_in % DqShape<T>::elems || n_in % 32) return hipErrorInvalidValue;
    const dim3 block(64 * kDqWaves);
    if (n_tok == 1) {
        hipLaunchKernelGGL((dq_matmul_kernel<T, 1>), dim3(unsigned((n_out + kDqWaves - 1) / kDqWaves), 1u), block, 0,
                           s, static_cast<const uint8_t*>(w), x, n_tok, n_in, n_out, y);
    } else {
        const dim3 grid(unsigned((n_out + kDqWaves - 1) / kDqWaves), unsigned((n_tok + kDqTokens - 1) / kDqTokens));
        hipLaunchKernelGGL((dq_matmul_kernel<T, kDqTokens>), grid, block, 0, s, static_cast<const uint8_t*>(w), x,
                           n_tok, n_in, n_out, y);
    }
    return hipGetLastError();
}

}  // namespace

bool f32path_type(uint32_t type) {
    switch (type) {
        case kF32: case kF16: case kBF16: case kQ4_1: case kQ5_0: case kQ5_1: case kQ2_K: case kQ3_K: case kIQ4_NL:
        case kMXFP4:
            return true;
        default:
            return false;
    }
}

hipError_t launch_dq_matmul(uint32_t type, const void* w, const float* x, int n_tok, int n_in, int n_out, float* y,
                            hipStream_t s) {
    if (n_tok <= 0 || n_in <= 0 || n_out <= 0) return hipErrorInvalidValue;
    switch (type) {
        case kF32: return dq_launch<kF32>(w, x, n_tok, n_in, n_out, y, s);
        case kF16: return dq_launch<kF16>(w, x, n_tok, n_in, n_out, y, s);
        case kBF16: return dq_launch<kBF16>(w, x, n_tok, n_in, n_out, y, s);
        case kQ4_1: return dq_launch<kQ4_1>(w, x, n_tok, n_in, n_out, y, s);
        case kQ5_0: return dq_launch<kQ5_0>(w, x, n_tok, n_in, n_out, y, s);
        case kQ5_1: return dq_launch<kQ5_1>(w, x, n_tok, n_in, n_out, y, s);
        case kQ2_K: return dq_launch<kQ2_K>(w, x, n_tok, n_in, n_out, y, s);
        case kQ3_K: return dq_launch<kQ3_K>(w, x, n_tok, n_in, n_out, y, s);
        case kIQ4_NL: return dq_launch<kIQ4_NL>(w, x, n_tok, n_in, n_out, y, s);
        case kMXFP4: return dq_launch<kMXFP4>(w, x, n_tok, n_in, n_out, y, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace fishhip
