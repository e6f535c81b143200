// matmul_batch for the weight types FISH multiplies in f32 (ops.cpp:219-250):
// Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, MXFP4 and plain F32 / F16 / BF16
// rows. FISH has no int8 kernel for them (quant.cpp:475-481): it
// dequantises each weight row to f32 and dots it with the f32 activations.
//
// Here the weights stay in their GGUF bytes on the device. A wavefront owns
// output rows; lane l takes each row's 32-value sub-blocks l, l + 64, ...,
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

// The non-linear 4-bit codebook of IQ4_NL (quant.cpp:286-288) as four dwords of
// int8, looked up four codes at a time with byte permutes.
constexpr uint32_t kNL0 = 0xBFAD9881u, kNL1 = 0xF6EADDCFu, kNL2 = 0x26190D01u, kNL3 = 0x71594535u;

__device__ __forceinline__ uint32_t nl_lookup4(uint32_t idx) {  // four indices 0..15, one per byte
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kNL1, kNL0, sel), hi = __builtin_amdgcn_perm(kNL3, kNL2, sel);
    const uint32_t m = ((idx >> 3) & 0x01010101u) * 0xFFu;  // 0xFF in bytes whose index is >= 8
    return (hi & m) | (lo & ~m);
}
__device__ __forceinline__ float sbyte(uint32_t w, int b) { return float(int8_t((w >> (8 * b)) & 0xFF)); }

// e2m1 magnitude codes 0..7 -> 0, 0.5, 1, 1.5, 2, 3, 4, 6 (exact), sign in bit 3
__device__ __forceinline__ float e2m1(int c) {
    const int mag = c & 7;
    const uint32_t bits = mag >= 2 ? ((126u + uint32_t(mag >> 1)) << 23) | (uint32_t(mag & 1) << 22)
                                   : (mag == 1 ? (126u << 23) : 0u);
    return __builtin_bit_cast(float, bits | (uint32_t(c & 8) << 28));
}

// Loads of the plain and the aligned block formats go through dwords (or
// wider); 2-byte aligned blocks through 16-bit loads, MXFP4 (17 bytes) byte by
// byte. Row starts keep every block's alignment: rows are whole blocks and the
// buffer is 256-byte aligned.
__device__ __forceinline__ uint32_t ld16x2(const uint8_t* p) {  // 2-byte aligned dword
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    return uint32_t(h[0]) | (uint32_t(h[1]) << 16);
}

// Values 32 j .. 32 j + 31 of the block (or row chunk) at p, in FISH's float
// order (quant.cpp:92-126, :218-331; F16 / BF16: exact widening).
template <uint32_t T>
__device__ __forceinline__ void dq32(const uint8_t* p, int j, float (&w)[32]) {
    if constexpr (T == kF32) {
        const float4* f = reinterpret_cast<const float4*>(p) + 8 * j;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float4 v = f[k];
            w[4 * k] = v.x; w[4 * k + 1] = v.y; w[4 * k + 2] = v.z; w[4 * k + 3] = v.w;
        }
    } else if constexpr (T == kF16 || T == kBF16) {
        const uint4* q = reinterpret_cast<const uint4*>(p) + 4 * j;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint4 v = q[k];
            const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint16_t b = uint16_t(d[i] >> (16 * h));
                    w[8 * k + 2 * i + h] = T == kF16 ? f16_bits_to_f32(b) : __builtin_bit_cast(float, uint32_t(b) << 16);
                }
        }
    } else if constexpr (T == kQ4_1 || T == kQ5_1) {
        // Q4_1: 20-byte blocks, 4-byte aligned; Q5_1: 24-byte blocks, 8-byte aligned
        const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
        const uint32_t dm = q[0];
        const float d = f16_bits_to_f32(uint16_t(dm & 0xFFFF)), m = f16_bits_to_f32(uint16_t(dm >> 16));
        const uint32_t qh = T == kQ5_1 ? q[1] : 0u;
        constexpr int o = T == kQ5_1 ? 2 : 1;
        const uint32_t qs[4] = {q[o], q[o + 1], q[o + 2], q[o + 3]};
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const uint32_t b = (qs[k >> 2] >> (8 * (k & 3))) & 0xFF;
            const int lo = int(b & 15) | int(((qh >> k) & 1) << 4), hi = int(b >> 4) | int(((qh >> (k + 16)) & 1) << 4);
            w[k] = d * float(lo) + m;
            w[k + 16] = d * float(hi) + m;
        }
    } else if constexpr (T == kQ5_0) {  // 22-byte blocks, 2-byte aligned
        const float d = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[0]);
        const uint32_t qh = ld16x2(p + 2);
        const uint32_t qs[4] = {ld16x2(p + 6), ld16x2(p + 10), ld16x2(p + 14), ld16x2(p + 18)};
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const uint32_t b = (qs[k >> 2] >> (8 * (k & 3))) & 0xFF;
            const int lo = int(b & 15) | int(((qh >> k) & 1) << 4), hi = int(b >> 4) | int(((qh >> (k + 16)) & 1) << 4);
            w[k] = d * float(lo - 16);
            w[k + 16] = d * float(hi - 16);
        }
    } else if constexpr (T == kQ2_K) {
        // 84-byte blocks, 4-byte aligned. Value 32 j + 16 h + l: scale byte 8 n + 2 jj + h,
        // bits 2 jj of qs[32 n + 16 h + l] (n = j / 4, jj = j % 4); (d * sc) * q - dmin * m
        const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
        const int n = j >> 2, jj = j & 3;
        const uint32_t dd = q[20];
        const float d = f16_bits_to_f32(uint16_t(dd & 0xFFFF)), dmin = f16_bits_to_f32(uint16_t(dd >> 16));
        const uint32_t sc2 = (q[(8 * n + 2 * jj) >> 2] >> (8 * ((2 * jj) & 3))) & 0xFFFF;
        uint32_t qs[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) qs[i] = q[4 + 8 * n + i];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t sc = (sc2 >> (8 * h)) & 0xFF;
            const float dl = d * float(sc & 15), ml = dmin * float(sc >> 4);
#pragma unroll
            for (int l = 0; l < 16; ++l) {
                const uint32_t b = (qs[(16 * h + l) >> 2] >> (8 * (l & 3))) & 0xFF;
                w[16 * h + l] = dl * float((b >> (2 * jj)) & 3) - ml;
            }
        }
    } else if constexpr (T == kQ3_K) {
        // 110-byte blocks, 2-byte aligned. 6-bit signed scales (low 4 bits in bytes
        // 96..103, high 2 in 104..107), 2-bit codes minus 4 where hmask bit 4 n + jj is clear
        const int n = j >> 2, jj = j & 3;
        const float dall = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[54]);
        uint32_t hm[8], qs[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            hm[i] = ld16x2(p + 4 * i);
            qs[i] = ld16x2(p + 32 + 32 * n + 4 * i);
        }
        // the two low-nibble bytes of scales i = 8 n + 2 jj + h (byte 96 + (i & 7)), and
        // bytes 104..107 with the high bits
        const uint32_t sl = uint32_t(reinterpret_cast<const uint16_t*>(p + 96 + 2 * jj)[0]);
        const uint32_t shi = ld16x2(p + 104);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int i = 8 * n + 2 * jj + h;
            const uint32_t sb = (sl >> (8 * h)) & 0xFF;
            const int lo = i < 8 ? int(sb & 15) : int(sb >> 4);
            const int hi = int((shi >> (8 * (i & 3) + 2 * (i >> 2))) & 3);
            const float dl = dall * float((lo | (hi << 4)) - 32);
#pragma unroll
            for (int l = 0; l < 16; ++l) {
                const int idx = 16 * h + l;
                const int q2 = int((qs[idx >> 2] >> (8 * (idx & 3) + 2 * jj)) & 3);
                const int hmb = int((hm[idx >> 2] >> (8 * (idx & 3) + 4 * n + jj)) & 1);
                w[idx] = dl * float(q2 - (hmb ? 0 : 4));
            }
        }
    } else if constexpr (T == kIQ4_NL) {  // 18-byte blocks, 2-byte aligned
        const float d = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[0]);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t qs = ld16x2(p + 2 + 4 * k);
            const uint32_t lo = nl_lookup4(qs & 0x0F0F0F0Fu), hi = nl_lookup4((qs >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                w[4 * k + b] = d * sbyte(lo, b);
                w[16 + 4 * k + b] = d * sbyte(hi, b);
            }
        }
    } else {  // MXFP4 (17-byte blocks): 2^(e - 127) times signed e2m1 codes
        const float d = ldexpf(1.0f, int(p[0]) - 127);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int c = p[1 + k];
            w[k] = d * e2m1(c & 15);
            w[k + 16] = d * e2m1(c >> 4);
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

// A wavefront owns RPW consecutive rows. For one token (NT == 1, RPW rows) the
// lane's 32 x values of a sub-block are loaded once and serve every row; for
// more tokens (RPW == 1) each token's x values are loaded per sub-block.
template <uint32_t T, int NT, int RPW>
__global__ __launch_bounds__(64 * kDqWaves) void dq_matmul_kernel(const uint8_t* __restrict__ w,
                                                                  const float* __restrict__ x, int n_tok, int n_in,
                                                                  int n_out, float* __restrict__ y) {
    static_assert(NT == 1 || RPW == 1, "several rows per wavefront only for one token");
    using S = DqShape<T>;
    const int row0 = (int(blockIdx.x) * kDqWaves + int(threadIdx.x >> 6)) * RPW;
    const int lane = threadIdx.x & 63;
    if (row0 >= n_out) return;  // uniform over the wavefront
    const int t0 = int(blockIdx.y) * NT, nt = min(NT, n_tok - t0);
    const size_t row_bytes = size_t(n_in / S::elems) * S::bytes;
    constexpr int per_block = S::elems / 32;
    float acc[RPW][NT];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[r][t] = 0.0f;
    auto dot32 = [](const float (&v)[32], const float4* xt, float a) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 xv = xt[q];
            a = fmaf(v[4 * q], xv.x, a);
            a = fmaf(v[4 * q + 1], xv.y, a);
            a = fmaf(v[4 * q + 2], xv.z, a);
            a = fmaf(v[4 * q + 3], xv.w, a);
        }
        return a;
    };
    for (int sb = lane; sb < n_in / 32; sb += 64) {
        const size_t boff = size_t(sb / per_block) * S::bytes;
        if constexpr (NT == 1) {
            float4 xr[8];
            const float4* xt = reinterpret_cast<const float4*>(x + size_t(t0) * n_in + 32 * sb);
#pragma unroll
            for (int q = 0; q < 8; ++q) xr[q] = xt[q];
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                float v[32];
                // rows past the end repeat the last one (decoded, never stored)
                dq32<T>(w + size_t(min(row0 + r, n_out - 1)) * row_bytes + boff, sb % per_block, v);
                acc[r][0] = dot32(v, xr, acc[r][0]);
            }
        } else {
            float v[32];
            dq32<T>(w + size_t(row0) * row_bytes + boff, sb % per_block, v);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (t >= nt) break;
                acc[0][t] = dot32(v, reinterpret_cast<const float4*>(x + size_t(t0 + t) * n_in + 32 * sb), acc[0][t]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float a = acc[r][t];
            for (int off = 32; off > 0; off >>= 1) a += __shfl_xor(a, off);
            if (lane == 0 && t < nt && row0 + r < n_out) y[size_t(t0 + t) * n_out + row0 + r] = a;
        }
}

// Rows per wavefront for one token: four for the packed block formats, whose
// x re-reads otherwise bound them (Q4_1 14336x4096: 30.9 -> 16.6 us); one for
// the plain float rows (wide loads, more wavefronts in flight: F16 39 vs 45 us)
// and MXFP4 (byte loads of four rows at once need 315 registers: 50 vs 106 us).
template <uint32_t T>
constexpr int dq_rows1() { return (T == kF32 || T == kF16 || T == kBF16 || T == kMXFP4) ? 1 : 4; }

template <uint32_t T>
hipError_t dq_launch(const void* w, const float* x, int n_tok, int n_in, int n_out, float* y, hipStream_t s) {
    if (n_in % DqShape<T>::elems || n_in % 32) return hipErrorInvalidValue;
    const dim3 block(64 * kDqWaves);
    if (n_tok == 1) {
        constexpr int R = dq_rows1<T>();
        const int per_wg = kDqWaves * R;
        hipLaunchKernelGGL((dq_matmul_kernel<T, 1, R>), dim3(unsigned((n_out + per_wg - 1) / per_wg), 1u),
                           block, 0, s, static_cast<const uint8_t*>(w), x, n_tok, n_in, n_out, y);
    } else {
        const dim3 grid(unsigned((n_out + kDqWaves - 1) / kDqWaves), unsigned((n_tok + kDqTokens - 1) / kDqTokens));
        hipLaunchKernelGGL((dq_matmul_kernel<T, kDqTokens, 1>), grid, block, 0, s, static_cast<const uint8_t*>(w),
                           x, n_tok, n_in, n_out, y);
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
