// Shared definitions of the gfx950 quantized-matmul path: GGUF type ids,
// the device layouts of weights and activations, and small device helpers.
//
// Device weight layout (one allocation per tensor, planes 256-byte aligned).
// GGUF blocks are 18/34/144/210 bytes, which defeats 128-bit loads, so a
// tensor is repacked once at upload into planes with the same total size:
//   Q8_0  codes [N][K] int8                 d    [N][K/32]  f16
//   Q4_0  codes [N][K/32][16] nibbles       d    [N][K/32]  f16
//   Q4_K  codes [N][K/32][16] nibbles       meta [N][K/256][16] (d, dmin, scales[12])
//   Q6_K  codes [N][K/32][16] low nibbles   qh   [N][K/32][8]  high bits
//         sc   [N][K/16] int8               d    [N][K/256] f16
// Every 16-byte code chunk holds one 32-element group in Q4_0's nibble order:
// byte j = element j (low nibble) | element j+16 (high nibble). For Q6_K the
// 8 qh bytes are two dwords (elements 0..15, 16..31); byte b of a dword holds
// in bits 2k..2k+1 the two high bits of element 4k+b of that half.
//
// Device activation layout (written by the quantizer, read by the matmuls):
//   q32  [M][K] int8   d32 [M][K/32] f32    s32 [M][K/32] int32   (Q8Act)
//   q256 [M][K] int8   d256 [M][K/256] f32  s16 [M][K/16] int16   (Q8ActK)
//   bsm  [M][K/256][16] int8: bytes 0..7 = bsum_g >> 6, 8..15 = bsum_g & 63
//   m32, m256 [M][K] int8: the q32 / q256 codes in MFMA operand order
//   gA   [M'/32][K/32][64][16] int8: q256 codes as A operands of
//        v_mfma_i32_32x32x32_i8, one 1 KB piece per (32-token block, 32-value
//        step): lane l holds token l % 32, values 16 (l / 32) .. +15 of the step
//   gX   [M'/32][K/256][2][16] f32: Q8ActK d in the order of that MFMA's
//        output registers: [h][i] is token 8 (i / 4) + 4 h + i % 4 of the block
//   gJ   [M'/32][K/256][64][8] f16: A operands of v_mfma_f32_32x32x16_f16
//        for the Q4_K / Q5_K mins term: lane l < 32 holds 64 (bsum_g >> 6) of token l,
//        lane 32 + l holds bsum_g & 63, g = 0..7
// (bsum_g = the Q8ActK per-32 sum; s16 holds per-16 sums, two of which make
// a bsum; M' = M rounded up to a multiple of 32, the extra tokens all zero).
// The 256 planes exist only when K % 256 == 0.
// MFMA operand order: within each 256-element unit (8 groups of 32), byte
// q*64 + g*8 + i holds element 4q+i (i < 4) or 16+4q+(i-4) (i >= 4) of group
// g, q < 4: the eight codes that lane quarter q of a 16x16x32 int8 MFMA
// takes for group g, which matches one dword of a 16-byte nibble chunk.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fishhip {

enum : uint32_t { kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14 };
// types FISH multiplies in f32 (dequantise, then f32 dot; ops.cpp:219-250)
enum : uint32_t { kQ4_1 = 3, kQ5_0 = 6, kQ5_1 = 7, kQ2_K = 10, kQ3_K = 11, kIQ4_NL = 20, kBF16 = 30, kMXFP4 = 39 };

// K-quants: 256-value super-blocks, multiplied with the Q8ActK activations.
constexpr bool kquant_type(uint32_t t) { return t == kQ4_K || t == kQ5_K || t == kQ6_K; }
// K-quants with a per-group min (w = d sc q - dmin m): the Q8ActK block sums enter.
constexpr bool has_mins(uint32_t t) { return t == kQ4_K || t == kQ5_K; }

inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

struct WeightLayout {
    uint32_t type = 0;
    int n_in = 0, n_out = 0;
    size_t codes = 0, aux = 0, sc = 0, d = 0, hb = 0, total = 0;  // plane byte offsets
};

// Plane offsets of a repacked tensor; total == 0 when the type/shape is refused.
inline WeightLayout weight_layout(uint32_t type, int n_in, int n_out) {
    WeightLayout L;
    L.type = type;
    L.n_in = n_in;
    L.n_out = n_out;
    const size_t N = size_t(n_out), K = size_t(n_in);
    if (n_in <= 0 || n_out <= 0) return L;
    size_t off = 0;
    switch (type) {
        case kQ8_0:
            if (K % 32) return L;
            L.codes = off; off = align256(off + N * K);
            L.d = off;     off = align256(off + N * (K / 32) * 2);
            break;
        case kQ4_0:
            if (K % 32) return L;
            L.codes = off; off = align256(off + N * (K / 32) * 16);
            L.d = off;     off = align256(off + N * (K / 32) * 2);
            break;
        case kQ4_K:
            if (K % 256) return L;
            L.codes = off; off = align256(off + N * (K / 32) * 16);
            L.aux = off;   off = align256(off + N * (K / 256) * 16);
            break;
        case kQ5_K:
            // Q4_K's planes plus the fifth bits: one dword per group, bit 8b + k
            // = element 4k + b, bit 8b + 4 + k = element 16 + 4k + b (k, b < 4),
            // so a shift and a mask put dword k's four bits at bit 4 of its bytes
            if (K % 256) return L;
            L.codes = off; off = align256(off + N * (K / 32) * 16);
            L.aux = off;   off = align256(off + N * (K / 256) * 16);
            L.hb = off;    off = align256(off + N * (K / 32) * 4);
            break;
        case kQ6_K:
            if (K % 256) return L;
            L.codes = off; off = align256(off + N * (K / 32) * 16);
            L.aux = off;   off = align256(off + N * (K / 32) * 8);
            L.sc = off;    off = align256(off + N * (K / 16));
            L.d = off;     off = align256(off + N * (K / 256) * 2);
            break;
        default:
            return L;
    }
    L.total = off;
    return L;
}

// GGUF bytes of one row (gguf.cpp:216-263 type table).
inline size_t gguf_row_bytes(uint32_t type, int n_in) {
    switch (type) {
        case kQ8_0: return size_t(n_in / 32) * 34;
        case kQ4_0: return size_t(n_in / 32) * 18;
        case kQ4_K: return size_t(n_in / 256) * 144;
        case kQ5_K: return size_t(n_in / 256) * 176;
        case kQ6_K: return size_t(n_in / 256) * 210;
        case kF32: return size_t(n_in) * 4;
        case kF16: case kBF16: return size_t(n_in) * 2;
        case kQ4_1: return size_t(n_in / 32) * 20;
        case kQ5_0: return size_t(n_in / 32) * 22;
        case kQ5_1: return size_t(n_in / 32) * 24;
        case kIQ4_NL: return size_t(n_in / 32) * 18;
        case kMXFP4: return size_t(n_in / 32) * 17;
        case kQ2_K: return size_t(n_in / 256) * 84;
        case kQ3_K: return size_t(n_in / 256) * 110;
        default: return 0;
    }
}

inline bool is_kquant(uint32_t type) { return kquant_type(type); }

struct ActLayout {
    int n_tok = 0, n_in = 0;
    size_t q32 = 0, d32 = 0, s32 = 0, q256 = 0, d256 = 0, s16 = 0, bsm = 0, m32 = 0, m256 = 0;
    size_t gA = 0, gX = 0, gJ = 0, total = 0;
    int n_tb = 0;  // 32-token blocks of the gA / gX / gJ planes
    bool has256 = false;
};

inline ActLayout act_layout(int n_tok, int n_in) {
    ActLayout L;
    L.n_tok = n_tok;
    L.n_in = n_in;
    if (n_tok <= 0 || n_in <= 0 || n_in % 32) return L;
    const size_t M = size_t(n_tok), K = size_t(n_in);
    size_t off = 0;
    L.q32 = off;  off = align256(off + M * K);
    L.d32 = off;  off = align256(off + M * (K / 32) * 4);
    L.s32 = off;  off = align256(off + M * (K / 32) * 4);
    L.has256 = (K % 256) == 0;
    if (L.has256) {
        L.q256 = off; off = align256(off + M * K);
        L.d256 = off; off = align256(off + M * (K / 256) * 4);
        L.s16 = off;  off = align256(off + M * (K / 16) * 2);
        L.bsm = off;  off = align256(off + M * (K / 256) * 16);
        L.m32 = off;  off = align256(off + M * K);
        L.m256 = off; off = align256(off + M * K);
        L.n_tb = (n_tok + 31) / 32;
        const size_t TB = size_t(L.n_tb), SB = K / 256;
        L.gA = off;   off = align256(off + TB * 32 * K);
        L.gX = off;   off = align256(off + TB * SB * 32 * 4);
        L.gJ = off;   off = align256(off + TB * SB * 64 * 16);
    }
    L.total = off;
    return L;
}

// Device pointers of one activation buffer.
struct ActPtrs {
    const int8_t* q32;
    const float* d32;
    const int32_t* s32;
    const int8_t* q256;
    const float* d256;
    const int16_t* s16;
    const int8_t* bsm;
    const int8_t* m32;
    const int8_t* m256;
    const int8_t* gA;
    const float* gX;
    const uint16_t* gJ;
    int n_tb;
};

inline ActPtrs act_ptrs(const void* base, const ActLayout& L) {
    const uint8_t* b = static_cast<const uint8_t*>(base);
    ActPtrs p;
    p.q32 = reinterpret_cast<const int8_t*>(b + L.q32);
    p.d32 = reinterpret_cast<const float*>(b + L.d32);
    p.s32 = reinterpret_cast<const int32_t*>(b + L.s32);
    p.q256 = L.has256 ? reinterpret_cast<const int8_t*>(b + L.q256) : nullptr;
    p.d256 = L.has256 ? reinterpret_cast<const float*>(b + L.d256) : nullptr;
    p.s16 = L.has256 ? reinterpret_cast<const int16_t*>(b + L.s16) : nullptr;
    p.bsm = L.has256 ? reinterpret_cast<const int8_t*>(b + L.bsm) : nullptr;
    p.m32 = L.has256 ? reinterpret_cast<const int8_t*>(b + L.m32) : nullptr;
    p.m256 = L.has256 ? reinterpret_cast<const int8_t*>(b + L.m256) : nullptr;
    p.gA = L.has256 ? reinterpret_cast<const int8_t*>(b + L.gA) : nullptr;
    p.gX = L.has256 ? reinterpret_cast<const float*>(b + L.gX) : nullptr;
    p.gJ = L.has256 ? reinterpret_cast<const uint16_t*>(b + L.gJ) : nullptr;
    p.n_tb = L.n_tb;
    return p;
}

struct WeightPtrs {
    const uint8_t* codes;
    const uint8_t* aux;
    const int8_t* sc;
    const uint16_t* d;
    const uint32_t* hb;  // Q5_K fifth bits
};

inline WeightPtrs weight_ptrs(const void* base, const WeightLayout& L) {
    const uint8_t* b = static_cast<const uint8_t*>(base);
    WeightPtrs p;
    p.codes = b + L.codes;
    p.aux = b + L.aux;
    p.sc = reinterpret_cast<const int8_t*>(b + L.sc);
    p.d = reinterpret_cast<const uint16_t*>(b + L.d);
    p.hb = reinterpret_cast<const uint32_t*>(b + L.hb);
    return p;
}

// ------------------------------------------------------------ device helpers

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// 6-bit scale and min of sub-block g (0..7) from the 12 packed bytes s0..s11
// held in three dwords (quant.cpp:136-144 layout).
__device__ __forceinline__ void k4_scale_min(uint32_t s03, uint32_t s47, uint32_t s811, int g, int& sc, int& mn) {
    const int h = (g & 3) * 8;
    const uint32_t a = (s03 >> h) & 0xFF, b = (s47 >> h) & 0xFF, c = (s811 >> h) & 0xFF;
    // selects, not branches: lanes of one wavefront hold different g
    const bool lo = g < 4;
    sc = int(lo ? (a & 63) : ((c & 15) | ((a >> 6) << 4)));
    mn = int(lo ? (b & 63) : ((c >> 4) | ((b >> 6) << 4)));
}

}  // namespace fishhip
