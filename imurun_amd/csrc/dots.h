// Integer dot products of one 32-element weight group with int8 activations,
// shared by the GEMV kernel, the grouped MoE kernels and the per-block
// diagnostic kernel, so that the integers checked for bit-exactness are the
// ones the matmuls use.
//
// The integers are the ones FISH's AVX2 kernels form per block
// (quant_x86.cpp:280-297 Q4_0, :299-309 Q8_0, :346-382 Q4_K, :445-495 Q6_K):
//   Q8_0  sum_k w_k x_k                          (w int8)
//   Q4_0  sum_k (nib_k - 8) x_k                  (nib 0..15)
//   Q4_K  dot_g = sum_l q_l x_l; the caller forms sc_g*dot_g and m_g*bsum_g
//   Q5_K  the same with 5-bit codes (quant_x86.cpp:384-427)
//   Q6_K  sc_a*sum_{16}(q-32)x + sc_b*sum_{16}(q-32)x  (two 16-groups)
#pragma once

#include "common.h"

namespace fishhip {

// 4 int8 codes per dword, in element order; one sdot4 per dword.
__device__ __forceinline__ int dot16(uint4 w, uint4 a, int acc) {
    acc = sdot4(w.x, a.x, acc);
    acc = sdot4(w.y, a.y, acc);
    acc = sdot4(w.z, a.z, acc);
    acc = sdot4(w.w, a.w, acc);
    return acc;
}

__device__ __forceinline__ uint4 lo_nibbles(uint4 w) {
    return make_uint4(w.x & 0x0F0F0F0Fu, w.y & 0x0F0F0F0Fu, w.z & 0x0F0F0F0Fu, w.w & 0x0F0F0F0Fu);
}

__device__ __forceinline__ uint4 hi_nibbles(uint4 w) {
    return make_uint4((w.x >> 4) & 0x0F0F0F0Fu, (w.y >> 4) & 0x0F0F0F0Fu, (w.z >> 4) & 0x0F0F0F0Fu,
                      (w.w >> 4) & 0x0F0F0F0Fu);
}

// 6-bit Q6_K codes of one half (16 elements) of a group: low nibbles `nib`
// plus the two high bits held in `qh` (byte b, bits 2k..2k+1 -> element 4k+b).
__device__ __forceinline__ uint4 q6_codes(uint4 nib, uint32_t qh) {
    return make_uint4(nib.x | ((qh & 0x03030303u) << 4), nib.y | (((qh >> 2) & 0x03030303u) << 4),
                      nib.z | (((qh >> 4) & 0x03030303u) << 4), nib.w | (((qh >> 6) & 0x03030303u) << 4));
}

__device__ __forceinline__ int isum_q8_0(uint4 w0, uint4 w1, uint4 a0, uint4 a1) {
    return dot16(w1, a1, dot16(w0, a0, 0));
}

__device__ __forceinline__ int isum_q4_0(uint4 w, uint4 alo, uint4 ahi, int asum) {
    return dot16(hi_nibbles(w), ahi, dot16(lo_nibbles(w), alo, 0)) - 8 * asum;
}

__device__ __forceinline__ int dot_q4_k(uint4 w, uint4 alo, uint4 ahi) {
    return dot16(hi_nibbles(w), ahi, dot16(lo_nibbles(w), alo, 0));
}

// Q5_K codes: nibbles plus the fifth bits of the group (the repacked dword
// whose bit 8b + k is element 4k + b and bit 8b + 4 + k element 16 + 4k + b):
// a shift and a mask move dword k's bits to bit 4 of its bytes.
__device__ __forceinline__ uint4 q5_codes_lo(uint4 lo, uint32_t h) {
    return make_uint4(lo.x | ((h << 4) & 0x10101010u), lo.y | ((h << 3) & 0x10101010u),
                      lo.z | ((h << 2) & 0x10101010u), lo.w | ((h << 1) & 0x10101010u));
}
__device__ __forceinline__ uint4 q5_codes_hi(uint4 hi, uint32_t h) {
    return make_uint4(hi.x | (h & 0x10101010u), hi.y | ((h >> 1) & 0x10101010u), hi.z | ((h >> 2) & 0x10101010u),
                      hi.w | ((h >> 3) & 0x10101010u));
}

__device__ __forceinline__ int dot_q5_k(uint4 w, uint32_t h, uint4 alo, uint4 ahi) {
    return dot16(q5_codes_hi(hi_nibbles(w), h), ahi, dot16(q5_codes_lo(lo_nibbles(w), h), alo, 0));
}

__device__ __forceinline__ int isum_q6_k(uint4 w, uint2 qh, uint4 alo, uint4 ahi, int s16a, int s16b, int sca,
                                         int scb) {
    const int da = dot16(q6_codes(lo_nibbles(w), qh.x), alo, 0) - 32 * s16a;
    const int db = dot16(q6_codes(hi_nibbles(w), qh.y), ahi, 0) - 32 * s16b;
    return sca * da + scb * db;
}

}  // namespace fishhip
