// Few-token matmul on int8 MFMA: batches of up to a few dozen tokens and
// expert work-list items (matmul_batch, ops.cpp:177-216; the grouped expert
// products of model.cpp:1563-1572).
//
// One v_mfma_i32_16x16x32_i8 forms the exact integer dot of one 32-element
// group for 16 tokens x 16 weight rows:
//   A (activations): lane l supplies token l % 16, eight codes;
//   B (weights):     lane l supplies row   l % 16, the same eight elements;
//   D:               lane l holds row l % 16 of tokens 4 (l / 16) + r, r < 4.
// Lane quarter q = l / 16 takes elements 4q..4q+3 and 16+4q..16+4q+3 of the
// group, which is dword q of a repacked 16-byte nibble chunk (low nibbles,
// then high nibbles) and dwords q and 4+q of a Q8_0 group. The quantizer
// writes the activation codes in exactly that order (the m32 / m256 planes),
// so a lane's activation operands for a 256-element unit are 64 contiguous
// bytes; v_mfma_i32_16x16x64_i8 takes two groups at once from the same
// 16 bytes. The weights keep the layout the GEMV streams; a lane loads 32
// (Q8_0: 64) contiguous bytes of its row per unit and a 4x4 dword transpose
// across the four lane quarters (v_permlane32_swap + v_permlane16_swap,
// register only) hands every lane its dword of each group.
//
// Because a lane's outputs all belong to one weight row, every per-row group
// scale is a lane scalar:
//   Q4_K  sc_g = 8 a_g + b_g with a_g, b_g <= 7, so a_g q and b_g q (<= 105)
//         are int8 planes: eight 16x16x64 MFMAs per unit accumulate
//         H = sum_g a_g dot_g and L = sum_g b_g dot_g, and 8 H + L is FISH's
//         exact sum_g sc_g dot_g; the mins term sum_g m_g bsum_g is two more
//         MFMAs on the split activation sums (bsum = 64 bh + bl, both int8);
//   Q6_K  the two 16-element scales of a group multiply the int32 MFMA sums
//         (24-bit multiplies, exact);
//   Q8_0, Q4_0  f32 per 32-group;
// and the f32 scales are applied once per 32-group (Q8_0, Q4_0) or 256-block
// (K-quants), as in FISH's AVX2 kernels (quant_x86.cpp:280-309, :346-382,
// :445-495).
//
// Q4_0 nibbles and Q6_K codes are made signed per byte without carries:
// (n + 0x78) ^ 0x80 = n - 8 for n in 0..15, (q + 0x60) ^ 0x80 = q - 32 for
// q in 0..63, so the MFMA sums are exactly FISH's sum (n - 8) x and
// sum (q - 32) x.
//
// Workgroup: four wavefronts on consecutive 16-row blocks of one item (or
// token block), all walking the 256-element units of K together. A unit's
// activations for the workgroup's tokens are staged once in a two-slot LDS
// ring (one barrier per unit) and read by all four; each wavefront keeps the
// weights of the next two units in flight in registers. Token blocks past an
// item's count are skipped (uniform branches).
#include "common.h"
#include "kernels.h"

namespace fishhip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned short v2us __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;

__device__ __forceinline__ v4i mfma32(long a, long b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4i mfma64(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Four byte codes (<= 15) times a factor (<= 7) held in both 16-bit halves:
// no product exceeds a byte, so the 16-bit multiplies carry nothing across bytes.
__device__ __forceinline__ uint32_t mul4(uint32_t codes, uint32_t f2) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2us, codes) * __builtin_bit_cast(v2us, f2));
}

// Byte g of x in bytes 0 and 2 (zeros in 1 and 3).
__device__ __forceinline__ uint32_t bcast2(uint32_t x, int g) {
    return __builtin_amdgcn_perm(x, x, uint32_t(g) | (uint32_t(g) << 16) | 0x0C000C00u);
}

__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) {
    return static_cast<long>((static_cast<unsigned long>(hi) << 32) | lo);
}

__device__ __forceinline__ uint32_t nib_lo(uint32_t w) { return w & 0x0F0F0F0Fu; }
__device__ __forceinline__ uint32_t nib_hi(uint32_t w) { return (w >> 4) & 0x0F0F0F0Fu; }
__device__ __forceinline__ uint32_t minus8(uint32_t n) { return (n + 0x78787878u) ^ 0x80808080u; }
__device__ __forceinline__ uint32_t minus32(uint32_t n) { return (n + 0x60606060u) ^ 0x80808080u; }

__device__ __forceinline__ float half_at(const uint4& v, int i) {
    const uint32_t w = (i < 2) ? v.x : (i < 4) ? v.y : (i < 6) ? v.z : v.w;
    return f16_bits_to_f32(uint16_t((i & 1) ? (w >> 16) : (w & 0xFFFF)));
}

__device__ __forceinline__ uint32_t dword_at(const uint4& v, int i) {
    return (i == 0) ? v.x : (i == 1) ? v.y : (i == 2) ? v.z : v.w;
}

__device__ __forceinline__ int byte_u(uint32_t w, int b) { return int((w >> (8 * b)) & 0xFF); }
__device__ __forceinline__ int byte_s(uint32_t w, int b) { return int(int8_t((w >> (8 * b)) & 0xFF)); }

// In-register 4x4 dword transpose across the lane quarters: on entry, quarter
// q holds row q of the matrix in v.x..v.w; on exit component k of quarter q
// holds element (k, q). permlane32_swap exchanges quarters 2,3 of its first
// operand with quarters 0,1 of its second; permlane16_swap exchanges the odd
// quarters of the first with the even quarters of the second.
__device__ __forceinline__ uint4 transpose4(uint4 v) {
    const auto a = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    return make_uint4(c[0], c[1], d[0], d[1]);
}

// Raw weight data of one 256-element unit for one 16-row block (the lane's row).
struct WUnit {
    uint4 v[4];     // codes: Q4 layouts chunks 2q, 2q+1 (v[0..1]); Q8_0 groups 2q, 2q+1 (v[0..3])
    uint4 m;        // Q8_0/Q4_0: 8 f16 group scales; Q4_K / Q5_K: d, dmin, scales; Q6_K: 16 int8 scales
    uint4 hb[2];    // Q5_K: fifth bits of the 8 groups (one dword each)
    uint4 qh[4];    // Q6_K: high bits of the 8 groups (8 bytes each)
    uint32_t d6;    // Q6_K: f16 d
};

// `row` counts from the first row of the expert W points at; every offset
// within one expert's matrix fits 32 bits (checked by the launcher).
template <uint32_t T>
__device__ __forceinline__ void load_w(WUnit& o, const WeightPtrs& W, uint32_t row, int u, int q, int n_in) {
    const uint32_t groups = uint32_t(n_in) / 32, units = uint32_t(n_in) / 256;
    const uint32_t c0 = 8 * uint32_t(u);
    if constexpr (T == kQ8_0) {
        const uint4* p = reinterpret_cast<const uint4*>(W.codes + (row * uint32_t(n_in) + uint32_t(u) * 256 + 64 * q));
#pragma unroll
        for (int i = 0; i < 4; ++i) o.v[i] = p[i];
        o.m = *reinterpret_cast<const uint4*>(W.d + (row * groups + c0));
    } else {
        const uint4* p = reinterpret_cast<const uint4*>(W.codes + (row * groups + c0 + 2 * q) * 16);
        o.v[0] = p[0];
        o.v[1] = p[1];
        if constexpr (T == kQ4_0) {
            o.m = *reinterpret_cast<const uint4*>(W.d + (row * groups + c0));
        } else if constexpr (has_mins(T)) {
            o.m = *reinterpret_cast<const uint4*>(W.aux + (row * units + u) * 16);
            if constexpr (T == kQ5_K) {
                const uint4* h = reinterpret_cast<const uint4*>(W.hb + (row * groups + c0));
                o.hb[0] = h[0];
                o.hb[1] = h[1];
            }
        } else {
            const uint4* h = reinterpret_cast<const uint4*>(W.aux + (row * groups + c0) * 8);
#pragma unroll
            for (int i = 0; i < 4; ++i) o.qh[i] = h[i];
            o.m = *reinterpret_cast<const uint4*>(W.sc + (row * (uint32_t(n_in) / 16) + 16 * u));
            o.d6 = W.d[row * units + u];
        }
    }
}

// The activations of one unit for the workgroup's NB x 16 tokens, staged in
// LDS: codes in MFMA order (token t's 16-byte chunk c at t * 16 + (c ^ (t & 15)),
// so the 16 lanes reading one chunk index hit 16 different bank groups), and
// the f32 scales (K-quants: d of token t; Q8_0 / Q4_0: the 8 group d of token
// t as two float4) and, for Q4_K, the 16 split bsum bytes of token t.
template <uint32_t T, int NB>
struct ALds {
    static constexpr bool kq = kquant_type(T);
    uint4 code[2][NB * 256];
    float dk[2][kq ? NB * 16 : 1];
    uint4 bs[2][has_mins(T) ? NB * 16 : 1];
    float4 da[2][kq ? 1 : NB * 32];
};

// One thread's share of a unit's activations on its way to LDS.
template <int NB>
struct AReg {
    uint4 c0, c1;  // code chunks of token blocks 0 and 1
    uint4 meta;  // Q4_K bsum bytes; Q8_0 / Q4_0 four group d
    float dk;
};

struct AMap {
    uint32_t code_off[2];  // element offset of the activation row of the thread's code chunks
    uint32_t meta_off;     // scale / bsum row offset (units or groups) of the thread's meta token
};

template <uint32_t T, int NB>
__device__ __forceinline__ AReg<NB> load_act(const ActPtrs& A, const AMap& m, int u, int tid) {
    constexpr bool kq = kquant_type(T);
    const int8_t* codes = kq ? A.m256 : A.m32;
    const uint32_t c = uint32_t(u) * 256 + (tid & 15) * 16;
    AReg<NB> r;
    r.c0 = *reinterpret_cast<const uint4*>(codes + (m.code_off[0] + c));
    r.c1 = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (NB > 1) r.c1 = *reinterpret_cast<const uint4*>(codes + (m.code_off[1] + c));
    r.meta = make_uint4(0u, 0u, 0u, 0u);
    r.dk = 0.0f;
    if constexpr (kq) {
        r.dk = A.d256[m.meta_off + u];
        if constexpr (has_mins(T)) r.meta = *reinterpret_cast<const uint4*>(A.bsm + (m.meta_off + u) * 16);
    } else {
        r.meta = *reinterpret_cast<const uint4*>(A.d32 + (m.meta_off + 8 * u + 4 * (tid & 1)));
    }
    return r;
}

template <uint32_t T, int NB>
__device__ __forceinline__ void store_act(ALds<T, NB>& L, int slot, const AReg<NB>& r, int nbu, int tid) {
    const int t0 = tid >> 4, c = tid & 15;
    L.code[slot][t0 * 16 + (c ^ t0)] = r.c0;
    if constexpr (NB > 1)
        if (nbu > 1) L.code[slot][(t0 + 16) * 16 + (c ^ t0)] = r.c1;
    if constexpr (kquant_type(T)) {
        if (tid < NB * 16) L.dk[slot][tid] = r.dk;
        if constexpr (has_mins(T))
            if (tid >= 128 && tid < 128 + NB * 16) L.bs[slot][tid - 128] = r.meta;
    } else {
        if (tid < NB * 32) L.da[slot][tid] = __builtin_bit_cast(float4, r.meta);
    }
}

// acc[nb][r] += contribution of one unit of one 16-row block (weights w) for
// the staged token blocks nb < nbu. q = lane quarter, j = lane % 16.
template <uint32_t T, int NB>
__device__ __forceinline__ void unit_dot(const WUnit& w, const ALds<T, NB>& L, int slot, int nbu, int q, int j,
                                         const int (&aidx)[4], float (&acc)[NB][4]) {
    // the lane's B operand dwords of the 8 groups (lo: elements 4q..4q+3, hi: 16+4q..16+4q+3)
    uint32_t lo[8], hi[8];
    if constexpr (T == kQ8_0) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint4 l = transpose4(w.v[2 * c]), h = transpose4(w.v[2 * c + 1]);
            lo[c] = l.x; lo[2 + c] = l.y; lo[4 + c] = l.z; lo[6 + c] = l.w;
            hi[c] = h.x; hi[2 + c] = h.y; hi[4 + c] = h.z; hi[6 + c] = h.w;
        }
    } else {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint4 t = transpose4(w.v[c]);
            lo[c] = t.x; lo[2 + c] = t.y; lo[4 + c] = t.z; lo[6 + c] = t.w;
        }
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            hi[g] = nib_hi(lo[g]);
            lo[g] = nib_lo(lo[g]);
        }
    }
    auto act = [&](int nb, uint4 (&av)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) av[i] = L.code[slot][nb * 256 + aidx[i]];
    };
    const v4i zero = {0, 0, 0, 0};

    if constexpr (T == kQ8_0 || T == kQ4_0) {
        long b[8];
        float dw[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            b[g] = (T == kQ8_0) ? pack2(lo[g], hi[g]) : pack2(minus8(lo[g]), minus8(hi[g]));
            dw[g] = half_at(w.m, g);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if (NB > 1 && nb >= nbu) continue;
            uint4 av[4];
            act(nb, av);
            float da[4][8];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float4 x = L.da[slot][(16 * nb + 4 * q + r) * 2], y = L.da[slot][(16 * nb + 4 * q + r) * 2 + 1];
                da[r][0] = x.x; da[r][1] = x.y; da[r][2] = x.z; da[r][3] = x.w;
                da[r][4] = y.x; da[r][5] = y.y; da[r][6] = y.z; da[r][7] = y.w;
            }
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                const uint4& v = av[g >> 1];
                const long a = (g & 1) ? pack2(v.z, v.w) : pack2(v.x, v.y);
                const v4i c = mfma32(a, b[g], zero);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[nb][r] += float(c[r]) * (dw[g] * da[r][g]);
            }
        }
    } else if constexpr (has_mins(T)) {
        const float d = f16_bits_to_f32(uint16_t(w.m.x & 0xFFFF));
        const float dmin = f16_bits_to_f32(uint16_t(w.m.x >> 16));
        const uint32_t sc_lo = w.m.y & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (w.m.w & 0x0F0F0F0Fu) | ((w.m.y >> 2) & 0x30303030u);
        const uint32_t mn_lo = w.m.z & 0x3F3F3F3Fu;
        const uint32_t mn_hi = ((w.m.w >> 4) & 0x0F0F0F0Fu) | ((w.m.z >> 2) & 0x30303030u);
        // sc = 8 a + b: planes a * q and b * q (<= 105) keep the group scales inside the int8 MFMAs
        const uint32_t fa[2] = {(sc_lo >> 3) & 0x07070707u, (sc_hi >> 3) & 0x07070707u};
        const uint32_t fb[2] = {sc_lo & 0x07070707u, sc_hi & 0x07070707u};
        const long m8 = pack2(mn_lo, mn_hi);
        const long mh = (q == 0) ? m8 : 0L, ml = (q == 1) ? m8 : 0L;
        // Q5_K: a third plane sc * (fifth bit) (<= 63), I = 8 H + L + 16 C
        const uint32_t sc2[2] = {sc_lo, sc_hi};
        // each set of planes is formed once and consumed by every staged token block at once
        v4i H[NB], Lo[NB], C[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) H[nb] = Lo[nb] = C[nb] = zero;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int g0 = 2 * i, g1 = 2 * i + 1;
            const uint32_t a0 = bcast2(fa[g0 >> 2], g0 & 3), a1 = bcast2(fa[g1 >> 2], g1 & 3);
            const uint32_t b0 = bcast2(fb[g0 >> 2], g0 & 3), b1 = bcast2(fb[g1 >> 2], g1 & 3);
            const v4i pa = {int(mul4(lo[g0], a0)), int(mul4(hi[g0], a0)), int(mul4(lo[g1], a1)), int(mul4(hi[g1], a1))};
            const v4i pb = {int(mul4(lo[g0], b0)), int(mul4(hi[g0], b0)), int(mul4(lo[g1], b1)), int(mul4(hi[g1], b1))};
            v4i pc = zero;
            if constexpr (T == kQ5_K) {
                // the lane's fifth bits: bit 8b + q (elements 4q + b), bit 8b + 4 + q (16 + 4q + b)
                const uint32_t h0 = dword_at(w.hb[g0 >> 2], g0 & 3), h1 = dword_at(w.hb[g1 >> 2], g1 & 3);
                const uint32_t s0 = bcast2(sc2[g0 >> 2], g0 & 3), s1 = bcast2(sc2[g1 >> 2], g1 & 3);
                pc = v4i{int(mul4((h0 >> q) & 0x01010101u, s0)), int(mul4((h0 >> (4 + q)) & 0x01010101u, s0)),
                         int(mul4((h1 >> q) & 0x01010101u, s1)), int(mul4((h1 >> (4 + q)) & 0x01010101u, s1))};
            }
            const v4i a_0 = __builtin_bit_cast(v4i, L.code[slot][aidx[i]]);
            H[0] = mfma64(a_0, pa, H[0]);
            Lo[0] = mfma64(a_0, pb, Lo[0]);
            if constexpr (T == kQ5_K) C[0] = mfma64(a_0, pc, C[0]);
            if constexpr (NB > 1) {
                if (nbu > 1) {
                    const v4i a_1 = __builtin_bit_cast(v4i, L.code[slot][256 + aidx[i]]);
                    H[1] = mfma64(a_1, pa, H[1]);
                    Lo[1] = mfma64(a_1, pb, Lo[1]);
                    if constexpr (T == kQ5_K) C[1] = mfma64(a_1, pc, C[1]);
                }
            }
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if (NB > 1 && nb >= nbu) continue;
            const uint4 bs4 = L.bs[slot][16 * nb + j];
            const long bsv = (q == 0) ? pack2(bs4.x, bs4.y) : (q == 1) ? pack2(bs4.z, bs4.w) : 0L;
            const v4i ch = mfma32(bsv, mh, zero);
            const v4i cl = mfma32(bsv, ml, zero);
            const float4 dk = *reinterpret_cast<const float4*>(&L.dk[slot][16 * nb + 4 * q]);
            const float dkr[4] = {dk.x, dk.y, dk.z, dk.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int isum = (H[nb][r] << 3) + Lo[nb][r] + (C[nb][r] << 4);
                const int mins = (ch[r] << 6) + cl[r];
                acc[nb][r] += dkr[r] * (d * float(isum) - dmin * float(mins));
            }
        }
    } else {
        const float d = f16_bits_to_f32(uint16_t(w.d6));
        int isum[NB][4];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) isum[nb][r] = 0;
        // each group's operands are formed once and consumed by every staged token block at once
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 av0 = L.code[slot][aidx[i]];
            uint4 av1 = av0;
            if constexpr (NB > 1)
                if (nbu > 1) av1 = L.code[slot][256 + aidx[i]];
            const uint4& h2 = w.qh[i];
            const uint32_t s2 = dword_at(w.m, i);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int g = 2 * i + e;
                const uint32_t qa = e ? h2.z : h2.x, qb = e ? h2.w : h2.y;
                const long ba = pack2(minus32(lo[g] | (((qa >> (2 * q)) & 0x03030303u) << 4)), 0u);
                const long bb = pack2(0u, minus32(hi[g] | (((qb >> (2 * q)) & 0x03030303u) << 4)));
                const int sa = byte_s(s2, 2 * e), sb = byte_s(s2, 2 * e + 1);
                // |x| <= 16 * 32 * 127 and |s| <= 128: exact in the 24-bit multiplier
                {
                    const long a = e ? pack2(av0.z, av0.w) : pack2(av0.x, av0.y);
                    const v4i xa = mfma32(a, ba, zero);
                    const v4i xb = mfma32(a, bb, zero);
#pragma unroll
                    for (int r = 0; r < 4; ++r) isum[0][r] += __mul24(sa, xa[r]) + __mul24(sb, xb[r]);
                }
                if constexpr (NB > 1) {
                    if (nbu > 1) {
                        const long a = e ? pack2(av1.z, av1.w) : pack2(av1.x, av1.y);
                        const v4i xa = mfma32(a, ba, zero);
                        const v4i xb = mfma32(a, bb, zero);
#pragma unroll
                        for (int r = 0; r < 4; ++r) isum[1][r] += __mul24(sa, xa[r]) + __mul24(sb, xb[r]);
                    }
                }
            }
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if (NB > 1 && nb >= nbu) continue;
            const float4 dk = *reinterpret_cast<const float4*>(&L.dk[slot][16 * nb + 4 * q]);
            const float dkr[4] = {dk.x, dk.y, dk.z, dk.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[nb][r] += (d * dkr[r]) * float(isum[nb][r]);
        }
    }
}

// Four wavefronts, each RB blocks of 16 rows, on one item (expert, up to
// 16 NB tokens) or one block of 16 NB tokens, over the whole K.
template <uint32_t T, int RB, int NB>
__global__ __launch_bounds__(64 * kWaves) void batch_mfma_kernel(WeightPtrs W, ActPtrs A, int n_in, int n_out,
                                                                 int n_tok, TokenMap map, float* __restrict__ y,
                                                                 int ldy) {
    constexpr int TOK = 16 * NB;
    constexpr bool kq = kquant_type(T);
    __shared__ ALds<T, NB> L;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, q = lane >> 4;
    const int units = n_in / 256, groups = n_in / 32;

    int s0, cnt;
    if (map.items) {
        const int it = int(blockIdx.y);
        if (it >= *map.n_items) return;  // uniform over the workgroup
        const size_t erow = size_t(map.items[3 * it]) * size_t(n_out);
        s0 = map.items[3 * it + 1];
        cnt = map.items[3 * it + 2];
        // the expert's rows: every further offset is within one expert's matrix
        if constexpr (T == kQ8_0) {
            W.codes += erow * size_t(n_in);
        } else {
            W.codes += erow * size_t(groups) * 16;
        }
        if constexpr (T == kQ8_0 || T == kQ4_0) W.d += erow * size_t(groups);
        if constexpr (has_mins(T)) W.aux += erow * size_t(units) * 16;
        if constexpr (T == kQ5_K) W.hb += erow * size_t(groups);
        if constexpr (T == kQ6_K) {
            W.aux += erow * size_t(groups) * 8;
            W.sc += erow * size_t(n_in / 16);
            W.d += erow * size_t(units);
        }
    } else {
        s0 = int(blockIdx.y) * TOK;
        cnt = min(TOK, n_tok - s0);
    }
    const int nbu = (cnt + 15) >> 4;  // token blocks holding tokens (uniform)
    auto arow_of = [&](int t) -> uint32_t {
        const int tt = (t < cnt) ? t : 0;
        return uint32_t(map.act_row ? map.act_row[s0 + tt] : s0 + tt);
    };
    AMap am;
#pragma unroll
    for (int i = 0; i < 2; ++i) am.code_off[i] = (i < NB) ? arow_of((tid >> 4) + 16 * i) * uint32_t(n_in) : 0u;
    if constexpr (kq) {
        am.meta_off = arow_of(tid & (TOK - 1)) * uint32_t(units);
    } else {
        am.meta_off = arow_of((tid >> 1) & (TOK - 1)) * uint32_t(groups);
    }
    int aidx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) aidx[i] = j * 16 + (((4 * q) ^ j) ^ i);

    const int row0 = (int(blockIdx.x) * kWaves + wave) * 16 * RB;
    uint32_t wrow[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) wrow[rb] = uint32_t(min(row0 + rb * 16 + j, n_out - 1));

    float acc[RB][NB][4];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[rb][nb][r] = 0.0f;

    // Every wavefront takes part in the staging and the barriers; one whose
    // rows all lie past n_out still loads (clamped) rows and stores nothing.
    WUnit w0[RB], w1[RB];
    auto load_ws = [&](WUnit (&w)[RB], int u) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) load_w<T>(w[rb], W, wrow[rb], u, q, n_in);
    };
    auto compute = [&](const WUnit (&w)[RB], int slot) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) unit_dot<T, NB>(w[rb], L, slot, nbu, q, j, aidx, acc[rb]);
    };
    // Prefetches past the last unit reload the last unit (in bounds, unused):
    // every path then has the same loads outstanding, so the waits before
    // each use count only the loads that use needs.
    const int last = units - 1;
    AReg<NB> ra = load_act<T, NB>(A, am, 0, tid);
    __builtin_amdgcn_sched_barrier(0);
    load_ws(w0, 0);
    __builtin_amdgcn_sched_barrier(0);
    load_ws(w1, min(1, last));
    __builtin_amdgcn_sched_barrier(0);
    store_act<T, NB>(L, 0, ra, nbu, tid);
    __builtin_amdgcn_sched_barrier(0);
    ra = load_act<T, NB>(A, am, min(1, last), tid);
    __syncthreads();
    // unit u: weights in w[u & 1], activations in LDS slot u & 1; the loads of
    // unit u + 1's activations and unit u + 2's weights are in flight
    // (the scheduling fences keep the loads in this order, which the waits rely on)
    int u = 0;
    for (; u + 2 <= units; u += 2) {
        compute(w0, 0);
        __builtin_amdgcn_sched_barrier(0);
        load_ws(w0, min(u + 2, last));
        __builtin_amdgcn_sched_barrier(0);
        store_act<T, NB>(L, 1, ra, nbu, tid);
        __builtin_amdgcn_sched_barrier(0);
        ra = load_act<T, NB>(A, am, min(u + 2, last), tid);
        __syncthreads();
        compute(w1, 1);
        __builtin_amdgcn_sched_barrier(0);
        load_ws(w1, min(u + 3, last));
        __builtin_amdgcn_sched_barrier(0);
        if (u + 2 < units) store_act<T, NB>(L, 0, ra, nbu, tid);
        __builtin_amdgcn_sched_barrier(0);
        ra = load_act<T, NB>(A, am, min(u + 3, last), tid);
        __syncthreads();
    }
    if (u < units) compute(w0, 0);  // odd count: the last unit is in w0 and slot 0

#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int row = row0 + rb * 16 + j;
        if (row >= n_out) continue;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * nb + 4 * q + r;
                if (t < cnt) y[size_t(s0 + t) * ldy + row] = acc[rb][nb][r];
            }
    }
}

template <uint32_t T, int RB, int NB>
hipError_t batch_launch(const WeightPtrs& W, const ActPtrs& A, int n_in, int n_out, int n_tok, const TokenMap& map,
                        int y_blocks, float* y, int ldy, hipStream_t s) {
    constexpr int ROWS_WG = 16 * RB * kWaves, TOK = 16 * NB;
    const unsigned gy = map.items ? unsigned(y_blocks) : unsigned((n_tok + TOK - 1) / TOK);
    const dim3 grid(unsigned((n_out + ROWS_WG - 1) / ROWS_WG), gy);
    hipLaunchKernelGGL((batch_mfma_kernel<T, RB, NB>), grid, dim3(64 * kWaves), 0, s, W, A, n_in, n_out, n_tok, map,
                       y, ldy);
    return hipGetLastError();
}

#define BATCH_ARGS W, A, n_in, n_out, n_tok, map, y_blocks, y, ldy, s
#define BATCH_PARAMS                                                                                              \
    const WeightPtrs &W, const ActPtrs &A, int n_in, int n_out, int n_tok, const TokenMap &map, int y_blocks, \
        float *y, int ldy, hipStream_t s

template <uint32_t T>
hipError_t batch_pick(int tok_per_wg, BATCH_PARAMS) {
    if (tok_per_wg <= 16) return batch_launch<T, 1, 1>(BATCH_ARGS);
    return batch_launch<T, 1, 2>(BATCH_ARGS);
}

}  // namespace

bool batch_mfma_supported(const WeightLayout& WL) { return WL.total && WL.n_in % 256 == 0; }

hipError_t launch_batch_mfma(const void* w, const WeightLayout& WL, const void* act, int act_rows, int n_tok, float* y,
                             int ldy, hipStream_t s, const TokenMap* group, int item_tokens, int max_items) {
    const ActLayout AL = act_layout(act_rows, WL.n_in);
    if (!batch_mfma_supported(WL) || !AL.total || !AL.has256 || n_tok <= 0) return hipErrorInvalidValue;
    if (group && (item_tokens <= 0 || item_tokens > kBatchItemTokens)) return hipErrorInvalidValue;
    const WeightPtrs W = weight_ptrs(w, WL);
    const ActPtrs A = act_ptrs(act, AL);
    TokenMap map{};
    int tok = n_tok, yb = 0, n_out = WL.n_out;
    if (group) {
        map = *group;
        tok = item_tokens;
        yb = max_items;
        n_out = map.rows_per_expert;
    }
    // the kernel forms offsets within one expert's matrix and one activation plane in 32 bits
    if (uint64_t(n_out) * uint64_t(WL.n_in) > 0xFFFFFFFFull || uint64_t(act_rows) * uint64_t(WL.n_in) > 0xFFFFFFFFull)
        return hipErrorInvalidValue;
    switch (WL.type) {
        case kQ8_0: return batch_pick<kQ8_0>(tok, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        case kQ4_0: return batch_pick<kQ4_0>(tok, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        case kQ4_K: return batch_pick<kQ4_K>(tok, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        case kQ5_K: return batch_pick<kQ5_K>(tok, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        case kQ6_K: return batch_pick<kQ6_K>(tok, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace fishhip
