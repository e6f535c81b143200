// One weight row's 32-element groups against one token's int8 activations,
// for the decode-shape kernels (GEMV, fused GEMV, single-token expert FFN):
// loading a group of the repacked weights, loading the token's matching
// activation group, and the group's f32 contribution from its exact integer
// dot (dots.h).
#pragma once

#include "common.h"
#include "dots.h"
#include "qact.h"

namespace fishhip {

struct Frag {
    uint4 w0, w1;   // codes (Q8_0 uses both)
    uint4 meta;     // Q4_K: d, dmin, scales[12]
    uint2 qh;       // Q6_K high bits
    uint32_t hb;    // Q5_K fifth bits
    uint32_t raw;   // as loaded: f16 d (Q8_0, Q4_0, Q6_K); one Q4_K meta dword (wavefront form)
    uint32_t raw2;  // as loaded: Q6_K's two int8 16-group scales
    float d, dmin;  // f32 weight scales
    int sca, scb;   // integer group scales (Q4_K / Q5_K: sc, min; Q6_K: two 16-group scales)
};

// Loads of one group, with no arithmetic on what they return, so that a
// caller can issue every load of a wavefront before the first wait (the
// memory counter is waited on in order: decoding one group right after its
// load would serialise the loads behind it). finish_group decodes.
// WAVE (Q4_K / Q5_K only): for wavefront-synchronous callers whose lanes 8j..8j+7
// hold the eight groups of one super-block (lane sub takes groups sub,
// sub + LPR, ... with LPR a multiple of 8): the meta is loaded as one dword
// per lane and assembled with four shuffles in finish_group, so a wavefront
// moves 4 instead of 16 meta bytes per lane.
typedef unsigned ntv4 __attribute__((ext_vector_type(4)));

// A 16-byte weight load, non-temporal (streamed past the caches' retention) when NT.
template <bool NT>
__device__ __forceinline__ uint4 load16(const uint8_t* p) {
    if constexpr (NT) {
        const ntv4 v = __builtin_nontemporal_load(reinterpret_cast<const ntv4*>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return *reinterpret_cast<const uint4*>(p);
    }
}

// NT: non-temporal code loads (Q8_0 / Q4_0; measured per kernel shape).
template <uint32_t T, bool WAVE, bool NT = false>
__device__ __forceinline__ Frag load_group_raw(const WeightPtrs& W, int row, int c, int n_in, int lane) {
    Frag f{};
    const size_t gi = size_t(row) * (n_in / 32) + c;
    if constexpr (T == kQ8_0) {
        const uint4* p = reinterpret_cast<const uint4*>(W.codes + size_t(row) * n_in + size_t(c) * 32);
        f.w0 = load16<NT>(reinterpret_cast<const uint8_t*>(p));
        f.w1 = load16<NT>(reinterpret_cast<const uint8_t*>(p + 1));
        f.raw = W.d[gi];
    } else if constexpr (T == kQ4_0) {
        f.w0 = load16<NT>(W.codes + gi * 16);
        f.raw = W.d[gi];
    } else if constexpr (has_mins(T)) {
        f.w0 = *reinterpret_cast<const uint4*>(W.codes + gi * 16);
        if constexpr (T == kQ5_K) f.hb = W.hb[gi];
        const uint8_t* m = W.aux + (size_t(row) * (n_in / 256) + (c >> 3)) * 16;
        if constexpr (WAVE) f.raw = reinterpret_cast<const uint32_t*>(m)[lane & 3];
        else f.meta = *reinterpret_cast<const uint4*>(m);
    } else {
        f.w0 = *reinterpret_cast<const uint4*>(W.codes + gi * 16);
        f.qh = *reinterpret_cast<const uint2*>(W.aux + gi * 8);
        f.raw2 = *reinterpret_cast<const uint16_t*>(W.sc + size_t(row) * (n_in / 16) + 2 * c);
        f.raw = W.d[size_t(row) * (n_in / 256) + (c >> 3)];
    }
    return f;
}

// The same loads in two parts, for callers that decode the scales while other
// work waits on the codes: every group's scale data first (load_group_scales),
// then every group's codes (load_group_codes); a wait for the scales then does
// not wait for the codes issued after them.
template <uint32_t T, bool WAVE>
__device__ __forceinline__ void load_group_scales(Frag& f, const WeightPtrs& W, int row, int c, int n_in, int lane) {
    const size_t gi = size_t(row) * (n_in / 32) + c;
    if constexpr (T == kQ8_0 || T == kQ4_0) {
        f.raw = W.d[gi];
    } else if constexpr (has_mins(T)) {
        const uint8_t* m = W.aux + (size_t(row) * (n_in / 256) + (c >> 3)) * 16;
        if constexpr (WAVE) f.raw = reinterpret_cast<const uint32_t*>(m)[lane & 3];
        else f.meta = *reinterpret_cast<const uint4*>(m);
    } else {
        f.raw2 = *reinterpret_cast<const uint16_t*>(W.sc + size_t(row) * (n_in / 16) + 2 * c);
        f.raw = W.d[size_t(row) * (n_in / 256) + (c >> 3)];
    }
}
template <uint32_t T, bool NT = false>
__device__ __forceinline__ void load_group_codes(Frag& f, const WeightPtrs& W, int row, int c, int n_in) {
    const size_t gi = size_t(row) * (n_in / 32) + c;
    if constexpr (T == kQ8_0) {
        const uint8_t* p = W.codes + size_t(row) * n_in + size_t(c) * 32;
        f.w0 = load16<NT>(p);
        f.w1 = load16<NT>(p + 16);
    } else if constexpr (T == kQ4_0) {
        f.w0 = load16<NT>(W.codes + gi * 16);
    } else if constexpr (has_mins(T)) {
        f.w0 = *reinterpret_cast<const uint4*>(W.codes + gi * 16);
        if constexpr (T == kQ5_K) f.hb = W.hb[gi];
    } else {
        f.w0 = *reinterpret_cast<const uint4*>(W.codes + gi * 16);
        f.qh = *reinterpret_cast<const uint2*>(W.aux + gi * 8);
    }
}

// Decodes the scales of a group loaded by load_group_raw<T, WAVE> or
// load_group_scales<T, WAVE> (group index c; every lane of the wavefront calls
// it in the WAVE form).
template <uint32_t T, bool WAVE>
__device__ __forceinline__ void finish_group(Frag& f, int c, int lane) {
    if constexpr (T == kQ8_0 || T == kQ4_0) {
        f.d = f16_bits_to_f32(uint16_t(f.raw));
    } else if constexpr (has_mins(T)) {
        if constexpr (WAVE) {
            const int base = lane & ~7;
            f.meta = make_uint4(__shfl(f.raw, base), __shfl(f.raw, base + 1), __shfl(f.raw, base + 2),
                                __shfl(f.raw, base + 3));
        }
        f.d = f16_bits_to_f32(uint16_t(f.meta.x & 0xFFFF));
        f.dmin = f16_bits_to_f32(uint16_t(f.meta.x >> 16));
        k4_scale_min(f.meta.y, f.meta.z, f.meta.w, c & 7, f.sca, f.scb);
    } else {
        f.sca = int(int8_t(f.raw2 & 0xFF));
        f.scb = int(int8_t(f.raw2 >> 8));
        f.d = f16_bits_to_f32(uint16_t(f.raw));
    }
}

// One group, loaded and decoded (callers that handle one group at a time).
template <uint32_t T>
__device__ __forceinline__ Frag load_group(const WeightPtrs& W, int row, int c, int n_in) {
    Frag f = load_group_raw<T, false>(W, row, c, n_in, 0);
    finish_group<T, false>(f, c, 0);
    return f;
}

// Activation side of one 32-element group for one token.
struct ActFrag {
    uint4 a0, a1;  // 32 int8 codes
    float d;       // Q8Act d (32-layouts) or Q8ActK d of the super-block
    int s, s2;     // Q4_0: block sum; K-quants: the two per-16 sums
};

template <uint32_t T>
__device__ __forceinline__ ActFrag load_act(const ActPtrs& A, int t, int c, int n_in) {
    ActFrag a;
    if constexpr (!kquant_type(T)) {
        const uint4* p = reinterpret_cast<const uint4*>(A.q32 + size_t(t) * n_in + size_t(c) * 32);
        a.a0 = p[0];
        a.a1 = p[1];
        const size_t bi = size_t(t) * (n_in / 32) + c;
        a.d = A.d32[bi];
        a.s = (T == kQ4_0) ? A.s32[bi] : 0;
        a.s2 = 0;
    } else {
        const uint4* p = reinterpret_cast<const uint4*>(A.q256 + size_t(t) * n_in + size_t(c) * 32);
        a.a0 = p[0];
        a.a1 = p[1];
        a.d = A.d256[size_t(t) * (n_in / 256) + (c >> 3)];
        const uint32_t s2 = *reinterpret_cast<const uint32_t*>(A.s16 + size_t(t) * (n_in / 16) + 2 * c);
        a.s = int(int16_t(s2 & 0xFFFF));
        a.s2 = int(int16_t(s2 >> 16));
    }
    return a;
}

// f32 contribution of one group (weights f, activations a).
template <uint32_t T>
__device__ __forceinline__ float group_dot(const Frag& f, const ActFrag& a) {
    if constexpr (T == kQ8_0) {
        return float(isum_q8_0(f.w0, f.w1, a.a0, a.a1)) * (f.d * a.d);
    } else if constexpr (T == kQ4_0) {
        return float(isum_q4_0(f.w0, a.a0, a.a1, a.s)) * (f.d * a.d);
    } else if constexpr (has_mins(T)) {
        const int sumi = f.sca * (T == kQ4_K ? dot_q4_k(f.w0, a.a0, a.a1) : dot_q5_k(f.w0, f.hb, a.a0, a.a1));
        const int mins = f.scb * (a.s + a.s2);
        return a.d * (f.d * float(sumi) - f.dmin * float(mins));
    } else {
        const int sumi = isum_q6_k(f.w0, f.qh, a.a0, a.a1, a.s, a.s2, f.sca, f.scb);
        return (f.d * a.d) * float(sumi);
    }
}

// Rows per wavefront: about BYTES of weights in flight per lane.
template <uint32_t T, int MAXC, int BYTES = 64>
constexpr int gemv_rb() {
    constexpr int per_group = (T == kQ8_0) ? 32 : 16;
    constexpr int rb = BYTES / (per_group * MAXC);
    return rb < 1 ? 1 : (rb > 8 ? 8 : rb);
}


// The activation side of group c from a workgroup's LDS copy (qact.h).
template <uint32_t T>
__device__ __forceinline__ ActFrag lds_act(const LdsAct& L, int c) {
    ActFrag a;
    a.a0 = L.codes[c];
    a.a1 = L.codes[L.maxg + c];
    if constexpr (!kquant_type(T)) {
        a.d = L.d[c];
        a.s = L.s[c];
        a.s2 = 0;
    } else {
        a.d = L.d[c >> 3];
        const int s2 = L.s[c];
        a.s = int(int16_t(s2 & 0xFFFF));
        a.s2 = s2 >> 16;
    }
    return a;
}

}  // namespace fishhip
