// Decode-shape matmul (few tokens) over the repacked weights, judged as a
// memory-bound kernel: every weight byte is read once with 128-bit loads.
//
// y[t][i] = dot(W_i, x_t) for t < n_tok (matmul_batch, ops.cpp:177-216).
// A group of LPR lanes owns one output row; lane `sub` of the group takes the
// row's 32-element groups sub, sub+LPR, ... so one load instruction of the
// wavefront covers LPR consecutive 16-byte chunks of a row. The lane computes
// each group's exact integer dot (dots.h) and scales it in f32; the LPR
// partial sums are reduced with cross-lane shuffles at the end. Activations
// (a few KB) are read through the caches; the weights stream past once.
//
// Also here: the per-block integer dump used by the parity tests, built from
// the same dots.h functions.
#include "common.h"
#include "dots.h"
#include "kernels.h"

namespace fishhip {

namespace {

struct Frag {
    uint4 w0, w1;   // codes (Q8_0 uses both)
    uint4 meta;     // Q4_K: d, dmin, scales[12]
    uint2 qh;       // Q6_K high bits
    float d, dmin;  // f32 weight scales
    int sca, scb;   // integer group scales (Q4_K: sc, min; Q6_K: two 16-group scales)
};

template <uint32_t T>
__device__ __forceinline__ Frag load_group(const WeightPtrs& W, int row, int c, int n_in) {
    Frag f{};
    const int groups = n_in / 32;
    const size_t gi = size_t(row) * groups + c;
    if constexpr (T == kQ8_0) {
        const uint4* p = reinterpret_cast<const uint4*>(W.codes + size_t(row) * n_in + size_t(c) * 32);
        f.w0 = p[0];
        f.w1 = p[1];
        f.d = f16_bits_to_f32(W.d[gi]);
    } else if constexpr (T == kQ4_0) {
        f.w0 = *reinterpret_cast<const uint4*>(W.codes + gi * 16);
        f.d = f16_bits_to_f32(W.d[gi]);
    } else if constexpr (T == kQ4_K) {
        f.w0 = *reinterpret_cast<const uint4*>(W.codes + gi * 16);
        f.meta = *reinterpret_cast<const uint4*>(W.aux + (size_t(row) * (n_in / 256) + (c >> 3)) * 16);
        f.d = f16_bits_to_f32(uint16_t(f.meta.x & 0xFFFF));
        f.dmin = f16_bits_to_f32(uint16_t(f.meta.x >> 16));
        k4_scale_min(f.meta.y, f.meta.z, f.meta.w, c & 7, f.sca, f.scb);
    } else {
        f.w0 = *reinterpret_cast<const uint4*>(W.codes + gi * 16);
        f.qh = *reinterpret_cast<const uint2*>(W.aux + gi * 8);
        const uint16_t s2 = *reinterpret_cast<const uint16_t*>(W.sc + size_t(row) * (n_in / 16) + 2 * c);
        f.sca = int(int8_t(s2 & 0xFF));
        f.scb = int(int8_t(s2 >> 8));
        f.d = f16_bits_to_f32(W.d[size_t(row) * (n_in / 256) + (c >> 3)]);
    }
    return f;
}

// f32 contribution of group c of a row for token t.
template <uint32_t T>
__device__ __forceinline__ float group_dot(const Frag& f, const ActPtrs& A, int t, int c, int n_in) {
    if constexpr (T == kQ8_0 || T == kQ4_0) {
        const uint4* a = reinterpret_cast<const uint4*>(A.q32 + size_t(t) * n_in + size_t(c) * 32);
        const uint4 a0 = a[0], a1 = a[1];
        const size_t bi = size_t(t) * (n_in / 32) + c;
        const float s = f.d * A.d32[bi];
        int isum;
        if constexpr (T == kQ8_0) isum = isum_q8_0(f.w0, f.w1, a0, a1);
        else isum = isum_q4_0(f.w0, a0, a1, A.s32[bi]);
        return float(isum) * s;
    } else {
        const uint4* a = reinterpret_cast<const uint4*>(A.q256 + size_t(t) * n_in + size_t(c) * 32);
        const uint4 a0 = a[0], a1 = a[1];
        const float xd = A.d256[size_t(t) * (n_in / 256) + (c >> 3)];
        const uint32_t s2 = *reinterpret_cast<const uint32_t*>(A.s16 + size_t(t) * (n_in / 16) + 2 * c);
        const int s16a = int(int16_t(s2 & 0xFFFF)), s16b = int(int16_t(s2 >> 16));
        if constexpr (T == kQ4_K) {
            const int sumi = f.sca * dot_q4_k(f.w0, a0, a1);
            const int mins = f.scb * (s16a + s16b);
            return xd * (f.d * float(sumi) - f.dmin * float(mins));
        } else {
            const int sumi = isum_q6_k(f.w0, f.qh, a0, a1, s16a, s16b, f.sca, f.scb);
            return (f.d * xd) * float(sumi);
        }
    }
}

template <uint32_t T, int NT, int LPR, int U>
__global__ __launch_bounds__(256) void gemv_kernel(WeightPtrs W, ActPtrs A, int n_in, int n_out, int n_tok,
                                                   float* __restrict__ y, int ldy) {
    constexpr int RPW = 64 / LPR;  // rows per wavefront
    const int lane = threadIdx.x & 63;
    const int sub = lane % LPR;
    const int row = (int(blockIdx.x) * 4 + int(threadIdx.x >> 6)) * RPW + lane / LPR;
    const int t0 = int(blockIdx.y) * NT;
    if (row >= n_out) return;  // whole LPR groups leave together
    const int groups = n_in / 32;
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;

    for (int c0 = sub; c0 < groups; c0 += LPR * U) {
        Frag f[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u * LPR;
            if (c < groups) f[u] = load_group<T>(W, row, c, n_in);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u * LPR;
            if (c < groups) {
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    if (t0 + t < n_tok) acc[t] += group_dot<T>(f[u], A, t0 + t, c, n_in);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float v = acc[t];
#pragma unroll
        for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
        acc[t] = v;
    }
    if (sub == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
            if (t0 + t < n_tok) y[size_t(t0 + t) * ldy + row] = acc[t];
    }
}

// Per-block integers for token 0 of A: Q8_0/Q4_0 one per 32-block; Q4_K two
// per super-block (sum_g sc_g dot_g, sum_g m_g bsum_g); Q6_K one per super-block.
template <uint32_t T>
__global__ void block_ints_kernel(WeightPtrs W, ActPtrs A, int n_in, int n_out, int32_t* __restrict__ out) {
    const long gid = long(blockIdx.x) * blockDim.x + threadIdx.x;
    constexpr bool kq = (T == kQ4_K || T == kQ6_K);
    const int per_row = kq ? n_in / 256 : n_in / 32;
    if (gid >= long(n_out) * per_row) return;
    const int row = int(gid / per_row), b = int(gid % per_row);
    if constexpr (!kq) {
        const Frag f = load_group<T>(W, row, b, n_in);
        const uint4* a = reinterpret_cast<const uint4*>(A.q32 + size_t(b) * 32);
        if constexpr (T == kQ8_0) out[gid] = isum_q8_0(f.w0, f.w1, a[0], a[1]);
        else out[gid] = isum_q4_0(f.w0, a[0], a[1], A.s32[b]);
    } else {
        int sumi = 0, mins = 0;
        for (int g = 0; g < 8; ++g) {
            const int c = 8 * b + g;
            const Frag f = load_group<T>(W, row, c, n_in);
            const uint4* a = reinterpret_cast<const uint4*>(A.q256 + size_t(c) * 32);
            const int s16a = A.s16[2 * c], s16b = A.s16[2 * c + 1];
            if constexpr (T == kQ4_K) {
                sumi += f.sca * dot_q4_k(f.w0, a[0], a[1]);
                mins += f.scb * (s16a + s16b);
            } else {
                sumi += isum_q6_k(f.w0, f.qh, a[0], a[1], s16a, s16b, f.sca, f.scb);
            }
        }
        if constexpr (T == kQ4_K) {
            out[2 * gid] = sumi;
            out[2 * gid + 1] = mins;
        } else {
            out[gid] = sumi;
        }
    }
}

template <uint32_t T, int NT, int LPR>
hipError_t gemv_launch(const WeightPtrs& W, const ActPtrs& A, int n_in, int n_out, int n_tok, float* y, int ldy,
                       hipStream_t s) {
    constexpr int U = (T == kQ8_0) ? 2 : 4;
    const int rows_per_block = 4 * (64 / LPR);
    const dim3 grid(unsigned((n_out + rows_per_block - 1) / rows_per_block), unsigned((n_tok + NT - 1) / NT));
    hipLaunchKernelGGL((gemv_kernel<T, NT, LPR, U>), grid, dim3(256), 0, s, W, A, n_in, n_out, n_tok, y, ldy);
    return hipGetLastError();
}

template <uint32_t T, int NT>
hipError_t gemv_pick_lpr(const WeightPtrs& W, const ActPtrs& A, int n_in, int n_out, int n_tok, float* y, int ldy,
                         hipStream_t s) {
    const int groups = n_in / 32;
    if (groups >= 64) return gemv_launch<T, NT, 64>(W, A, n_in, n_out, n_tok, y, ldy, s);
    if (groups >= 32) return gemv_launch<T, NT, 32>(W, A, n_in, n_out, n_tok, y, ldy, s);
    if (groups >= 16) return gemv_launch<T, NT, 16>(W, A, n_in, n_out, n_tok, y, ldy, s);
    return gemv_launch<T, NT, 8>(W, A, n_in, n_out, n_tok, y, ldy, s);
}

template <uint32_t T>
hipError_t gemv_pick_nt(const WeightPtrs& W, const ActPtrs& A, int n_in, int n_out, int n_tok, float* y, int ldy,
                        hipStream_t s) {
    if (n_tok <= 1) return gemv_pick_lpr<T, 1>(W, A, n_in, n_out, n_tok, y, ldy, s);
    if (n_tok <= 2) return gemv_pick_lpr<T, 2>(W, A, n_in, n_out, n_tok, y, ldy, s);
    if (n_tok <= 4) return gemv_pick_lpr<T, 4>(W, A, n_in, n_out, n_tok, y, ldy, s);
    return gemv_pick_lpr<T, 8>(W, A, n_in, n_out, n_tok, y, ldy, s);
}

}  // namespace

hipError_t launch_gemv(const void* w, const WeightLayout& WL, const void* act, int n_tok, float* y, int ldy,
                       hipStream_t s) {
    const ActLayout AL = act_layout(n_tok, WL.n_in);
    if (!WL.total || !AL.total || n_tok <= 0) return hipErrorInvalidValue;
    if (is_kquant(WL.type) && !AL.has256) return hipErrorInvalidValue;
    const WeightPtrs W = weight_ptrs(w, WL);
    const ActPtrs A = act_ptrs(act, AL);
    switch (WL.type) {
        case kQ8_0: return gemv_pick_nt<kQ8_0>(W, A, WL.n_in, WL.n_out, n_tok, y, ldy, s);
        case kQ4_0: return gemv_pick_nt<kQ4_0>(W, A, WL.n_in, WL.n_out, n_tok, y, ldy, s);
        case kQ4_K: return gemv_pick_nt<kQ4_K>(W, A, WL.n_in, WL.n_out, n_tok, y, ldy, s);
        case kQ6_K: return gemv_pick_nt<kQ6_K>(W, A, WL.n_in, WL.n_out, n_tok, y, ldy, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_block_ints(const void* w, const WeightLayout& WL, const void* act, int32_t* out, hipStream_t s) {
    const ActLayout AL = act_layout(1, WL.n_in);
    if (!WL.total || !AL.total) return hipErrorInvalidValue;
    const WeightPtrs W = weight_ptrs(w, WL);
    const ActPtrs A = act_ptrs(act, AL);
    const bool kq = is_kquant(WL.type);
    const long items = long(WL.n_out) * (kq ? WL.n_in / 256 : WL.n_in / 32);
    const dim3 grid(unsigned((items + 255) / 256)), block(256);
    switch (WL.type) {
        case kQ8_0: hipLaunchKernelGGL(block_ints_kernel<kQ8_0>, grid, block, 0, s, W, A, WL.n_in, WL.n_out, out); break;
        case kQ4_0: hipLaunchKernelGGL(block_ints_kernel<kQ4_0>, grid, block, 0, s, W, A, WL.n_in, WL.n_out, out); break;
        case kQ4_K: hipLaunchKernelGGL(block_ints_kernel<kQ4_K>, grid, block, 0, s, W, A, WL.n_in, WL.n_out, out); break;
        case kQ6_K: hipLaunchKernelGGL(block_ints_kernel<kQ6_K>, grid, block, 0, s, W, A, WL.n_in, WL.n_out, out); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace fishhip
