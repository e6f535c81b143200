// Decode-shape matmul (few tokens) over the repacked weights, judged as a
// memory-bound kernel: every weight byte is read once with 128-bit loads.
//
// y[t][i] = dot(W_i, x_t) for t < n_tok (matmul_batch, ops.cpp:177-216).
// A group of LPR lanes owns one output row; lane `sub` of the group takes the
// row's 32-element groups sub, sub+LPR, ... so one load instruction of the
// wavefront covers LPR consecutive 16-byte chunks of a row. The lane computes
// each group's exact integer dot (dots.h) and scales it in f32; the LPR
// partial sums are reduced with cross-lane shuffles at the end. Each
// wavefront walks several rows with their loads issued together; for a single
// token its activation groups are loaded once into registers, otherwise they
// are read through the caches. The weights stream past once.
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

// Activation side of one 32-element group for one token.
struct ActFrag {
    uint4 a0, a1;  // 32 int8 codes
    float d;       // Q8Act d (32-layouts) or Q8ActK d of the super-block
    int s, s2;     // Q4_0: block sum; K-quants: the two per-16 sums
};

template <uint32_t T>
__device__ __forceinline__ ActFrag load_act(const ActPtrs& A, int t, int c, int n_in) {
    ActFrag a;
    if constexpr (T == kQ8_0 || T == kQ4_0) {
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
    } else if constexpr (T == kQ4_K) {
        const int sumi = f.sca * dot_q4_k(f.w0, a.a0, a.a1);
        const int mins = f.scb * (a.s + a.s2);
        return a.d * (f.d * float(sumi) - f.dmin * float(mins));
    } else {
        const int sumi = isum_q6_k(f.w0, f.qh, a.a0, a.a1, a.s, a.s2, f.sca, f.scb);
        return (f.d * a.d) * float(sumi);
    }
}

// Wavefront-row scheme: LPR lanes per row; a wavefront owns RPW = 64/LPR
// interleaved rows per pass and `rpw` passes, RB passes at a time with all of
// their weight loads in flight together. Lane `sub` covers groups
// sub, sub + LPR, ... (at most MAXC of them). For one token the lane's
// activation groups stay in registers for every row of the wavefront.
// blockIdx.y selects up to NT tokens: consecutive rows of the batch, or one
// item of an expert work list (TokenMap).
template <uint32_t T, int NT, int LPR, int MAXC, int RB>
__global__ __launch_bounds__(256) void gemv_kernel(WeightPtrs W, ActPtrs A, int n_in, int n_out, int n_tok, int rpw,
                                                   TokenMap map, float* __restrict__ y, int ldy) {
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int sub = lane % LPR;
    const int wave_id = int(blockIdx.x) * 4 + int(threadIdx.x >> 6);
    const int row_base = wave_id * rpw * RPW + lane / LPR;
    const int groups = n_in / 32;

    int s0, cnt;
    size_t wrow0 = 0;  // first weight row of the expert
    if (map.items) {
        const int it = int(blockIdx.y);
        if (it >= *map.n_items) return;
        wrow0 = size_t(map.items[3 * it]) * size_t(n_out);
        s0 = map.items[3 * it + 1];
        cnt = map.items[3 * it + 2];
    } else {
        s0 = int(blockIdx.y) * NT;
        cnt = min(NT, n_tok - s0);
    }
    int arow[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) arow[t] = (t < cnt) ? (map.act_row ? map.act_row[s0 + t] : s0 + t) : 0;

    ActFrag ac[NT == 1 ? MAXC : 1];
    if constexpr (NT == 1) {
#pragma unroll
        for (int k = 0; k < MAXC; ++k) {
            const int c = sub + k * LPR;
            if (c < groups) ac[k] = load_act<T>(A, arow[0], c, n_in);
        }
    }

    for (int p0 = 0; p0 < rpw; p0 += RB) {
        Frag f[RB][MAXC];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int row = row_base + (p0 + rb) * RPW;
#pragma unroll
            for (int k = 0; k < MAXC; ++k) {
                const int c = sub + k * LPR;
                if (row < n_out && c < groups) f[rb][k] = load_group<T>(W, int(wrow0) + row, c, n_in);
            }
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int row = row_base + (p0 + rb) * RPW;
            float acc[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
#pragma unroll
            for (int k = 0; k < MAXC; ++k) {
                const int c = sub + k * LPR;
                if (row < n_out && c < groups) {
                    if constexpr (NT == 1) {
                        acc[0] += group_dot<T>(f[rb][k], ac[k]);
                    } else {
#pragma unroll
                        for (int t = 0; t < NT; ++t)
                            if (t < cnt) acc[t] += group_dot<T>(f[rb][k], load_act<T>(A, arow[t], c, n_in));
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
            if (sub == 0 && row < n_out) {
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    if (t < cnt) y[size_t(s0 + t) * ldy + row] = acc[t];
            }
        }
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
        const ActFrag a = load_act<T>(A, 0, b, n_in);
        if constexpr (T == kQ8_0) out[gid] = isum_q8_0(f.w0, f.w1, a.a0, a.a1);
        else out[gid] = isum_q4_0(f.w0, a.a0, a.a1, a.s);
    } else {
        int sumi = 0, mins = 0;
        for (int g = 0; g < 8; ++g) {
            const int c = 8 * b + g;
            const Frag f = load_group<T>(W, row, c, n_in);
            const ActFrag a = load_act<T>(A, 0, c, n_in);
            if constexpr (T == kQ4_K) {
                sumi += f.sca * dot_q4_k(f.w0, a.a0, a.a1);
                mins += f.scb * (a.s + a.s2);
            } else {
                sumi += isum_q6_k(f.w0, f.qh, a.a0, a.a1, a.s, a.s2, f.sca, f.scb);
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

template <uint32_t T, int NT, int LPR, int MAXC>
hipError_t gemv_launch(const WeightPtrs& W, const ActPtrs& A, int n_in, int n_out, int n_tok, const TokenMap& map,
                       int y_blocks, float* y, int ldy, hipStream_t s) {
    constexpr int RPW = 64 / LPR;
    constexpr int RB = (NT == 1) ? (MAXC <= 2 ? 4 : (MAXC <= 4 ? 2 : 2)) : 1;
    // passes per wavefront: enough rows that ~4096 wavefronts cover the matrix
    const int row_groups = (n_out + RPW - 1) / RPW;
    const int rpw = RB * ((row_groups + RB * 4096 - 1) / (RB * 4096));
    const int waves = (row_groups + rpw - 1) / rpw;
    const unsigned gy = map.items ? unsigned(y_blocks) : unsigned((n_tok + NT - 1) / NT);
    const dim3 grid(unsigned((waves + 3) / 4), gy);
    hipLaunchKernelGGL((gemv_kernel<T, NT, LPR, MAXC, RB>), grid, dim3(256), 0, s, W, A, n_in, n_out, n_tok, rpw, map,
                       y, ldy);
    return hipGetLastError();
}

#define GEMV_ARGS W, A, n_in, n_out, n_tok, map, y_blocks, y, ldy, s
#define GEMV_PARAMS                                                                                                \
    const WeightPtrs &W, const ActPtrs &A, int n_in, int n_out, int n_tok, const TokenMap &map, int y_blocks, \
        float *y, int ldy, hipStream_t s

template <uint32_t T, int NT, int LPR>
hipError_t gemv_pick_maxc(GEMV_PARAMS) {
    const int per_lane = (n_in / 32 + LPR - 1) / LPR;
    if (per_lane <= 1) return gemv_launch<T, NT, LPR, 1>(GEMV_ARGS);
    if (per_lane <= 2) return gemv_launch<T, NT, LPR, 2>(GEMV_ARGS);
    if (per_lane <= 4) return gemv_launch<T, NT, LPR, 4>(GEMV_ARGS);
    if (per_lane <= 8) return gemv_launch<T, NT, LPR, 8>(GEMV_ARGS);
    return gemv_launch<T, NT, LPR, 16>(GEMV_ARGS);
}

template <uint32_t T, int NT>
hipError_t gemv_pick_lpr(GEMV_PARAMS) {
    const int groups = n_in / 32;
    if (groups >= 64) return gemv_pick_maxc<T, NT, 64>(GEMV_ARGS);
    if (groups >= 32) return gemv_pick_maxc<T, NT, 32>(GEMV_ARGS);
    if (groups >= 16) return gemv_pick_maxc<T, NT, 16>(GEMV_ARGS);
    return gemv_pick_maxc<T, NT, 8>(GEMV_ARGS);
}

// nt: tokens per block (the batch size for plain launches, the item size for
// expert work lists)
template <uint32_t T>
hipError_t gemv_pick_nt(int nt, GEMV_PARAMS) {
    if (nt <= 1) return gemv_pick_lpr<T, 1>(GEMV_ARGS);
    if (nt <= 2) return gemv_pick_lpr<T, 2>(GEMV_ARGS);
    if (nt <= 4) return gemv_pick_lpr<T, 4>(GEMV_ARGS);
    if (nt <= 8) return gemv_pick_lpr<T, 8>(GEMV_ARGS);
    return gemv_pick_lpr<T, 16>(GEMV_ARGS);
}

}  // namespace

hipError_t launch_gemv(const void* w, const WeightLayout& WL, const void* act, int act_rows, int n_tok, float* y,
                       int ldy, hipStream_t s, const TokenMap* group, int item_tokens, int max_items) {
    const ActLayout AL = act_layout(act_rows, WL.n_in);
    if (!WL.total || !AL.total || n_tok <= 0) return hipErrorInvalidValue;
    if (is_kquant(WL.type) && !AL.has256) return hipErrorInvalidValue;
    const WeightPtrs W = weight_ptrs(w, WL);
    const ActPtrs A = act_ptrs(act, AL);
    TokenMap map{};
    int nt = n_tok, yb = 0;
    int n_out = WL.n_out;
    if (group) {
        map = *group;
        nt = item_tokens;
        yb = max_items;
        n_out = map.rows_per_expert;
    }
    switch (WL.type) {
        case kQ8_0: return gemv_pick_nt<kQ8_0>(nt, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        case kQ4_0: return gemv_pick_nt<kQ4_0>(nt, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        case kQ4_K: return gemv_pick_nt<kQ4_K>(nt, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        case kQ6_K: return gemv_pick_nt<kQ6_K>(nt, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
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
