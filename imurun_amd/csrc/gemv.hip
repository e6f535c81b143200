// Decode-shape matmul (few tokens) over the repacked weights, judged as a
// memory-bound kernel: every weight byte is read once with 128-bit loads.
//
// y[t][i] = dot(W_i, x_t) for t < n_tok (matmul_batch, ops.cpp:177-216).
// A group of LPR lanes owns one output row; lane `sub` of the group takes the
// row's 32-element groups sub, sub+LPR, ... so one load instruction of the
// wavefront covers LPR consecutive 16-byte chunks of a row. The lane computes
// each group's exact integer dot (dots.h) and scales it in f32; the LPR
// partial sums are reduced with cross-lane shuffles at the end. A wavefront
// reads its rows once, with every load issued before the first use.
//
// Also here: the per-block integer dump used by the parity tests, built from
// the same dots.h functions.
#include <algorithm>

#include "common.h"
#include "dots.h"
#include "kernels.h"
#include "qact.h"
#include "rowdot.h"

namespace fishhip {

namespace {

// One-shot wavefront scheme: LPR lanes per row; a wavefront owns RB passes of
// RPP = 64/LPR interleaved rows and reads each of them exactly once. Lane
// `sub` covers groups sub, sub + LPR, ... (MAXC of them). Every load of the
// wavefront is unconditional -- out-of-range rows and groups read a clamped,
// valid address and their contribution is zeroed with a select -- so all of
// its weight (and, for one token, activation) loads are in flight together
// instead of being serialised by per-load branches. For one token the lane's
// activation groups are loaded once into registers; for more tokens they are
// read per token through the caches. blockIdx.y selects up to NT tokens:
// consecutive rows of the batch, or one item of an expert work list (TokenMap).
template <uint32_t T, int NT, int LPR, int MAXC, int RB>
__global__ __launch_bounds__(256) void gemv_kernel(WeightPtrs W, ActPtrs A, int n_in, int n_out, int n_tok,
                                                   TokenMap map, float* __restrict__ y, int ldy) {
    constexpr int RPP = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int sub = lane % LPR;
    const int wave_id = int(blockIdx.x) * 4 + int(threadIdx.x >> 6);
    const int row_base = wave_id * (RPP * RB) + lane / LPR;
    if (wave_id * (RPP * RB) >= n_out) return;  // uniform over the wavefront
    const int groups = n_in / 32;

    int s0, cnt;
    int wrow0 = 0;  // first weight row of the expert
    if (map.items) {
        const int it = int(blockIdx.y);
        if (it >= *map.n_items) return;
        wrow0 = map.items[3 * it] * n_out;
        s0 = map.items[3 * it + 1];
        cnt = map.items[3 * it + 2];
    } else {
        s0 = int(blockIdx.y) * NT;
        cnt = min(NT, n_tok - s0);
    }
    int arow[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) arow[t] = map.act_row ? map.act_row[s0 + min(t, cnt - 1)] : s0 + min(t, cnt - 1);

    int cg[MAXC];    // clamped group index
    bool cv[MAXC];   // group exists
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
        const int c = sub + k * LPR;
        cv[k] = c < groups;
        cg[k] = cv[k] ? c : groups - 1;
    }

    Frag f[RB][MAXC];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int row = wrow0 + min(row_base + rb * RPP, n_out - 1);
#pragma unroll
        for (int k = 0; k < MAXC; ++k) f[rb][k] = load_group_raw<T, true>(W, row, cg[k], n_in, lane);
    }
    __builtin_amdgcn_sched_barrier(0);

    float acc[RB][NT];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[rb][t] = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        ActFrag ac[MAXC];
#pragma unroll
        for (int k = 0; k < MAXC; ++k) ac[k] = load_act<T>(A, arow[t], cg[k], n_in);
        if (t == 0) {
            // the first token's activation loads are in flight: decode the weight scales
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int k = 0; k < MAXC; ++k) finish_group<T, true>(f[rb][k], cg[k], lane);
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int k = 0; k < MAXC; ++k) {
                const float v = group_dot<T>(f[rb][k], ac[k]);
                acc[rb][t] += cv[k] ? v : 0.0f;
            }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int row = row_base + rb * RPP;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float v = acc[rb][t];
#pragma unroll
            for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
            if (sub == 0 && row < n_out && t < cnt) y[size_t(s0 + t) * ldy + row] = v;
        }
    }
}

// Per-block integers for token 0 of A: Q8_0/Q4_0 one per 32-block; Q4_K / Q5_K
// two per super-block (sum_g sc_g dot_g, sum_g m_g bsum_g); Q6_K one per super-block.
template <uint32_t T>
__global__ void block_ints_kernel(WeightPtrs W, ActPtrs A, int n_in, int n_out, int32_t* __restrict__ out) {
    const long gid = long(blockIdx.x) * blockDim.x + threadIdx.x;
    constexpr bool kq = kquant_type(T);
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
            if constexpr (has_mins(T)) {
                sumi += f.sca * (T == kQ4_K ? dot_q4_k(f.w0, a.a0, a.a1) : dot_q5_k(f.w0, f.hb, a.a0, a.a1));
                mins += f.scb * (a.s + a.s2);
            } else {
                sumi += isum_q6_k(f.w0, f.qh, a.a0, a.a1, a.s, a.s2, f.sca, f.scb);
            }
        }
        if constexpr (has_mins(T)) {
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
    constexpr int RB = gemv_rb<T, MAXC>();
    constexpr int RPW = (64 / LPR) * RB;
    const int waves = (n_out + RPW - 1) / RPW;
    const unsigned gy = map.items ? unsigned(y_blocks) : unsigned((n_tok + NT - 1) / NT);
    const dim3 grid(unsigned((waves + 3) / 4), gy);
    hipLaunchKernelGGL((gemv_kernel<T, NT, LPR, MAXC, RB>), grid, dim3(256), 0, s, W, A, n_in, n_out, n_tok, map, y,
                       ldy);
    return hipGetLastError();
}

#define GEMV_ARGS W, A, n_in, n_out, n_tok, map, y_blocks, y, ldy, s
#define GEMV_PARAMS                                                                                                \
    const WeightPtrs &W, const ActPtrs &A, int n_in, int n_out, int n_tok, const TokenMap &map, int y_blocks, \
        float *y, int ldy, hipStream_t s

// groups per lane, rounded up to an instantiated count (extra groups are masked)
template <uint32_t T, int NT, int LPR>
hipError_t gemv_pick_maxc(GEMV_PARAMS) {
    const int per_lane = (n_in / 32 + LPR - 1) / LPR;
    switch (per_lane) {
        case 1: return gemv_launch<T, NT, LPR, 1>(GEMV_ARGS);
        case 2: return gemv_launch<T, NT, LPR, 2>(GEMV_ARGS);
        case 3: return gemv_launch<T, NT, LPR, 3>(GEMV_ARGS);
        case 4: return gemv_launch<T, NT, LPR, 4>(GEMV_ARGS);
        default: break;
    }
    if constexpr (LPR == 64) {
        if (per_lane <= 6) return gemv_launch<T, NT, LPR, 6>(GEMV_ARGS);
        if (per_lane <= 8) return gemv_launch<T, NT, LPR, 8>(GEMV_ARGS);
        if (per_lane <= 12) return gemv_launch<T, NT, LPR, 12>(GEMV_ARGS);
        if (per_lane <= 16) return gemv_launch<T, NT, LPR, 16>(GEMV_ARGS);
    }
    return hipErrorInvalidValue;
}

// lanes per row: all 64 for rows of >= 64 groups, else 16 or 8
template <uint32_t T, int NT>
hipError_t gemv_pick_lpr(GEMV_PARAMS) {
    const int groups = n_in / 32;
    if (groups >= 64) return gemv_pick_maxc<T, NT, 64>(GEMV_ARGS);
    if (groups >= 16) return gemv_pick_maxc<T, NT, 16>(GEMV_ARGS);
    return gemv_pick_maxc<T, NT, 8>(GEMV_ARGS);
}

// nt: tokens per block (the batch size for plain launches, the item size for
// expert work lists); larger batches take blocks of four tokens
template <uint32_t T>
hipError_t gemv_pick_nt(int nt, GEMV_PARAMS) {
    if (nt <= 1) return gemv_pick_lpr<T, 1>(GEMV_ARGS);
    if (nt <= 2) return gemv_pick_lpr<T, 2>(GEMV_ARGS);
    return gemv_pick_lpr<T, 4>(GEMV_ARGS);
}

// ---------------------------------------------------------------- one token, f32 input

// matmul_batch's convenience form (ops.cpp:254-264) for one token: every
// workgroup (kGemvXWaves wavefronts) quantizes x itself into LDS -- with the
// quantize kernel's exact arithmetic, so the int8 codes, scales and sums are
// the same bytes -- and then runs the one-shot GEMV above on them. The x loads go out first, then
// the workgroup's weight loads, so the quantization waits only for x (from
// L2) while the weights stream in; no separate quantize launch. Up to
// kGemmGroupMax tensors on the same x share the grid (gate and up).
constexpr int kGemvXWaves = 16;

struct GemvXGroup {
    WeightPtrs w[kGemmGroupMax];
    float* y[kGemmGroupMax];
    uint32_t type[kGemmGroupMax];
    int n_out[kGemmGroupMax];
    int wg_end[kGemmGroupMax];  // cumulative workgroups
    int n;
    RowNorm norm;               // norm.w == nullptr: x as given
    RowResid resid;             // resid.x == nullptr: y only
    int pair_act;               // kActNone, or gate / up pairs: y[0] = act(gate) * up
};

// The RowNorm prologue on the workgroup's x chunks (thread tid holds values
// 4 (tid + TH i) ..): the double sum of x^2 over the row (rmsnorm,
// ops.cpp:18-23: products and sums in double, then one float scale), then
// x * scale * w in place; workgroup 0 writes the result.
template <int XV, int TH>
__device__ __forceinline__ void row_norm(float4 (&xv)[XV], const RowNorm& nm, int n_in, int tid, double* red) {
    const int lane = tid & 63, wave = tid >> 6;
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < XV; ++i) {
        if (4 * (tid + TH * i) < n_in) {
            s = __dadd_rn(s, __dmul_rn(double(xv[i].x), double(xv[i].x)));
            s = __dadd_rn(s, __dmul_rn(double(xv[i].y), double(xv[i].y)));
            s = __dadd_rn(s, __dmul_rn(double(xv[i].z), double(xv[i].z)));
            s = __dadd_rn(s, __dmul_rn(double(xv[i].w), double(xv[i].w)));
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s = __dadd_rn(s, __shfl_xor(s, off));
    if (lane == 0) red[wave] = s;
    __syncthreads();
    double sum = 0.0;
    for (int w = 0; w < TH / 64; ++w) sum = __dadd_rn(sum, red[w]);
    const float scale = 1.0f / sqrtf(float(sum / n_in) + nm.eps);
#pragma unroll
    for (int i = 0; i < XV; ++i) {
        const int k0 = 4 * (tid + TH * i);
        const float4 v = xv[i], wv = *reinterpret_cast<const float4*>(nm.w + min(k0, n_in - 4));
        xv[i] = make_float4(v.x * scale * wv.x, v.y * scale * wv.y, v.z * scale * wv.z, v.w * scale * wv.w);
        if (blockIdx.x == 0 && k0 < n_in && nm.xn_out) *reinterpret_cast<float4*>(nm.xn_out + k0) = xv[i];
    }
}

// The rows of group member gm for wavefront wave_id of that member, on x held
// as the float4 chunks xv (loaded by the caller before anything else).
// PAIR: the workgroup's first half of wavefronts holds gate rows (member 0),
// the second half the same rows of up (member 1); up's results reach the gate
// wavefronts through s_pair, which write act(gate) * up, and up is stored.
// Rows per wavefront of the one-token kernels: gemv_rb, or gemv_rb / RBD (at least
// one) for a launch whose grid would leave CUs without a workgroup.
template <uint32_t T, int MAXC, int RBD>
constexpr int gemv_x_rb() {
    return gemv_rb<T, MAXC>() / RBD < 1 ? 1 : gemv_rb<T, MAXC>() / RBD;
}
constexpr int kGemvCUs = 256;  // MI355X compute units

template <uint32_t T, int LPR, int MAXC, int XV, bool NORM, bool PAIR = false, int RBD = 1>
__device__ __forceinline__ void gemv_x_rows(const GemvXGroup& G, int gm, int wave_id, float4 (&xv)[XV], int n_in,
                                            uint4* s_codes, float* s_d, int* s_s, double* s_red,
                                            float* s_pair = nullptr) {
    constexpr bool kq = kquant_type(T);
    constexpr int RPP = 64 / LPR;
    constexpr int RB = gemv_x_rb<T, MAXC, RBD>();
    const int tid = threadIdx.x, lane = tid & 63, sub = lane % LPR;
    const WeightPtrs W = G.w[gm];
    const int n_out = G.n_out[gm];
    const int row_base = wave_id * (RPP * RB) + lane / LPR;
    const int groups = n_in / 32;

    // every weight load of the wavefront (clamped, unconditional)
    int cg[MAXC];
    bool cv[MAXC];
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
        const int c = sub + k * LPR;
        cv[k] = c < groups;
        cg[k] = cv[k] ? c : groups - 1;
    }
    // Q8_0 / Q4_0 rows of up to 128 groups: non-temporal code loads (5 % faster on
    // the Q4_0 2 x 14336x4096 gate+up, 3 % on the Q8_0 4096x4096; slower on
    // longer rows and on the K-quants)
    constexpr bool NT = (T == kQ4_0 || T == kQ8_0) && MAXC <= 2;
    // K-quants: the scale data of every group first, then every group's codes, so
    // that decoding the scales (the meta shuffles and 6-bit unpacking) waits only
    // for them and runs before the barrier, under the other wavefronts'
    // quantization (Q4_K down 4096x14336: 10.5 -> 10.1 us). Q8_0 / Q4_0 (one f16 scale
    // a group) keep each group's loads together and decode after the barrier (the split
    // made the Q8_0 4096^2 GEMV 3 % slower).
    Frag f[RB][MAXC];
    if constexpr (kq) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int row = min(row_base + rb * RPP, n_out - 1);
#pragma unroll
            for (int k = 0; k < MAXC; ++k) load_group_scales<T, true>(f[rb][k], W, row, cg[k], n_in, lane);
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int row = min(row_base + rb * RPP, n_out - 1);
#pragma unroll
            for (int k = 0; k < MAXC; ++k) load_group_codes<T, NT>(f[rb][k], W, row, cg[k], n_in);
        }
    } else {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int row = min(row_base + rb * RPP, n_out - 1);
#pragma unroll
            for (int k = 0; k < MAXC; ++k) f[rb][k] = load_group_raw<T, true, NT>(W, row, cg[k], n_in, lane);
        }
    }

    // every load is issued before the quantization's first use of x
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NORM) row_norm<XV, 64 * kGemvXWaves>(xv, G.norm, n_in, tid, s_red);
    const LdsAct L{s_codes, s_d, s_s, kGemvXMaxGroups};
    quantize_to_lds<kq, XV, 64 * kGemvXWaves>(xv, n_in, tid, L);
    if constexpr (kq) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int k = 0; k < MAXC; ++k) finish_group<T, true>(f[rb][k], cg[k], lane);
    }
    __syncthreads();
    // (a pair's wavefronts all reach its second barrier; their rows past the end are
    // clamped loads whose results are not stored)
    if (!PAIR && wave_id * (RPP * RB) >= n_out) return;  // uniform over the wavefront
    if constexpr (!kq) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int k = 0; k < MAXC; ++k) finish_group<T, true>(f[rb][k], cg[k], lane);
    }

    float acc[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = 0.0f;
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
        const ActFrag ac = lds_act<T>(L, cg[k]);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const float v = group_dot<T>(f[rb][k], ac);
            acc[rb] += cv[k] ? v : 0.0f;
        }
    }
    float* __restrict__ y = G.y[gm];
    if constexpr (PAIR) {
        const int slot = (wave_id % (kGemvXWaves / 2)) * (RPP * RB) + lane / LPR;
        float v[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            v[rb] = acc[rb];
#pragma unroll
            for (int off = LPR / 2; off > 0; off >>= 1) v[rb] += __shfl_xor(v[rb], off);
            if (gm == 1 && sub == 0) {
                s_pair[slot + rb * RPP] = v[rb];
                if (row_base + rb * RPP < n_out) y[row_base + rb * RPP] = v[rb];
            }
        }
        __syncthreads();
        if (gm == 0 && sub == 0) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
                if (row_base + rb * RPP < n_out)
                    y[row_base + rb * RPP] = act_mul(v[rb], s_pair[slot + rb * RPP], G.pair_act == kActGelu);
        }
        return;
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        float v = acc[rb];
#pragma unroll
        for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
        const int row = row_base + rb * RPP;
        if (sub == 0 && row < n_out) {
            y[row] = v;
            // the residual add, FISH's order x + (v + bias) (single-tensor launches)
            if (G.resid.x) G.resid.x[row] = G.resid.x[row] + (G.resid.bias ? v + G.resid.bias[row] : v);
        }
    }
}

// The group member of this workgroup and the workgroup's index within it.
__device__ __forceinline__ int gemv_x_member(const GemvXGroup& G, int& wg) {
    int gm = 0;
#pragma unroll
    for (int j = 1; j < kGemmGroupMax; ++j)
        if (j < G.n && int(blockIdx.x) >= G.wg_end[j - 1]) gm = j;
    wg = int(blockIdx.x) - (gm ? G.wg_end[gm - 1] : 0);
    return gm;
}

// The wavefront's index in its workgroup. SCALAR: read as a scalar (uniform over
// the wavefront), so that row indices derived from it take no vector registers:
// the gate / up pair kernel needs that to fit two workgroups per CU; the others
// measured 2 % slower with it (Q8_0 4096^2: 5.76 against 5.85 us).
template <bool SCALAR = false>
__device__ __forceinline__ int wave_index() {
    if constexpr (SCALAR) return __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    return int(threadIdx.x >> 6);
}

// x loads first: unconditional, from a clamped address (chunks past the end lie in
// whole 32/256-value blocks the quantizer discards, and a load inside a branch would
// make the compiler wait for every outstanding load at the join)
template <int XV>
__device__ __forceinline__ void gemv_x_loads(const float* __restrict__ x, int n_in, float4 (&xv)[XV]) {
#pragma unroll
    for (int i = 0; i < XV; ++i) {
        const int k0 = 4 * (int(threadIdx.x) + 64 * kGemvXWaves * i);
        xv[i] = *reinterpret_cast<const float4*>(x + min(k0, n_in - 4));
    }
}

template <uint32_t T, int LPR, int MAXC, int XV, bool NORM, int RBD>
__global__ __launch_bounds__(64 * kGemvXWaves) void gemv_x_kernel(GemvXGroup G, const float* __restrict__ x,
                                                                  int n_in) {
    __shared__ uint4 s_codes[2 * kGemvXMaxGroups];  // [half][group]: elements 16 h .. 16 h + 15
    __shared__ float s_d[kGemvXMaxGroups];           // Q8Act d per group / Q8ActK d per super-block
    __shared__ int s_s[kGemvXMaxGroups];             // Q8Act sum per group / the group's two per-16 sums
    __shared__ double s_red[kGemvXWaves];
    int wg;
    const int gm = gemv_x_member(G, wg);
    float4 xv[XV];
    gemv_x_loads<XV>(x, n_in, xv);
    gemv_x_rows<T, LPR, MAXC, XV, NORM, false, RBD>(G, gm, wg * kGemvXWaves + wave_index(), xv, n_in, s_codes,
                                                    s_d, s_s, s_red);
}

// A layer's gate and up (one type and shape) with the FFN activation in the
// epilogue: workgroup wg computes rows wg * 8 RB .. of both, and writes
// y[0] = act(gate) * up (FISH's silu / gelu, then the product) and y[1] = up,
// so no separate activation launch runs (model.cpp:1504-1508).
// (Q4_0 / Q8_0 / Q4_K rows of up to two groups per lane: registers for two
// workgroups per CU, as the launch without the epilogue has; the others would spill)
template <uint32_t T, int LPR, int MAXC, int XV>
__global__ __launch_bounds__(64 * kGemvXWaves) __attribute__((
    amdgpu_waves_per_eu(MAXC <= 2 && T != kQ5_K && T != kQ6_K ? 8 : 1))) void gemv_xp_kernel(GemvXGroup G,
                                                                                           const float* __restrict__ x,
                                                                                           int n_in) {
    constexpr int HALF = kGemvXWaves / 2;
    __shared__ uint4 s_codes[2 * kGemvXMaxGroups];
    __shared__ float s_d[kGemvXMaxGroups];
    __shared__ int s_s[kGemvXMaxGroups];
    __shared__ double s_red[kGemvXWaves];
    __shared__ float s_pair[HALF * (64 / LPR) * gemv_rb<T, MAXC>()];
    const int wave = wave_index<true>();
    float4 xv[XV];
    gemv_x_loads<XV>(x, n_in, xv);
    gemv_x_rows<T, LPR, MAXC, XV, true, true>(G, wave / HALF, int(blockIdx.x) * HALF + wave % HALF, xv, n_in,
                                              s_codes, s_d, s_s, s_red, s_pair);
}

// Two K-quant types in one launch (a layer's q / k in Q4_K and v in Q6_K): both
// read the same Q8ActK quantization of x; each workgroup takes its member's
// type's path (a branch uniform over the workgroup).
template <uint32_t T1, uint32_t T2, int LPR, int MAXC, int XV, bool NORM, int RBD>
__global__ __launch_bounds__(64 * kGemvXWaves) void gemv_x2_kernel(GemvXGroup G, const float* __restrict__ x,
                                                                   int n_in) {
    static_assert(kquant_type(T1) && kquant_type(T2), "one activation layout for both types");
    __shared__ uint4 s_codes[2 * kGemvXMaxGroups];
    __shared__ float s_d[kGemvXMaxGroups];
    __shared__ int s_s[kGemvXMaxGroups];
    __shared__ double s_red[kGemvXWaves];
    int wg;
    const int gm = gemv_x_member(G, wg);
    float4 xv[XV];
    gemv_x_loads<XV>(x, n_in, xv);
    const int wave_id = wg * kGemvXWaves + wave_index();
    if (G.type[gm] == T1)
        gemv_x_rows<T1, LPR, MAXC, XV, NORM, false, RBD>(G, gm, wave_id, xv, n_in, s_codes, s_d, s_s, s_red);
    else
        gemv_x_rows<T2, LPR, MAXC, XV, NORM, false, RBD>(G, gm, wave_id, xv, n_in, s_codes, s_d, s_s, s_red);
}

// rows per wavefront of type t at MAXC groups per lane (gemv_x_rb)
inline int gemv_rb_of(uint32_t t, int maxc, int rbd = 1) {
    const int per_group = t == kQ8_0 ? 32 : 16;
    int rb = 64 / (per_group * maxc);
    rb = rb < 1 ? 1 : (rb > 8 ? 8 : rb);
    return rb / rbd < 1 ? 1 : rb / rbd;
}

// 4-value chunks per thread: >= n_in / (4 TH) for every n_in of this (LPR, MAXC)
template <int LPR, int MAXC>
constexpr int gemv_x_xv() {
    return LPR == 64 ? (64 * 32 * MAXC / 4 + 64 * kGemvXWaves - 1) / (64 * kGemvXWaves) : 1;
}

// workgroups of each member (each type's own rows per wavefront; one quantization of x
// serves the kGemvXWaves wavefronts of a workgroup)
template <int LPR, int MAXC>
int gemv_x_grid(GemvXGroup& G, int rbd = 1) {
    int wgs = 0;
    for (int j = 0; j < G.n; ++j) {
        const int rpw = (64 / LPR) * gemv_rb_of(G.type[j], MAXC, rbd);
        wgs += ((G.n_out[j] + rpw - 1) / rpw + kGemvXWaves - 1) / kGemvXWaves;
        G.wg_end[j] = wgs;
    }
    return wgs;
}

template <uint32_t T, int LPR, int MAXC>
hipError_t gemv_x_launch(GemvXGroup G, const float* x, int n_in, hipStream_t s) {
    static_assert(gemv_rb<T, MAXC>() >= 1, "rows per wavefront");
    constexpr int TH = 64 * kGemvXWaves;
    constexpr int XV = gemv_x_xv<LPR, MAXC>();
    if (G.pair_act) {
        // gate / up pairs: half the wavefronts of a workgroup per member, the same rows
        if constexpr (MAXC <= 4) {
            constexpr int RPW = (64 / LPR) * gemv_rb<T, MAXC>();
            const int wgs = (G.n_out[0] + (kGemvXWaves / 2) * RPW - 1) / ((kGemvXWaves / 2) * RPW);
            hipLaunchKernelGGL((gemv_xp_kernel<T, LPR, MAXC, XV>), dim3(unsigned(wgs)), dim3(TH), 0, s, G, x, n_in);
            return hipGetLastError();
        } else {
            return hipErrorInvalidValue;
        }
    }
    int wgs = gemv_x_grid<LPR, MAXC>(G);
    // a grid that leaves half the CUs idle (a 4096-row projection at two rows per
    // wavefront: 128 workgroups) takes half the rows per wavefront instead; measured on
    // 4096x4096: Q4_K 5.85 -> 4.76 us, Q4_0 5.13 -> 4.50, Q6_K 6.72 -> 5.78. A grid of
    // 192 (q|k|v) was 4 % slower halved, so larger grids keep the default.
    if constexpr (LPR == 64 && MAXC <= 2 && gemv_rb<T, MAXC>() >= 2) {
        if (2 * wgs <= kGemvCUs) {
            wgs = gemv_x_grid<LPR, MAXC>(G, 2);
            if (G.norm.w)
                hipLaunchKernelGGL((gemv_x_kernel<T, LPR, MAXC, XV, true, 2>), dim3(unsigned(wgs)), dim3(TH), 0, s, G,
                                   x, n_in);
            else
                hipLaunchKernelGGL((gemv_x_kernel<T, LPR, MAXC, XV, false, 2>), dim3(unsigned(wgs)), dim3(TH), 0, s,
                                   G, x, n_in);
            return hipGetLastError();
        }
    }
    if (G.norm.w) {
        // rows of up to 4 groups per lane (n_in <= 8192): the prologue spills registers beyond
        if constexpr (MAXC <= 4)
            hipLaunchKernelGGL((gemv_x_kernel<T, LPR, MAXC, XV, true, 1>), dim3(unsigned(wgs)), dim3(TH), 0, s, G, x,
                               n_in);
        else
            return hipErrorInvalidValue;
    } else
        hipLaunchKernelGGL((gemv_x_kernel<T, LPR, MAXC, XV, false, 1>), dim3(unsigned(wgs)), dim3(TH), 0, s, G, x,
                           n_in);
    return hipGetLastError();
}

template <uint32_t T1, uint32_t T2, int MAXC>
hipError_t gemv_x2_launch(GemvXGroup G, const float* x, int n_in, hipStream_t s) {
    constexpr int TH = 64 * kGemvXWaves;
    constexpr int XV = gemv_x_xv<64, MAXC>();
    int wgs = gemv_x_grid<64, MAXC>(G);
    if constexpr (MAXC <= 2) {  // both types 16 bytes per group: at least two rows per wavefront
        if (2 * wgs <= kGemvCUs) {
            wgs = gemv_x_grid<64, MAXC>(G, 2);
            if (G.norm.w)
                hipLaunchKernelGGL((gemv_x2_kernel<T1, T2, 64, MAXC, XV, true, 2>), dim3(unsigned(wgs)), dim3(TH), 0,
                                   s, G, x, n_in);
            else
                hipLaunchKernelGGL((gemv_x2_kernel<T1, T2, 64, MAXC, XV, false, 2>), dim3(unsigned(wgs)), dim3(TH), 0,
                                   s, G, x, n_in);
            return hipGetLastError();
        }
    }
    if (G.norm.w)
        hipLaunchKernelGGL((gemv_x2_kernel<T1, T2, 64, MAXC, XV, true, 1>), dim3(unsigned(wgs)), dim3(TH), 0, s, G,
                           x, n_in);
    else
        hipLaunchKernelGGL((gemv_x2_kernel<T1, T2, 64, MAXC, XV, false, 1>), dim3(unsigned(wgs)), dim3(TH), 0, s, G,
                           x, n_in);
    return hipGetLastError();
}

template <uint32_t T1, uint32_t T2>
hipError_t gemv_x2_pick(GemvXGroup G, const float* x, int n_in, hipStream_t s) {
    switch ((n_in / 32 + 63) / 64) {
        case 1: return gemv_x2_launch<T1, T2, 1>(G, x, n_in, s);
        case 2: return gemv_x2_launch<T1, T2, 2>(G, x, n_in, s);
        case 3: return gemv_x2_launch<T1, T2, 3>(G, x, n_in, s);
        case 4: return gemv_x2_launch<T1, T2, 4>(G, x, n_in, s);
        default: return hipErrorInvalidValue;
    }
}

template <uint32_t T, int LPR>
hipError_t gemv_x_pick_maxc(GemvXGroup G, const float* x, int n_in, hipStream_t s) {
    const int per_lane = (n_in / 32 + LPR - 1) / LPR;
    switch (per_lane) {
        case 1: return gemv_x_launch<T, LPR, 1>(G, x, n_in, s);
        case 2: return gemv_x_launch<T, LPR, 2>(G, x, n_in, s);
        case 3: return gemv_x_launch<T, LPR, 3>(G, x, n_in, s);
        case 4: return gemv_x_launch<T, LPR, 4>(G, x, n_in, s);
        default: break;
    }
    if constexpr (LPR == 64) {
        switch (per_lane) {
            case 5: return gemv_x_launch<T, LPR, 5>(G, x, n_in, s);
            case 6: return gemv_x_launch<T, LPR, 6>(G, x, n_in, s);
            case 7: return gemv_x_launch<T, LPR, 7>(G, x, n_in, s);
            case 8: return gemv_x_launch<T, LPR, 8>(G, x, n_in, s);
            default: break;
        }
    }
    return hipErrorInvalidValue;
}

template <uint32_t T>
hipError_t gemv_x_pick(GemvXGroup G, const float* x, int n_in, hipStream_t s) {
    const int groups = n_in / 32;
    if (groups >= 64) return gemv_x_pick_maxc<T, 64>(G, x, n_in, s);
    if (groups >= 16) return gemv_x_pick_maxc<T, 16>(G, x, n_in, s);
    return gemv_x_pick_maxc<T, 8>(G, x, n_in, s);
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
        if (item_tokens <= 0 || item_tokens > kGemvItemTokens) return hipErrorInvalidValue;
        map = *group;
        nt = item_tokens;
        yb = max_items;
        n_out = map.rows_per_expert;
    }
    switch (WL.type) {
        case kQ8_0: return gemv_pick_nt<kQ8_0>(nt, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        case kQ4_0: return gemv_pick_nt<kQ4_0>(nt, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        case kQ4_K: return gemv_pick_nt<kQ4_K>(nt, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        case kQ5_K: return gemv_pick_nt<kQ5_K>(nt, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
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
        case kQ5_K: hipLaunchKernelGGL(block_ints_kernel<kQ5_K>, grid, block, 0, s, W, A, WL.n_in, WL.n_out, out); break;
        case kQ6_K: hipLaunchKernelGGL(block_ints_kernel<kQ6_K>, grid, block, 0, s, W, A, WL.n_in, WL.n_out, out); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace fishhip

namespace fishhip {

bool gemv_x_supported(const WeightLayout& L) {
    return L.total && L.n_in <= 32 * kGemvXMaxGroups && (!is_kquant(L.type) || L.n_in % 256 == 0);
}

namespace {

// the two-type launches instantiated: K-quants of one layer's projections
bool gemv_x2_pair(uint32_t a, uint32_t b) {
    return (a == kQ4_K && (b == kQ5_K || b == kQ6_K)) || (a == kQ5_K && b == kQ6_K);
}

}  // namespace

bool gemv_x_mixed_supported(int n, const WeightLayout* WLs) {
    if (n < 2 || n > kGemmGroupMax) return false;
    uint32_t a = WLs[0].type, b = WLs[0].type;
    for (int j = 0; j < n; ++j) {
        if (!gemv_x_supported(WLs[j]) || WLs[j].n_in != WLs[0].n_in) return false;
        a = std::min(a, WLs[j].type);
        b = std::max(b, WLs[j].type);
    }
    for (int j = 0; j < n; ++j)
        if (WLs[j].type != a && WLs[j].type != b) return false;
    const int n_in = WLs[0].n_in;
    return a != b && gemv_x2_pair(a, b) && n_in / 32 >= 64 && (n_in / 32 + 63) / 64 <= 4;
}

bool gemv_x_pair_supported(const WeightLayout* WLs) {
    const WeightLayout &a = WLs[0], &b = WLs[1];
    return gemv_x_supported(a) && b.total && a.type == b.type && a.n_in == b.n_in && a.n_out == b.n_out &&
           (a.n_in / 32 + 63) / 64 <= 4 && a.n_in % 4 == 0;
}

hipError_t launch_gemv_x(int n, const void* const* ws, const WeightLayout* WLs, const float* x, float* const* ys,
                         hipStream_t s, const RowNorm* norm, const RowResid* resid, int pair_act) {
    if (n <= 0 || n > kGemmGroupMax || !gemv_x_supported(WLs[0])) return hipErrorInvalidValue;
    if ((norm && (!norm->w || WLs[0].n_in % 4)) || (resid && (!resid->x || n != 1 || resid->x == x)))
        return hipErrorInvalidValue;
    if (pair_act != kActNone &&
        ((pair_act != kActSilu && pair_act != kActGelu) || n != 2 || !norm || resid || !gemv_x_pair_supported(WLs)))
        return hipErrorInvalidValue;
    GemvXGroup G{};
    G.n = n;
    G.pair_act = pair_act;
    if (norm) G.norm = *norm;
    if (resid) G.resid = *resid;
    bool mixed = false;
    for (int j = 0; j < n; ++j) {
        if (!WLs[j].total || WLs[j].n_in != WLs[0].n_in) return hipErrorInvalidValue;
        mixed = mixed || WLs[j].type != WLs[0].type;
        G.w[j] = weight_ptrs(ws[j], WLs[j]);
        G.y[j] = ys[j];
        G.type[j] = WLs[j].type;
        G.n_out[j] = WLs[j].n_out;
    }
    if (mixed) {
        if (!gemv_x_mixed_supported(n, WLs)) return hipErrorInvalidValue;
        uint32_t a = WLs[0].type, b = WLs[0].type;
        for (int j = 0; j < n; ++j) {
            a = std::min(a, WLs[j].type);
            b = std::max(b, WLs[j].type);
        }
        if (a == kQ4_K && b == kQ5_K) return gemv_x2_pick<kQ4_K, kQ5_K>(G, x, WLs[0].n_in, s);
        if (a == kQ4_K && b == kQ6_K) return gemv_x2_pick<kQ4_K, kQ6_K>(G, x, WLs[0].n_in, s);
        return gemv_x2_pick<kQ5_K, kQ6_K>(G, x, WLs[0].n_in, s);
    }
    switch (WLs[0].type) {
        case kQ8_0: return gemv_x_pick<kQ8_0>(G, x, WLs[0].n_in, s);
        case kQ4_0: return gemv_x_pick<kQ4_0>(G, x, WLs[0].n_in, s);
        case kQ4_K: return gemv_x_pick<kQ4_K>(G, x, WLs[0].n_in, s);
        case kQ5_K: return gemv_x_pick<kQ5_K>(G, x, WLs[0].n_in, s);
        case kQ6_K: return gemv_x_pick<kQ6_K>(G, x, WLs[0].n_in, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace fishhip
