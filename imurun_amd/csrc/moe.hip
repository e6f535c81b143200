// Expert-routed FFN (Mixtral / Qwen3-MoE style) on the device.
//
// FISH's moe_ffn (model.cpp:1523-1580) runs, per layer: router logits ->
// softmax over all experts (ops.cpp:40-55) -> the k most probable, descending
// -> renormalise by their sum (expert_weights_norm, model.cpp:461-462) ->
// for each expert in ascending order, its tokens in ascending order as one
// batch: gate, up, silu(gate) * up, requantise, down -> out[t] += w * down.
// Here the same work is one routing kernel, one quantization of x, one
// grouped launch each for gate, up and down over a device work list of
// (expert, slot range) items, a fused silu*up requantization, and a combine
// kernel that adds the experts of each token in ascending expert order with
// FISH's separate multiply and add.
#include "common.h"
#include "kernels.h"
#include "qact.h"
#include "rowdot.h"

namespace fishhip {

namespace {

constexpr int kMaxExperts = 256;
constexpr int kMaxK = 16;
constexpr int kMaxTok = 2048;  // grouping bitmap: kMaxExperts x kMaxTok bits in LDS
constexpr int kMoe1UpWaves = 16;      // wavefronts per workgroup: one-token gate+up
constexpr int kMoe1DownWaves = 16;    // and down: KMAX expert slots x 16 / KMAX row groups
constexpr int kMoe1MaxGroups = 1024;  // k * n_ff <= 32768 hidden values in LDS

// One token's routing by one wavefront (model.cpp:1528-1547): softmax over
// the experts in FISH's order (max, then exp(x - max) summed left to right,
// then times 1/sum), the k most probable by k wavefront argmax rounds (ties:
// lower expert), renormalised by their sum when norm. The results land in
// LDS: e_out[j] / w_out[j], j < k, in descending probability, readable by
// every lane of the wavefront on return. s_p: LDS scratch of kMaxExperts
// floats owned by this wavefront, 16-byte aligned.
//
// The logits come in registers (load_logits: lane l holds experts l + 64 q),
// fetched in one batch at kernel entry. Fetching them inside the routing, one
// load and wait per loop, put several dependent round trips -- each queued
// behind the other workgroups' weight traffic -- in front of every
// workgroup's weight loads (measured: 9 us of the 15.7 us Qwen3 gate+up).
constexpr int kLgPerLane = kMaxExperts / 64;

__device__ __forceinline__ void load_logits(const float* __restrict__ lg, int n_expert, int lane,
                                            float (&v)[kLgPerLane]) {
    // unconditional loads from clamped addresses: no branch, so no wait for other loads at a join
#pragma unroll
    for (int q = 0; q < kLgPerLane; ++q) v[q] = lg[min(lane + 64 * q, n_expert - 1)];
}

__device__ void route_token(const float (&v)[kLgPerLane], int n_expert, int k, int norm, float* s_p, int* e_out,
                            float* w_out, int lane) {
    // every cross-lane step is a DPP swizzle, a readlane or a ballot: no LDS round trips
    // besides the ordered sum's reads
    float lm = -INFINITY;
#pragma unroll
    for (int q = 0; q < kLgPerLane; ++q)
        if (lane + 64 * q < n_expert) lm = fmaxf(lm, v[q]);
    const float m = wave_max64(lm);
    float ex[kLgPerLane];
#pragma unroll
    for (int q = 0; q < kLgPerLane; ++q) {
        ex[q] = lane + 64 * q < n_expert ? expf(__fsub_rn(v[q], m)) : 0.0f;
        s_p[lane + 64 * q] = ex[q];  // zeros past n_expert
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    // FISH's left-to-right sum, by lane 0, eight 16-byte reads in flight at a time. The
    // zeros past n_expert (up to the next multiple of 32) leave it unchanged: the sum
    // starts at +0 and every term is >= +0.
    float sum = 0.0f;
    if (lane == 0) {
        const float4* s4 = reinterpret_cast<const float4*>(s_p);
        for (int e0 = 0; e0 < n_expert; e0 += 32) {
            float4 r[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) r[i] = s4[(e0 >> 2) + i];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                sum = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(sum, r[i].x), r[i].y), r[i].z), r[i].w);
        }
    }
    sum = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sum), 0));
    const bool uniform = !(sum > 0.0f);
    const float inv = uniform ? 0.0f : 1.0f / sum, pu = 1.0f / float(n_expert);
    float p[kLgPerLane];
#pragma unroll
    for (int q = 0; q < kLgPerLane; ++q)
        p[q] = (lane + 64 * q < n_expert) ? (uniform ? pu : __fmul_rn(ex[q], inv)) : -1.0f;
    // k rounds: the largest remaining probability, then the lowest expert holding it
    float wsum = 0.0f;
    for (int j = 0; j < k; ++j) {
        const float mb = wave_max64(fmaxf(fmaxf(p[0], p[1]), fmaxf(p[2], p[3])));
        int be = -1;
#pragma unroll
        for (int q = 0; q < kLgPerLane; ++q) {
            const unsigned long long b = __ballot(p[q] == mb);
            if (be < 0 && b) be = 64 * q + __builtin_ctzll(b);
        }
        if (lane == 0) {
            e_out[j] = be;
            w_out[j] = mb;
        }
        wsum = __fadd_rn(wsum, mb);
#pragma unroll
        for (int q = 0; q < kLgPerLane; ++q)
            if (lane + 64 * q == be) p[q] = -2.0f;  // taken
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    // renormalised by the sum of the k (model.cpp:1545-1546), one choice per lane
    if (norm && wsum > 0.0f && lane < k) w_out[lane] = w_out[lane] / wsum;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
}

// One wavefront per token.
__global__ __launch_bounds__(256) void topk_kernel(const float* __restrict__ logits, int n_tok, int n_expert, int k,
                                                   int norm, MoeRouting r) {
    __shared__ __align__(16) float s_p[4][kMaxExperts];
    __shared__ int s_e[4][kMaxK];
    __shared__ float s_w[4][kMaxK];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int t = int(blockIdx.x) * 4 + w;
    if (t >= n_tok) return;
    float lv[kLgPerLane];
    load_logits(logits + size_t(t) * n_expert, n_expert, lane, lv);
    route_token(lv, n_expert, k, norm, s_p[w], s_e[w], s_w[w], lane);
    if (lane < k) {
        r.sel[t * k + lane] = s_e[w][lane];
        r.wsel[t * k + lane] = s_w[w][lane];
    }
}

// Exclusive prefix sum of v over the 256 threads of the workgroup (LDS
// Hillis-Steele); every thread gets its own prefix and the total.
__device__ __forceinline__ int block_exclusive_scan(int v, int* s, int tid, int& total) {
    s[tid] = v;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        const int a = (tid >= off) ? s[tid - off] : 0;
        __syncthreads();
        s[tid] += a;
        __syncthreads();
    }
    const int incl = s[tid];
    total = s[255];
    __syncthreads();
    return incl - v;
}

// One workgroup: group the (token, choice) pairs by expert, tokens ascending,
// through an expert x token bitmap (rank = set bits before the token), and
// write the work list of items of at most item_tokens slots (experts
// ascending, then slot ranges ascending). One thread per expert forms its
// count, offsets and items from two workgroup prefix sums.
__global__ __launch_bounds__(256) void group_kernel(int n_tok, int n_expert, int k, int item_tokens, MoeRouting r) {
    static_assert(kMaxExperts <= 256, "one thread per expert");
    __shared__ uint32_t s_bits[kMaxExperts * (kMaxTok / 32)];
    __shared__ int s_off[kMaxExperts + 1];
    __shared__ int s_scan[256];
    const int tid = threadIdx.x;
    const int words = (n_tok + 31) / 32;
    for (int i = tid; i < n_expert * words; i += blockDim.x) s_bits[i] = 0;
    __syncthreads();
    for (int i = tid; i < n_tok * k; i += blockDim.x) {
        const int t = i / k, e = r.sel[i];
        atomicOr(&s_bits[e * words + t / 32], 1u << (t % 32));
    }
    __syncthreads();
    int c = 0;
    if (tid < n_expert)
        for (int q = 0; q < words; ++q) c += __popc(s_bits[tid * words + q]);
    const int n_it = (c + item_tokens - 1) / item_tokens;
    int total_slots = 0, total_items = 0;
    const int off = block_exclusive_scan(c, s_scan, tid, total_slots);
    const int ioff = block_exclusive_scan(n_it, s_scan, tid, total_items);
    if (tid < n_expert) {
        s_off[tid] = off;
        r.counts[tid] = c;
        r.offsets[tid] = off;
        for (int b = 0; b < n_it; ++b) {
            r.items[3 * (ioff + b)] = tid;
            r.items[3 * (ioff + b) + 1] = off + b * item_tokens;
            r.items[3 * (ioff + b) + 2] = min(item_tokens, c - b * item_tokens);
        }
    }
    if (tid == 0) {
        s_off[n_expert] = total_slots;
        r.offsets[n_expert] = total_slots;
        *r.n_items = total_items;
    }
    __syncthreads();
    for (int i = tid; i < n_tok * k; i += blockDim.x) {
        const int t = i / k, e = r.sel[i];
        const uint32_t* row = s_bits + e * words;
        int rank = __popc(row[t / 32] & ((1u << (t % 32)) - 1u));
        for (int q = 0; q < t / 32; ++q) rank += __popc(row[q]);
        const int slot = s_off[e] + rank;
        r.slot_tok[slot] = t;
        r.tok_slot[i] = slot;
    }
}

// Workgroup (token t, 1024-column chunk): the token's k choices ranked in
// ascending expert order (thread j counts the choices before its own; the
// experts of one token are distinct), then four columns per thread add the
// experts' weighted down rows (workspace rows, 16-byte aligned) in that order.
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ down, MoeRouting r, int n_tok, int k,
                                                      int n_embd, float* __restrict__ out) {
    __shared__ int s_sel[kMaxK];
    __shared__ int s_slot[kMaxK];
    __shared__ float s_w[kMaxK];
    const int t = int(blockIdx.x), tid = threadIdx.x;
    int sel = 0, slot = 0;
    float w = 0.0f;
    if (tid < k) {
        sel = r.sel[t * k + tid];
        slot = r.tok_slot[t * k + tid];
        w = r.wsel[t * k + tid];
        s_sel[tid] = sel;
    }
    __syncthreads();
    if (tid < k) {
        int rank = 0;
        for (int j = 0; j < k; ++j) rank += (s_sel[j] < sel) ? 1 : 0;
        s_slot[rank] = slot;
        s_w[rank] = w;
    }
    __syncthreads();
    const int i = (int(blockIdx.y) * 256 + tid) * 4;
    if (i >= n_embd) return;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int q = 0; q < k; ++q) {
        // w * down is rounded before the add: this file is built without
        // multiply-add contraction
        const float wq = s_w[q];
        const float4 d = *reinterpret_cast<const float4*>(down + size_t(s_slot[q]) * n_embd + i);
        acc.x = acc.x + wq * d.x;
        acc.y = acc.y + wq * d.y;
        acc.z = acc.z + wq * d.z;
        acc.w = acc.w + wq * d.w;
    }
    float* o = out + size_t(t) * n_embd + i;  // the caller's buffer: 4-byte alignment only
    o[0] = acc.x;
    o[1] = acc.y;
    o[2] = acc.z;
    o[3] = acc.w;
}

// ---------------------------------------------------------------- one token

// The expert FFN of a single token in two launches (decode). The slot order
// is the workspace's: the k chosen experts ascending (model.cpp:1551-1561).
//
// Launch 1, gate and up: every workgroup quantizes x into LDS while the
// router logits are in flight, routes the token itself (wavefront 0,
// route_token), then for rows i of its slot's expert e computes gate_e[i], up_e[i]
// (the same lanes, so h = silu(gate) * up is formed in place) and writes
// gate, up and h. Workgroup 0 also writes the routing (sel, wsel, tok_slot,
// slot_tok).
template <uint32_t T, int LPR, int MAXC, int RB, int XV>
__global__ __launch_bounds__(64 * kMoe1UpWaves) void moe1_gate_up_kernel(
    const float* __restrict__ x, const float* __restrict__ logits, int n_embd, int n_ff, int n_expert, int k,
    int norm, WeightPtrs Wg, WeightPtrs Wu, int wgs_per_slot, MoeRouting r, float* __restrict__ g_out,
    float* __restrict__ u_out, float* __restrict__ h_out) {
    constexpr bool kq = kquant_type(T);
    constexpr int RPP = 64 / LPR, TH = 64 * kMoe1UpWaves;
    __shared__ uint4 s_codes[2 * kGemvXMaxGroups];
    __shared__ float s_d[kGemvXMaxGroups];
    __shared__ int s_s[kGemvXMaxGroups];
    __shared__ __align__(16) float s_p[kMaxExperts];
    __shared__ int s_exp[kMaxK];
    __shared__ int s_sel[kMaxK];
    __shared__ float s_wsel[kMaxK];

    const int tid = threadIdx.x, lane = tid & 63, sub = lane % LPR;
    // the router logits first: the routing (wavefront 0) gates every weight load
    float lv[kLgPerLane];
    load_logits(logits, n_expert, lane, lv);
    float4 xv[XV];
#pragma unroll
    for (int i = 0; i < XV; ++i) {
        const int k0 = 4 * (tid + TH * i);
        // unconditional load from a clamped address: chunks past the end lie in whole
        // 32/256-value blocks the quantizer discards, and a load inside a branch would
        // make the compiler wait for every outstanding load at the join
        xv[i] = *reinterpret_cast<const float4*>(x + min(k0, n_embd - 4));
    }
    // x into LDS while the logits are in flight: the routing, not the quantization,
    // then stands between the kernel's start and its weight loads
    const LdsAct L{s_codes, s_d, s_s, kGemvXMaxGroups};
    quantize_to_lds<kq, XV, TH>(xv, n_embd, tid, L);
    if (tid < 64) {
        route_token(lv, n_expert, k, norm, s_p, s_sel, s_wsel, lane);
        if (lane < k) {
            const int me = s_sel[lane];
            const float mw = s_wsel[lane];
            int rank = 0;
            for (int j = 0; j < k; ++j) rank += s_sel[j] < me;
            s_exp[rank] = me;
            if (blockIdx.x == 0) {
                r.sel[lane] = me;
                r.wsel[lane] = mw;
                r.tok_slot[lane] = rank;
                r.slot_tok[rank] = 0;
            }
        }
    }
    __syncthreads();
    const int slot = int(blockIdx.x) / wgs_per_slot, wg = int(blockIdx.x) % wgs_per_slot;
    const int e = s_exp[slot];
    const int wave_id = wg * kMoe1UpWaves + (tid >> 6);
    const int row_base = wave_id * (RPP * RB) + lane / LPR;
    const int groups = n_embd / 32;
    int cg[MAXC];
    bool cv[MAXC];
#pragma unroll
    for (int q = 0; q < MAXC; ++q) {
        const int c = sub + q * LPR;
        cv[q] = c < groups;
        cg[q] = cv[q] ? c : groups - 1;
    }
    Frag fg[RB][MAXC], fu[RB][MAXC];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int row = e * n_ff + min(row_base + rb * RPP, n_ff - 1);
#pragma unroll
        for (int q = 0; q < MAXC; ++q) {
            fg[rb][q] = load_group_raw<T, true>(Wg, row, cg[q], n_embd, lane);
            fu[rb][q] = load_group_raw<T, true>(Wu, row, cg[q], n_embd, lane);
        }
    }
    // every load is issued before the first wait
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int q = 0; q < MAXC; ++q) {
            finish_group<T, true>(fg[rb][q], cg[q], lane);
            finish_group<T, true>(fu[rb][q], cg[q], lane);
        }
    if (wave_id * (RPP * RB) >= n_ff) return;  // uniform over the wavefront
    float ag[RB], au[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) ag[rb] = au[rb] = 0.0f;
#pragma unroll
    for (int q = 0; q < MAXC; ++q) {
        const ActFrag ac = lds_act<T>(L, cg[q]);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const float vg = group_dot<T>(fg[rb][q], ac), vu = group_dot<T>(fu[rb][q], ac);
            ag[rb] += cv[q] ? vg : 0.0f;
            au[rb] += cv[q] ? vu : 0.0f;
        }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        float g = ag[rb], u = au[rb];
#pragma unroll
        for (int off = LPR / 2; off > 0; off >>= 1) {
            g += __shfl_xor(g, off);
            u += __shfl_xor(u, off);
        }
        const int row = row_base + rb * RPP;
        if (sub == 0 && row < n_ff) {
            const size_t o = size_t(slot) * n_ff + row;
            g_out[o] = g;
            u_out[o] = u;
            h_out[o] = silu_mul(g, u);
        }
    }
}

// Launch 2, down and combine: every workgroup quantizes the k hidden rows
// (each row on its own, as ActBatch::quantize does per expert batch) into
// LDS; its 16 wavefronts are KMAX slots x (16 / KMAX) row groups, so each
// wavefront reads one expert's rows. down_e[i] is written per slot, and
// out[i] = sum of w_e * down_e[i] is formed from LDS in ascending slot
// (= expert) order with FISH's separate multiply and add
// (model.cpp:1574-1579).
// XV > 0: the workgroup quantizes the k * n_ff <= 4 * 64 * kMoe1DownWaves * XV
// hidden values itself (small experts); XV == 0: they were quantized by the
// quantize kernel into `act` (one row per slot) and the workgroup copies
// them into the same LDS layout.
template <uint32_t T, int LPR, int MAXC, int KMAX, int XV>
__global__ __launch_bounds__(64 * kMoe1DownWaves) void moe1_down_kernel(const float* __restrict__ h, ActPtrs act,
                                                                        int n_embd, int n_ff, int k, WeightPtrs Wd,
                                                                        MoeRouting r, float* __restrict__ dn,
                                                                        float* __restrict__ out) {
    constexpr bool kq = kquant_type(T);
    constexpr int RPP = 64 / LPR, TH = 64 * kMoe1DownWaves;
    constexpr int R = kMoe1DownWaves / KMAX, ROWS = R * RPP;         // row groups, rows per workgroup
    constexpr int MG = XV > 0 ? XV * TH * 4 / 32 : kMoe1MaxGroups;  // LDS groups
    __shared__ uint4 s_codes[2 * MG];
    __shared__ float s_d[MG];
    __shared__ int s_s[MG];
    __shared__ int s_exp[kMaxK];
    __shared__ float s_w[kMaxK];
    __shared__ float s_dn[KMAX][ROWS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, sub = lane % LPR;
    const int slot = wave / R, rw = wave % R;
    const int n_h = k * n_ff;
    float4 xv[XV > 0 ? XV : 1];
#pragma unroll
    for (int i = 0; i < XV; ++i) {
        // unconditional load from a clamped address (chunks past the end lie in blocks the
        // quantizer discards): no load in a branch, so no wait for all outstanding loads
        const int k0 = 4 * (tid + TH * i);
        xv[i] = *reinterpret_cast<const float4*>(h + min(k0, n_h - 4));
    }
    if (tid < k) {
        const int sl = r.tok_slot[tid];
        s_exp[sl] = r.sel[tid];
        s_w[sl] = r.wsel[tid];
    }
    __syncthreads();
    const int lrow = rw * RPP + lane / LPR;  // row within the workgroup
    const int row = int(blockIdx.x) * ROWS + lrow;
    const int rowc = min(row, n_embd - 1);
    const int sc = min(slot, k - 1);  // wavefronts of slots past k read the last slot's rows, unused
    const int e = s_exp[sc];
    const int groups = n_ff / 32;
    int cg[MAXC];
    bool cv[MAXC];
#pragma unroll
    for (int q = 0; q < MAXC; ++q) {
        const int c = sub + q * LPR;
        cv[q] = c < groups;
        cg[q] = cv[q] ? c : groups - 1;
    }
    Frag f[MAXC];
#pragma unroll
    for (int q = 0; q < MAXC; ++q) f[q] = load_group_raw<T, true>(Wd, e * n_embd + rowc, cg[q], n_ff, lane);
    __builtin_amdgcn_sched_barrier(0);
    // weight scales decoded before h is quantized or staged (faster than after, as in launch 1)
#pragma unroll
    for (int q = 0; q < MAXC; ++q) finish_group<T, true>(f[q], cg[q], lane);
    const LdsAct L{s_codes, s_d, s_s, MG};
    if constexpr (XV > 0) {
        quantize_to_lds<kq, XV, TH>(xv, n_h, tid, L);
    } else {
        const int ng = n_h / 32;  // groups of all k rows (rows are contiguous in act)
        const int8_t* q = kq ? act.q256 : act.q32;
#pragma unroll 4
        for (int i = tid; i < 2 * ng; i += TH) {
            const int hh = i / ng, g = i - hh * ng;
            s_codes[hh * MG + g] = *reinterpret_cast<const uint4*>(q + size_t(g) * 32 + hh * 16);
        }
#pragma unroll 2
        for (int i = tid; i < ng; i += TH) {
            if constexpr (kq) {
                s_s[i] = *reinterpret_cast<const int*>(act.s16 + 2 * i);
                if (i < n_h / 256) s_d[i] = act.d256[i];
            } else {
                s_s[i] = act.s32[i];
                s_d[i] = act.d32[i];
            }
        }
    }
    __syncthreads();
    float d = 0.0f;
#pragma unroll
    for (int q = 0; q < MAXC; ++q) {
        const float v = group_dot<T>(f[q], lds_act<T>(L, sc * groups + cg[q]));
        d += cv[q] ? v : 0.0f;
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) d += __shfl_xor(d, off);
    if (sub == 0) {
        s_dn[slot][lrow] = d;
        if (slot < k && row < n_embd) dn[size_t(slot) * n_embd + row] = d;
    }
    __syncthreads();
    if (tid < ROWS) {
        const int orow = int(blockIdx.x) * ROWS + tid;
        float acc = 0.0f;
        for (int j = 0; j < k; ++j) {
            // w * down rounded, then added: this file is built without contraction
            const float p = s_w[j] * s_dn[j][tid];
            acc = acc + p;
        }
        if (orow < n_embd) out[orow] = acc;
    }
}

// Router logits (model.cpp:1529: matmul_batch over the f32 or f16 gate_inp
// tensor, n_expert rows of n_embd): logits[t][e] = sum_k x[t][k] * w[e][k] in
// f32. One wavefront covers TT tokens x TE experts; lane l owns k = 4l + 256j,
// fuses its products in k order into one f32 accumulator per (token, expert),
// then the 64 lanes are added by a xor butterfly. Every (t, e) therefore sums
// in the same order whatever the tile shape, so a token's logits do not
// depend on how many tokens share the launch. FISH's AVX2 f32 dot keeps 8 lane
// partials: the two agree to f32 rounding, not bit for bit.
template <bool F16>
__device__ __forceinline__ float4 router_w4(const void* w, size_t off) {
    if constexpr (F16) {
        const uint2 h = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(w) + off);
        return make_float4(f16_bits_to_f32(uint16_t(h.x & 0xFFFF)), f16_bits_to_f32(uint16_t(h.x >> 16)),
                           f16_bits_to_f32(uint16_t(h.y & 0xFFFF)), f16_bits_to_f32(uint16_t(h.y >> 16)));
    } else {
        return *reinterpret_cast<const float4*>(static_cast<const float*>(w) + off);
    }
}

template <bool F16, int TT, int TE, int U>
__device__ __forceinline__ void router_steps(const float* __restrict__ x, const void* __restrict__ w,
                                             const size_t (&xo)[TT], const size_t (&wo)[TE], int k,
                                             float (&acc)[TT][TE]) {
    float4 xv[U][TT], wv[U][TE];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int i = 0; i < TT; ++i) xv[u][i] = *reinterpret_cast<const float4*>(x + xo[i] + k + 256 * u);
#pragma unroll
        for (int j = 0; j < TE; ++j) wv[u][j] = router_w4<F16>(w, wo[j] + k + 256 * u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < TT; ++i)
#pragma unroll
            for (int j = 0; j < TE; ++j) {
                float a = acc[i][j];
                a = fmaf(xv[u][i].x, wv[u][j].x, a);
                a = fmaf(xv[u][i].y, wv[u][j].y, a);
                a = fmaf(xv[u][i].z, wv[u][j].z, a);
                acc[i][j] = fmaf(xv[u][i].w, wv[u][j].w, a);
            }
}

template <bool F16, int TT, int TE>
__global__ __launch_bounds__(256) void router_kernel(const float* __restrict__ x, const void* __restrict__ w,
                                                     int n_tok, int n_embd, int n_expert, float* __restrict__ logits) {
    // loads of U steps are issued together before their products (same sums, more loads in flight)
    constexpr int U = TT * TE == 1 ? 4 : 2;
    const int tiles_e = (n_expert + TE - 1) / TE;
    const int wave = __builtin_amdgcn_readfirstlane(int(blockIdx.x) * 4 + int(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    if (wave >= (n_tok + TT - 1) / TT * tiles_e) return;  // uniform over the wavefront
    const int t0 = wave / tiles_e * TT, e0 = wave % tiles_e * TE;
    // rows past the end repeat the last one (loaded, never stored)
    size_t xo[TT], wo[TE];
#pragma unroll
    for (int i = 0; i < TT; ++i) xo[i] = size_t(min(t0 + i, n_tok - 1)) * n_embd;
#pragma unroll
    for (int j = 0; j < TE; ++j) wo[j] = size_t(min(e0 + j, n_expert - 1)) * n_embd;
    float acc[TT][TE];
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
        for (int j = 0; j < TE; ++j) acc[i][j] = 0.0f;
    int k = 4 * lane;
    if constexpr (U > 1)
        for (; k + 256 * (U - 1) < n_embd; k += 256 * U) router_steps<F16, TT, TE, U>(x, w, xo, wo, k, acc);
    for (; k < n_embd; k += 256) router_steps<F16, TT, TE, 1>(x, w, xo, wo, k, acc);
    float mine = 0.0f;
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
        for (int j = 0; j < TE; ++j) {
            float a = acc[i][j];
            for (int off = 32; off > 0; off >>= 1) a += __shfl_xor(a, off);
            if (lane == i * TE + j) mine = a;
        }
    const int i = lane / TE, j = lane % TE;
    if (lane < TT * TE && t0 + i < n_tok && e0 + j < n_expert) logits[size_t(t0 + i) * n_expert + e0 + j] = mine;
}

template <bool F16, int TT, int TE>
void router_launch(const float* x, const void* w, int n_tok, int n_embd, int n_expert, float* logits,
                   hipStream_t stream) {
    const int waves = (n_tok + TT - 1) / TT * ((n_expert + TE - 1) / TE);
    hipLaunchKernelGGL((router_kernel<F16, TT, TE>), dim3(unsigned((waves + 3) / 4)), dim3(256), 0, stream, x, w,
                       n_tok, n_embd, n_expert, logits);
}

// The largest tile that still gives at least one wavefront per SIMD (1024);
// few-token calls keep one (token, expert) per wavefront. Measured with f32
// rows: 256 tokens x 128 experts x 2048 take 9.4 us as 2x4 tiles, 10.0 as
// 4x8 and 17.5 as 1x1; 1024 tokens take 20.4 us as 8x8, 30.1 as 2x4.
template <bool F16>
void router_pick(const float* x, const void* w, int n_tok, int n_embd, int n_expert, float* logits,
                 hipStream_t stream) {
    auto waves = [&](int tt, int te) { return long((n_tok + tt - 1) / tt) * ((n_expert + te - 1) / te); };
    if (waves(8, 8) >= 1024) router_launch<F16, 8, 8>(x, w, n_tok, n_embd, n_expert, logits, stream);
    else if (waves(2, 4) >= 1024) router_launch<F16, 2, 4>(x, w, n_tok, n_embd, n_expert, logits, stream);
    else router_launch<F16, 1, 1>(x, w, n_tok, n_embd, n_expert, logits, stream);
}

}  // namespace

hipError_t launch_moe_route(const float* logits, int n_tok, int n_expert, int k, int norm, int item_tokens,
                            const MoeRouting& r, hipStream_t stream) {
    if (n_tok <= 0 || n_tok > kMaxTok || n_expert <= 0 || n_expert > kMaxExperts || k <= 0 || k > kMaxK ||
        k > n_expert || item_tokens <= 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(topk_kernel, dim3(unsigned((n_tok + 3) / 4)), dim3(256), 0, stream, logits, n_tok, n_expert, k,
                       norm, r);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(group_kernel, dim3(1), dim3(256), 0, stream, n_tok, n_expert, k, item_tokens, r);
    return hipGetLastError();
}

hipError_t launch_router(const float* x, int n_tok, int n_embd, uint32_t type, const void* w, int n_expert,
                         float* logits, hipStream_t stream) {
    // sizes that keep k + 1024 and the wavefront count inside an int
    if (n_tok <= 0 || n_embd <= 0 || n_embd % 4 || n_embd > (1 << 30) || n_expert <= 0 ||
        long(n_tok) * n_expert > (1L << 30) || (type != kF32 && type != kF16))
        return hipErrorInvalidValue;
    if (type == kF16) router_pick<true>(x, w, n_tok, n_embd, n_expert, logits, stream);
    else router_pick<false>(x, w, n_tok, n_embd, n_expert, logits, stream);
    return hipGetLastError();
}

hipError_t launch_moe_combine(const float* down, const MoeRouting& r, int n_tok, int k, int n_embd, float* out,
                              hipStream_t stream) {
    if (n_tok <= 0 || k <= 0 || k > kMaxK || n_embd % 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(combine_kernel, dim3(unsigned(n_tok), unsigned((n_embd + 1023) / 1024)), dim3(256), 0, stream,
                       down, r, n_tok, k, n_embd, out);
    return hipGetLastError();
}

}  // namespace fishhip

namespace fishhip {

namespace {

template <uint32_t T, int LPR, int MAXC>
hipError_t moe1_gate_up_launch(const float* x, const float* logits, int n_embd, int n_ff, int n_expert, int k,
                               int norm, const WeightPtrs& Wg, const WeightPtrs& Wu, const MoeRouting& r, float* g,
                               float* u, float* h, hipStream_t s) {
    // one row (of gate and of up) per wavefront: the fewest registers and the most workgroups
    // (two rows per wavefront left one 16-wavefront workgroup per CU)
    constexpr int RB = 1;
    constexpr int RPW = (64 / LPR) * RB;
    constexpr int TH = 64 * kMoe1UpWaves;
    constexpr int XV = LPR == 64 ? (64 * 32 * MAXC / 4 + TH - 1) / TH : 1;
    const int wgs_per_slot = ((n_ff + RPW - 1) / RPW + kMoe1UpWaves - 1) / kMoe1UpWaves;
    hipLaunchKernelGGL((moe1_gate_up_kernel<T, LPR, MAXC, RB, XV>), dim3(unsigned(wgs_per_slot * k)), dim3(TH), 0, s,
                       x, logits, n_embd, n_ff, n_expert, k, norm, Wg, Wu, wgs_per_slot, r, g, u, h);
    return hipGetLastError();
}

// hidden values a workgroup quantizes itself: up to 2 chunks per thread
constexpr int kMoe1LdsXV = 2;
constexpr int kMoe1LdsHidden = 4 * 64 * kMoe1DownWaves * kMoe1LdsXV;

template <uint32_t T, int LPR, int MAXC, int KMAX>
hipError_t moe1_down_launch_k(const float* h, const ActPtrs& act, int n_embd, int n_ff, int k, const WeightPtrs& Wd,
                              const MoeRouting& r, float* dn, float* out, hipStream_t s) {
    constexpr int ROWS = (kMoe1DownWaves / KMAX) * (64 / LPR);
    const dim3 grid(unsigned((n_embd + ROWS - 1) / ROWS)), block(64 * kMoe1DownWaves);
    if (k * n_ff <= kMoe1LdsHidden)
        hipLaunchKernelGGL((moe1_down_kernel<T, LPR, MAXC, KMAX, kMoe1LdsXV>), grid, block, 0, s, h, act, n_embd, n_ff,
                           k, Wd, r, dn, out);
    else
        hipLaunchKernelGGL((moe1_down_kernel<T, LPR, MAXC, KMAX, 0>), grid, block, 0, s, h, act, n_embd, n_ff, k, Wd,
                           r, dn, out);
    return hipGetLastError();
}

template <uint32_t T, int LPR, int MAXC>
hipError_t moe1_down_launch(const float* h, const ActPtrs& act, int n_embd, int n_ff, int k, const WeightPtrs& Wd,
                            const MoeRouting& r, float* dn, float* out, hipStream_t s) {
    if (k <= 2) return moe1_down_launch_k<T, LPR, MAXC, 2>(h, act, n_embd, n_ff, k, Wd, r, dn, out, s);
    if (k <= 4) return moe1_down_launch_k<T, LPR, MAXC, 4>(h, act, n_embd, n_ff, k, Wd, r, dn, out, s);
    return moe1_down_launch_k<T, LPR, MAXC, 8>(h, act, n_embd, n_ff, k, Wd, r, dn, out, s);
}

// (LPR, groups per lane) as the GEMV picks them
template <uint32_t T, bool DOWN>
hipError_t moe1_pick(int n_in, const float* a, const ActPtrs& act, const float* logits, int n_embd, int n_ff,
                     int n_expert, int k, int norm, const WeightPtrs& W0, const WeightPtrs& W1, const MoeRouting& r,
                     float* o0, float* o1, float* o2, hipStream_t s) {
    const int groups = n_in / 32;
    const int lpr = groups >= 64 ? 64 : (groups >= 16 ? 16 : 8);
    const int per_lane = (groups + lpr - 1) / lpr;
#define MOE1_CASE(LPR_, MAXC_)                                                                                  \
    if (lpr == LPR_ && per_lane == MAXC_) {                                                                     \
        if constexpr (DOWN) return moe1_down_launch<T, LPR_, MAXC_>(a, act, n_embd, n_ff, k, W0, r, o0, o1, s); \
        else return moe1_gate_up_launch<T, LPR_, MAXC_>(a, logits, n_embd, n_ff, n_expert, k, norm, W0, W1, r, \
                                                        o0, o1, o2, s);                                      \
    }
    MOE1_CASE(64, 1) MOE1_CASE(64, 2) MOE1_CASE(64, 3) MOE1_CASE(64, 4)
    MOE1_CASE(64, 5) MOE1_CASE(64, 6) MOE1_CASE(64, 7) MOE1_CASE(64, 8)
    MOE1_CASE(16, 1) MOE1_CASE(16, 2) MOE1_CASE(16, 3) MOE1_CASE(16, 4)
    MOE1_CASE(8, 1) MOE1_CASE(8, 2)
#undef MOE1_CASE
    return hipErrorInvalidValue;
}

template <bool DOWN>
hipError_t moe1_type(uint32_t t, int n_in, const float* a, const ActPtrs& act, const float* logits, int n_embd,
                     int n_ff, int n_expert, int k, int norm, const WeightPtrs& W0, const WeightPtrs& W1,
                     const MoeRouting& r, float* o0, float* o1, float* o2, hipStream_t s) {
#define MOE1_TYPE(T_) moe1_pick<T_, DOWN>(n_in, a, act, logits, n_embd, n_ff, n_expert, k, norm, W0, W1, r, o0, o1, o2, s)
    switch (t) {
        case kQ8_0: return MOE1_TYPE(kQ8_0);
        case kQ4_0: return MOE1_TYPE(kQ4_0);
        case kQ4_K: return MOE1_TYPE(kQ4_K);
        case kQ5_K: return MOE1_TYPE(kQ5_K);
        case kQ6_K: return MOE1_TYPE(kQ6_K);
        default: return hipErrorInvalidValue;
    }
#undef MOE1_TYPE
}

}  // namespace

bool moe1_supported(uint32_t tg, uint32_t tu, int n_embd, int n_ff, int n_expert, int k) {
    const int g_in = n_embd / 32, g_ff = n_ff / 32;
    auto fits = [](int groups) {
        const int lpr = groups >= 64 ? 64 : (groups >= 16 ? 16 : 8);
        return (groups + lpr - 1) / lpr <= (lpr == 64 ? 8 : (lpr == 16 ? 4 : 2));
    };
    return tg == tu && n_embd <= 32 * kGemvXMaxGroups && k <= 8 && k * n_ff <= 32 * kMoe1MaxGroups &&
           n_expert <= kMaxExperts && fits(g_in) && fits(g_ff);
}

hipError_t launch_moe1(const float* x, const float* logits, int n_embd, int n_ff, int n_expert, int k, int norm,
                       uint32_t tg, const void* wg, uint32_t tu, const void* wu, uint32_t td, const void* wd,
                       const MoeRouting& r, float* g, float* u, float* h, void* act_h, float* dn, float* out,
                       hipStream_t s) {
    if (!moe1_supported(tg, tu, n_embd, n_ff, n_expert, k)) return hipErrorInvalidValue;
    const WeightPtrs Wg = weight_ptrs(wg, weight_layout(tg, n_embd, n_expert * n_ff));
    const WeightPtrs Wu = weight_ptrs(wu, weight_layout(tu, n_embd, n_expert * n_ff));
    const WeightPtrs Wd = weight_ptrs(wd, weight_layout(td, n_ff, n_expert * n_embd));
    const ActPtrs A = act_ptrs(act_h, act_layout(k, n_ff));
    hipError_t e = moe1_type<false>(tg, n_embd, x, A, logits, n_embd, n_ff, n_expert, k, norm, Wg, Wu, r, g, u, h, s);
    // large hidden rows: quantized once here rather than by every down workgroup
    if (e == hipSuccess && k * n_ff > kMoe1LdsHidden)
        e = launch_quantize(h, k, n_ff, n_ff, act_h, nullptr, nullptr, s, kPlanesGemv);
    if (e == hipSuccess)
        e = moe1_type<true>(td, n_ff, h, A, logits, n_embd, n_ff, n_expert, k, norm, Wd, Wd, r, dn, out, nullptr, s);
    return e;
}

}  // namespace fishhip
