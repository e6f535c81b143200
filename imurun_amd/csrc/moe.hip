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

namespace fishhip {

namespace {

constexpr int kMaxExperts = 256;
constexpr int kMaxK = 16;
constexpr int kMaxTok = 2048;  // grouping bitmap: kMaxExperts x kMaxTok bits in LDS

// One wavefront per token: softmax over the experts in FISH's order (max,
// then exp(x - max) summed left to right, then times 1/sum), the k most
// probable by k wavefront argmax rounds (ties: lower expert), renormalised.
__global__ __launch_bounds__(256) void topk_kernel(const float* __restrict__ logits, int n_tok, int n_expert, int k,
                                                   int norm, MoeRouting r) {
    __shared__ float s_p[4][kMaxExperts];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int t = int(blockIdx.x) * 4 + w;
    if (t >= n_tok) return;
    const float* lg = logits + size_t(t) * n_expert;
    float m = -INFINITY;
    for (int e = lane; e < n_expert; e += 64) m = fmaxf(m, lg[e]);
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    for (int e = lane; e < n_expert; e += 64) s_p[w][e] = expf(__fsub_rn(lg[e], m));
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    float sum = 0.0f;
    if (lane == 0)
        for (int e = 0; e < n_expert; ++e) sum = __fadd_rn(sum, s_p[w][e]);
    sum = __shfl(sum, 0);
    const bool uniform = !(sum > 0.0f);
    const float inv = uniform ? 0.0f : 1.0f / sum;
    float p[kMaxExperts / 64];
    for (int q = 0; q < kMaxExperts / 64; ++q) {
        const int e = lane + 64 * q;
        p[q] = (e < n_expert) ? (uniform ? 1.0f / float(n_expert) : __fmul_rn(s_p[w][e], inv)) : -1.0f;
    }
    float wsum = 0.0f;
    float prob[kMaxK];
    int chosen[kMaxK];
    for (int j = 0; j < k; ++j) {
        float bp = -1.0f;
        int be = 0x7fffffff;
        for (int q = 0; q < kMaxExperts / 64; ++q) {
            const int e = lane + 64 * q;
            if (p[q] > bp) { bp = p[q]; be = e; }
        }
        for (int off = 32; off > 0; off >>= 1) {
            const float op = __shfl_xor(bp, off);
            const int oe = __shfl_xor(be, off);
            if (op > bp || (op == bp && oe < be)) { bp = op; be = oe; }
        }
        chosen[j] = be;
        prob[j] = bp;
        wsum = __fadd_rn(wsum, bp);
        for (int q = 0; q < kMaxExperts / 64; ++q)
            if (lane + 64 * q == be) p[q] = -2.0f;  // taken
    }
    if (lane == 0)
        for (int j = 0; j < k; ++j) {
            r.sel[t * k + j] = chosen[j];
            r.wsel[t * k + j] = (norm && wsum > 0.0f) ? prob[j] / wsum : prob[j];
        }
}

// One workgroup: group the (token, choice) pairs by expert, tokens ascending,
// through an expert x token bitmap (rank = set bits before the token), and
// write the work list of items of at most item_tokens slots.
__global__ __launch_bounds__(256) void group_kernel(int n_tok, int n_expert, int k, int item_tokens, MoeRouting r) {
    __shared__ uint32_t s_bits[kMaxExperts * (kMaxTok / 32)];
    __shared__ int s_off[kMaxExperts + 1];
    const int tid = threadIdx.x;
    const int words = (n_tok + 31) / 32;
    for (int i = tid; i < n_expert * words; i += blockDim.x) s_bits[i] = 0;
    __syncthreads();
    for (int i = tid; i < n_tok * k; i += blockDim.x) {
        const int t = i / k, e = r.sel[i];
        atomicOr(&s_bits[e * words + t / 32], 1u << (t % 32));
    }
    __syncthreads();
    for (int e = tid; e < n_expert; e += blockDim.x) {
        int c = 0;
        for (int q = 0; q < words; ++q) c += __popc(s_bits[e * words + q]);
        r.counts[e] = c;
    }
    __syncthreads();
    if (tid == 0) {
        int off = 0, n_items = 0;
        for (int e = 0; e < n_expert; ++e) {
            const int c = r.counts[e];
            s_off[e] = off;
            r.offsets[e] = off;
            for (int b = 0; b < c; b += item_tokens) {
                r.items[3 * n_items] = e;
                r.items[3 * n_items + 1] = off + b;
                r.items[3 * n_items + 2] = min(item_tokens, c - b);
                ++n_items;
            }
            off += c;
        }
        s_off[n_expert] = off;
        r.offsets[n_expert] = off;
        *r.n_items = n_items;
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

// One thread per (token, column).
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ down, MoeRouting r, int n_tok, int k,
                                                      int n_embd, float* __restrict__ out) {
    const long gid = long(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= long(n_tok) * n_embd) return;
    const int t = int(gid / n_embd), i = int(gid % n_embd);
    // the token's choices in ascending expert order (k is small)
    int order[kMaxK];
    for (int j = 0; j < k; ++j) order[j] = j;
    for (int a = 1; a < k; ++a) {
        const int v = order[a];
        int b = a - 1;
        while (b >= 0 && r.sel[t * k + order[b]] > r.sel[t * k + v]) {
            order[b + 1] = order[b];
            --b;
        }
        order[b + 1] = v;
    }
    float acc = 0.0f;
    for (int q = 0; q < k; ++q) {
        // w * down is rounded before the add: this file is built without
        // multiply-add contraction
        const int j = order[q];
        const int slot = r.tok_slot[t * k + j];
        const float p = r.wsel[t * k + j] * down[size_t(slot) * n_embd + i];
        acc = acc + p;
    }
    out[gid] = acc;
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

hipError_t launch_moe_combine(const float* down, const MoeRouting& r, int n_tok, int k, int n_embd, float* out,
                              hipStream_t stream) {
    const long n = long(n_tok) * n_embd;
    hipLaunchKernelGGL(combine_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, down, r, n_tok, k,
                       n_embd, out);
    return hipGetLastError();
}

}  // namespace fishhip
