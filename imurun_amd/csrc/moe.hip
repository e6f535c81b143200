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

// One workgroup: routing of every token, then grouping by expert.
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits, int n_tok, int n_expert, int k,
                                                    int norm, int item_tokens, MoeRouting r) {
    __shared__ int s_cnt[kMaxExperts];
    __shared__ int s_off[kMaxExperts + 1];
    const int tid = threadIdx.x;

    for (int t = tid; t < n_tok; t += blockDim.x) {
        const float* lg = logits + size_t(t) * n_expert;
        // softmax in FISH's order: max, exp(x - max) summed left to right, times 1/sum
        float m = lg[0];
        for (int e = 1; e < n_expert; ++e) m = lg[e] > m ? lg[e] : m;
        float sum = 0.0f;
        for (int e = 0; e < n_expert; ++e) sum = __fadd_rn(sum, expf(__fsub_rn(lg[e], m)));
        const bool uniform = !(sum > 0.0f);
        const float inv = uniform ? 0.0f : 1.0f / sum;
        // top-k by probability, descending; equal probabilities: lower expert first
        int chosen[kMaxK];
        float prob[kMaxK];
        float wsum = 0.0f;
        for (int j = 0; j < k; ++j) {
            int best = -1;
            float bp = 0.0f;
            for (int e = 0; e < n_expert; ++e) {
                bool used = false;
                for (int q = 0; q < j; ++q) used |= (chosen[q] == e);
                if (used) continue;
                const float p = uniform ? 1.0f / float(n_expert) : __fmul_rn(expf(__fsub_rn(lg[e], m)), inv);
                if (best < 0 || p > bp) {
                    best = e;
                    bp = p;
                }
            }
            chosen[j] = best;
            prob[j] = bp;
            wsum = __fadd_rn(wsum, bp);
        }
        for (int j = 0; j < k; ++j) {
            r.sel[t * k + j] = chosen[j];
            r.wsel[t * k + j] = (norm && wsum > 0.0f) ? prob[j] / wsum : prob[j];
        }
    }
    __syncthreads();

    for (int e = tid; e < n_expert; e += blockDim.x) {
        int c = 0;
        for (int i = 0; i < n_tok * k; ++i) c += (r.sel[i] == e);
        s_cnt[e] = c;
    }
    __syncthreads();
    if (tid == 0) {
        int off = 0, n_items = 0;
        for (int e = 0; e < n_expert; ++e) {
            s_off[e] = off;
            r.offsets[e] = off;
            r.counts[e] = s_cnt[e];
            for (int b = 0; b < s_cnt[e]; b += item_tokens) {
                r.items[3 * n_items] = e;
                r.items[3 * n_items + 1] = off + b;
                r.items[3 * n_items + 2] = min(item_tokens, s_cnt[e] - b);
                ++n_items;
            }
            off += s_cnt[e];
        }
        s_off[n_expert] = off;
        r.offsets[n_expert] = off;
        *r.n_items = n_items;
    }
    __syncthreads();
    for (int e = tid; e < n_expert; e += blockDim.x) {
        int pos = s_off[e];
        for (int t = 0; t < n_tok; ++t)
            for (int j = 0; j < k; ++j)
                if (r.sel[t * k + j] == e) {
                    r.slot_tok[pos] = t;
                    r.tok_slot[t * k + j] = pos;
                    ++pos;
                }
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
        const int j = order[q];
        const int slot = r.tok_slot[t * k + j];
        acc = __fadd_rn(acc, __fmul_rn(r.wsel[t * k + j], down[size_t(slot) * n_embd + i]));
    }
    out[gid] = acc;
}

}  // namespace

hipError_t launch_moe_route(const float* logits, int n_tok, int n_expert, int k, int norm, int item_tokens,
                            const MoeRouting& r, hipStream_t stream) {
    if (n_tok <= 0 || n_expert <= 0 || n_expert > kMaxExperts || k <= 0 || k > kMaxK || k > n_expert ||
        item_tokens <= 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(route_kernel, dim3(1), dim3(256), 0, stream, logits, n_tok, n_expert, k, norm, item_tokens, r);
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
