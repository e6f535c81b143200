// Host-side launchers of the gfx950 kernels (internal to libfish_hip.so).
// Every launcher is asynchronous on `stream` and returns the launch status.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "common.h"

namespace fishhip {

// The calling thread's fish_hip_last_error() message (capi.cpp).
void set_last_error(const std::string& msg);

// Planes of an activation buffer a quantization writes (common.h layout):
// each matmul kernel reads its own, so a batch writes only what its
// consumers read.
enum : unsigned {
    kPlanesGemv = 1,      // q32 d32 s32 q256 d256 s16: GEMV (<= 4 tokens), per-block integers
    kPlanesBatch32 = 2,   // m32 d32: 16x16 MFMA batch kernel, Q8_0 / Q4_0
    kPlanesBatch256 = 4,  // m256 d256 bsm: 16x16 MFMA batch kernel, K-quants
    kPlanesGemm = 8,      // gA gX gJ: the K-quant GEMM
    kPlanesAll = 15,
};
// The planes a matmul of n_tok tokens reads (the dispatch of capi.cpp; rows
// that are not whole 256-value units only ever go to the GEMV).
inline unsigned planes_for_tokens(int n_tok, int n_in) {
    if (n_tok <= 4 || n_in % 256) return kPlanesGemv;
    if (n_tok <= 64) return kPlanesBatch32 | kPlanesBatch256;
    return kPlanesBatch32 | kPlanesGemm;
}

// f32 x[n_tok][ldx] -> device activation buffer `act` (act_layout(n_tok, n_in)),
// the planes in `planes` only. aos32 / aos256 (nullable) receive FISH's
// Q8Act / Q8ActK bytes as well. With u != nullptr the quantized values are
// silu(x) * u, or gelu(x) * u with gelu set (FFN gate and up, ops.cpp:25-38
// and model.cpp:1504-1508), optionally also written to h_out (row stride
// n_in; h_out == x rewrites x in place when ldx == n_in).
hipError_t launch_quantize(const float* x, int n_tok, int n_in, int ldx, void* act, void* aos32, void* aos256,
                           hipStream_t stream, unsigned planes, const float* u = nullptr, float* h_out = nullptr,
                           bool gelu = false);
// A layer's RMS norm and the quantization of its output in one launch (more
// than one token): x += y (+ b) when y is given, xn = rmsnorm(x) * w (written
// to xn, rows of n), then xn quantized into `act` (the planes in `planes`).
// Bit for bit the span's launch_rmsnorm followed by launch_quantize of xn.
hipError_t launch_rmsnorm_quantize(float* x, const float* y, const float* b, const float* w, float* xn, int n_tok,
                                   int n, float eps, void* act, unsigned planes, hipStream_t stream);

// Expert routing from router logits (model.cpp:1528-1547) and grouping of
// the chosen (token, expert) pairs by expert, tokens ascending
// (model.cpp:1551-1561). Single workgroup.
struct MoeRouting {
    int* sel;       // [n_tok][k] chosen experts, by probability
    float* wsel;    // [n_tok][k] their weights (renormalised when norm)
    int* counts;    // [n_expert]
    int* offsets;   // [n_expert + 1] first slot of each expert
    int* slot_tok;  // [n_tok * k] token of each slot
    int* tok_slot;  // [n_tok][k] slot of each (token, choice)
    int* items;     // [max_items][3] work list: expert, first slot, count
    int* n_items;   // [1]
};
hipError_t launch_moe_route(const float* logits, int n_tok, int n_expert, int k, int norm, int item_tokens,
                            const MoeRouting& r, hipStream_t stream);

// matmul_batch's f32 path (ops.cpp:219-250) for the types FISH has no int8
// kernel for: w = n_out rows of GGUF bytes on the device, x f32 [n_tok][n_in]
// (16-byte aligned), y f32 [n_tok][n_out]; n_in % 32 == 0 (256 for Q2_K, Q3_K).
bool f32path_type(uint32_t type);
hipError_t launch_dq_matmul(uint32_t type, const void* w, const float* x, int n_tok, int n_in, int n_out, float* y,
                            hipStream_t s);

// logits[t][e] = dot(x[t], w[e]) in f32 over f32 (type 0) or f16 (type 1)
// router rows (model.cpp:1529); n_embd % 4 == 0, x 16-byte and w 16-byte
// (f32) or 8-byte (f16) aligned.
hipError_t launch_router(const float* x, int n_tok, int n_embd, uint32_t type, const void* w, int n_expert,
                         float* logits, hipStream_t stream);

// The expert FFN of one token: gate+up (routing and x quantization
// in-kernel; writes the routing, gate, up and h = silu(gate)*up rows), then
// down+combine (h quantized in-kernel for small experts, else by one quantize
// launch into act_h first; writes the down rows and out).
// Slots as the grouped path's: the chosen experts ascending.
bool moe1_supported(uint32_t tg, uint32_t tu, int n_embd, int n_ff, int n_expert, int k);
hipError_t launch_moe1(const float* x, const float* logits, int n_embd, int n_ff, int n_expert, int k, int norm,
                       uint32_t tg, const void* wg, uint32_t tu, const void* wu, uint32_t td, const void* wd,
                       const MoeRouting& r, float* g, float* u, float* h, void* act_h, float* dn, float* out,
                       hipStream_t stream);

// out[t][i] = sum over the token's experts in ascending expert order of
// w * down[slot][i] (model.cpp:1574-1579).
hipError_t launch_moe_combine(const float* down, const MoeRouting& r, int n_tok, int k, int n_embd, float* out,
                              hipStream_t stream);

// GGUF rows (device bytes) -> repacked device layout (weight_layout()).
hipError_t launch_repack(uint32_t type, const void* gguf, int n_in, int n_out, void* dst, hipStream_t stream);
// The same for rows row0 .. row0 + n_rows - 1 of an n_out-row tensor (gguf holds
// just those rows): uploads stage a large tensor through a bounded buffer.
hipError_t launch_repack_rows(uint32_t type, const void* gguf, int n_in, int n_out, int row0, int n_rows, void* dst,
                              hipStream_t stream);

// Token mapping of a few-token matmul launch. Plain launches (items ==
// nullptr) take tokens 0..n_tok-1 of the activation buffer and write the same
// rows of y. Grouped launches walk a device work list of items
// {expert, first slot, count}: weight rows expert * rows_per_expert + i,
// activation rows act_row[slot] (or the slot itself when act_row is
// nullptr), output rows `slot`.
struct TokenMap {
    const int* items;
    const int* n_items;
    const int* act_row;
    int rows_per_expert;
};

// Few-token matmul: y[t * ldy + i] for t < n_tok, i < n_out. `act` holds
// act_rows rows. With `group`, blocks walk at most max_items work-list items
// of up to item_tokens (<= kGemvItemTokens) tokens each.
constexpr int kGemvItemTokens = 4;
hipError_t launch_gemv(const void* w, const WeightLayout& L, const void* act, int act_rows, int n_tok, float* y,
                       int ldy, hipStream_t stream, const TokenMap* group = nullptr, int item_tokens = 0,
                       int max_items = 0);

// One token, f32 input (matmul_batch's convenience form, ops.cpp:254-264):
// every workgroup quantizes x into LDS and runs the GEMV on it; n <= 4
// tensors of one type and n_in on the same x in one launch; y_i [n_out_i].
constexpr int kGemvXMaxGroups = 512;  // n_in <= 16384
bool gemv_x_supported(const WeightLayout& L);
// Optional prologue of launch_gemv_x (a layer's RMS norm in front of its
// projections, model.cpp:1654-1660 and 1770-1776), for n_in <= 8192: the GEMV
// input is rmsnorm(x) * w over the row, computed by every workgroup;
// workgroup 0 also writes it to xn_out.
struct RowNorm {
    const float* w;
    float* xn_out;
    float eps;
};
// Optional epilogue (a residual add after a projection, model.cpp:1749-1756
// and 1795-1800), single-tensor launches only: besides y[i] = v, x[i] =
// x[i] + (v + bias[i]) (bias may be null), by the lane that owns row i.
struct RowResid {
    float* x;
    const float* bias;
};
// An FFN's hidden activation formed by the quantization of the down
// projection's input (more than one token): h = act(g) * u, written to h
// (which may be g itself).
struct GateUp {
    const float* u;
    float* h;
    bool gelu;
};
// A layer's RMS norm in front of a group of more than one token (the span's
// prefill): x += y (+ b) when y is given, then the group's input xn =
// rmsnorm(x) * w; formed by the group's quantization when it has one.
struct PreNorm {
    float* x;
    const float* y;
    const float* b;
    const float* w;
    float eps;
};
// Tensors of two K-quant types (Q4_K with Q5_K or Q6_K, Q5_K with Q6_K) may share
// one launch when gemv_x_mixed_supported (n_in 2048..8192): both read the same
// quantization of x.
bool gemv_x_mixed_supported(int n, const WeightLayout* WLs);
// Optional epilogue of a two-tensor launch with a RowNorm, the layer's gate and
// up of one type and shape (gemv_x_pair_supported: n_in up to 8192): ys[0] =
// act(gate) * up with FISH's float steps (model.cpp:1504-1508), ys[1] = up.
enum : int { kActNone = 0, kActSilu = 1, kActGelu = 2 };
bool gemv_x_pair_supported(const WeightLayout* WLs);
hipError_t launch_gemv_x(int n, const void* const* ws, const WeightLayout* WLs, const float* x, float* const* ys,
                         hipStream_t stream, const RowNorm* norm = nullptr, const RowResid* resid = nullptr,
                         int pair_act = kActNone);

// Few-token matmul on int8 MFMA (16x16 tiles), same token mapping as
// launch_gemv; work-list items of up to kBatchItemTokens tokens. Needs
// n_in % 256 == 0.
constexpr int kBatchItemTokens = 32;
bool batch_mfma_supported(const WeightLayout& L);
hipError_t launch_batch_mfma(const void* w, const WeightLayout& L, const void* act, int act_rows, int n_tok, float* y,
                             int ldy, hipStream_t stream, const TokenMap* group = nullptr, int item_tokens = 0,
                             int max_items = 0);

// Many-token matmul on int8 MFMA (K-quants).
hipError_t launch_gemm(const void* w, const WeightLayout& L, const void* act, int n_tok, float* y, int ldy,
                       hipStream_t stream);

// Up to kGemmGroupMax weight tensors of one type and n_in applied to the same
// activations in one launch (matmul_tensors, ops.cpp:283-299): their row
// tiles share one grid, so small tensors (k, v) ride along with large ones.
constexpr int kGemmGroupMax = 4;
struct GemmGroup {
    WeightPtrs w[kGemmGroupMax];
    float* y[kGemmGroupMax];
    int n_out[kGemmGroupMax];
    int ldy[kGemmGroupMax];
    int tiles_end[kGemmGroupMax];  // cumulative row tiles
    int n;
};
hipError_t launch_gemm_group(int n, const void* const* ws, const WeightLayout* WLs, const void* act, int n_tok,
                             float* const* ys, const int* ldys, hipStream_t stream);

// Layer-span steps (span.hip): rmsnorm per token row; q/k/v preparation (biases,
// per-head q/k RMS norms, RoPE of q into q_out and of k into the f16 KV-cache
// rows pos0.., v into its cache rows); causal GQA attention per (token, head)
// over positions < ld (ld >= pos0 + n_tok): a few tokens split over position
// chunks with partials in `part`, more tokens in one pass; g = silu(g) * u;
// x += y. With pos_dev, the kernels read the first position from device memory
// instead of pos0 (a graph replayed for every decode position; the caller
// keeps pos_dev[0] + n_tok <= the cache and ld). rmsnorm with y != nullptr
// first adds y (+ b when given) into x (written back). Attention of more than
// kAttnSplitTok tokens with head dims 64, 128 or 256 (and no pos_dev, f16 cache)
// runs on MFMA tiles of 32 tokens x 32 positions, f16 products at f32 accuracy
// (q and p split into two f16 parts).
struct SpanVecs {
    const float* q_norm;  // [head_dim] or null (Qwen-3)
    const float* k_norm;
    const float* bias_q;  // [q_dim] or null
    const float* bias_k;  // [kv_dim]
    const float* bias_v;
};
constexpr int kAttnSplitTok = 4;  // tokens per call that split attention over position chunks
// One layer's K or V cache: f16 rows [n_ctx][kv_dim] (d == nullptr), or int8
// rows with one f32 scale d per 32 values [n_ctx][kv_dim / 32], value = code * d
// (d = amax / 127 and the codes by the activation quantizer's arithmetic):
// FISH's int8 span cache at 2.25 bytes per K + V element instead of 4
// (SpanParams::kv_q8, backend.h:152-156). int8 needs kv_dim and head_dim
// multiples of 32; its prefill attention takes the non-MFMA kernel.
struct KvCache {
    void* c;
    float* d;
};
hipError_t launch_rmsnorm(float* x, const float* y, const float* b, const float* w, float* out, int n_tok, int n,
                          float eps, hipStream_t s);
hipError_t launch_qkv_prep(const float* q, const float* k, const float* v, const SpanVecs& vecs, float* q_out,
                           const KvCache& kc, const KvCache& vc, int n_tok, int H, int HKV, int D, int rot_dim, bool neox,
                           float eps, int pos0, const float* cosv, const float* sinv, hipStream_t s,
                           const int* pos_dev = nullptr);
// `part` holds attention_scratch_floats(n_tok, H, D, ld) floats (0 above kAttnSplitTok tokens).
size_t attention_scratch_floats(int n_tok, int H, int D, int ld);
// softcap > 0: scores c tanh(s / c); window > 0: positions pos - window + 1 .. pos only.
hipError_t launch_attention(const float* q, const KvCache& kc, const KvCache& vc, float* out, float* part, int ld,
                            int n_tok, int H, int HKV, int D, int pos0, float scale, hipStream_t s,
                            const int* pos_dev = nullptr, float softcap = 0.0f, int window = 0);
// One token: launch_qkv_prep and launch_attention in one step (the attention
// workgroups prepare q, and the position's k / v rows, themselves).
hipError_t launch_attention_prep(const float* q, const float* k, const float* v, const SpanVecs& vecs, float* q_out,
                                 const KvCache& kc, const KvCache& vc, float* out, float* part, int ld, int H, int HKV, int D,
                                 int rot_dim, bool neox, float eps, int pos0, const float* cosv, const float* sinv,
                                 float scale, hipStream_t s, const int* pos_dev = nullptr, float softcap = 0.0f,
                                 int window = 0);
hipError_t launch_silu_mul(float* g, const float* u, size_t n, hipStream_t s, bool gelu = false);
hipError_t launch_split_rows(const float* src, int n_tok, float* d0, int w0, float* d1, int w1, float* d2, int w2,
                             hipStream_t s);
hipError_t launch_add(float* x, const float* y, size_t n, hipStream_t s);

// Per-block integer dots of every row with token 0 of `act`.
hipError_t launch_block_ints(const void* w, const WeightLayout& L, const void* act, int32_t* out, hipStream_t stream);

}  // namespace fishhip
