/*
 * fish_hip.h -- C ABI of the MI355X (gfx950) quantized-matmul path of FISH.
 *
 * libfish_hip.so exports these entry points. They replace FISH's CPU
 * matmul hot path and plug in where FISH's device backends plug in:
 *   - the operator surface (device pointers, asynchronous on a HIP stream)
 *     replaces ActBatch::quantize / matmul_batch / moe_ffn;
 *   - the backend surface (host pointers, synchronous) is the
 *     ComputeBackend contract of include/fish/backend.h, reachable from C.
 * Citations are files of the reference repository under model/fish/.
 *
 * Conventions
 *   type       GGUF type id (gguf.h:25-33): 2 Q4_0, 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K
 *              (int8 path); 0 F32, 1 F16, 3 Q4_1, 6 Q5_0, 7 Q5_1, 10 Q2_K, 11 Q3_K,
 *              20 IQ4_NL, 30 BF16, 39 MXFP4 (FISH's f32 path, ops.cpp:219-250: the
 *              device keeps their GGUF bytes; fish_hip_matmul_tensors and the
 *              backend surface take them, the quantized-activation entry points
 *              and the expert FFN do not)
 *   n_in (K)   reduction length; n_out (N) weight rows; n_tok (M) tokens
 *   y          f32 [n_tok][n_out], row-major (ops.h:78-84)
 *   stream     a hipStream_t passed as void*, NULL = the null stream
 *   return     0 on success, a negative code on error (fish_hip_last_error()
 *              says why), like the int-returning fish_* functions (c_api.h:98-102)
 * No entry point allocates device memory except the backend surface, which
 * owns its weight copies and staging buffers (backend.h:41-71).
 */
#ifndef FISH_HIP_H
#define FISH_HIP_H

#include <stdint.h>

#if defined(_WIN32)
#define FISH_HIP_API __declspec(dllexport)
#else
#define FISH_HIP_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define FISH_HIP_ABI_VERSION 3

#define FISH_HIP_ERR_ARG (-1)     /* bad argument or unsupported type/shape */
#define FISH_HIP_ERR_DEVICE (-2)  /* HIP runtime error; the backend is disabled */
#define FISH_HIP_ERR_NODEV (-3)   /* no usable gfx950 device */

/* ---------------------------------------------------------------- identity */

/* replaces fish_abi_version (c_api.h:93) for this library */
FISH_HIP_API int fish_hip_abi_version(void);
/* replaces fish_kernel_name (c_api.h:155-156, c_api.cpp:477): "hip-gfx950" */
FISH_HIP_API const char* fish_hip_kernel_name(void);
/* replaces fish_last_error (c_api.h:98-102); one message per calling thread */
FISH_HIP_API const char* fish_hip_last_error(void);

/* ---------------------------------------------------------------- layouts */

/* Bytes of the repacked device copy of an [n_out][n_in] tensor, 0 when the
 * type/shape is unsupported (the device counterpart of ggml_row_size * n_out,
 * gguf.cpp:258-263). */
FISH_HIP_API uint64_t fish_hip_weight_bytes(uint32_t type, int n_in, int n_out);
/* Bytes of a device activation buffer for n_tok rows of n_in values (both
 * int8 layouts of ActBatch, ops.h:63-76). */
FISH_HIP_API uint64_t fish_hip_act_bytes(int n_tok, int n_in);

/* ---------------------------------------------------------------- block writer (host) */

/* FISH's quantize_row (quant.h:119, quantize.cpp:400-416) for n_rows rows of
 * n_in f32 values on the host, byte-identical to FISH's packer, on n_threads
 * threads. Prepares weights for upload. */
FISH_HIP_API int fish_hip_quantize_rows(uint32_t type, const float* x, void* dst, int n_rows, int n_in,
                                        int n_threads);

/* ---------------------------------------------------------------- operators (device pointers) */

/* ActBatch::quantize (ops.cpp:158-175) on the device: x f32 [n_tok][n_in] ->
 * act (fish_hip_act_bytes), written with the planes a matmul of n_tok tokens
 * reads (fish_hip_matmul / _group with the same n_tok, and
 * fish_hip_block_ints for n_tok <= 4). q32_fish / q256_fish (nullable) also receive
 * FISH's byte layouts Q8Act[n_tok][n_in/32] / Q8ActK[n_tok][n_in/256]
 * (quant.h:58-70), bit-identical to quantize_acts / quantize_acts_k. */
FISH_HIP_API int fish_hip_quantize(const float* x, int n_tok, int n_in, void* act, void* q32_fish, void* q256_fish,
                                   void* stream);

/* fish_hip_quantize for the matmuls of one int8-path weight type at n_tok
 * tokens: only the planes that type's kernel reads (the K-quant GEMM, for
 * instance, reads none of the 32-value planes). The same buffer size
 * (fish_hip_act_bytes). ActBatch::quantize (ops.cpp:158-175) builds both of
 * FISH's layouts because its consumer is not known yet; a caller that knows
 * it (the device backend's matmul_tensors path, ops.cpp:283-299) skips the
 * work. Returns 0, or FISH_HIP_ERR_ARG for a type outside the int8 path. */
FISH_HIP_API int fish_hip_quantize_for(uint32_t type, const float* x, int n_tok, int n_in, void* act, void* stream);

/* Upload-time repack of GGUF rows already in device memory (n_out rows of
 * ggml_row_size(type, n_in) bytes) into the device layout at w (the device
 * side of ComputeBackend::upload, backend.h:41-42). */
FISH_HIP_API int fish_hip_repack(uint32_t type, const void* gguf, int n_in, int n_out, void* w, void* stream);

/* matmul_batch's int8 path (ops.cpp:177-216): y[t][i] = W_i . x_t on a
 * repacked tensor and a quantized activation buffer. */
FISH_HIP_API int fish_hip_matmul(uint32_t type, const void* w, const void* act, int n_tok, int n_in, int n_out,
                                 float* y, void* stream);

/* matmul_tensors (ops.cpp:283-299) and ComputeBackend::matmul_group
 * (backend.h:81-87) on the device: n (<= 4) repacked tensors ws[i] of one
 * type and n_in applied to the same quantized activations (the q/k/v or
 * gate/up projections of a layer); ys[i] f32 [n_tok][n_outs[i]]. Many-token
 * K-quant batches run as one launch whose grid spans all n tensors. */
FISH_HIP_API int fish_hip_matmul_group(uint32_t type, int n, const void* const* ws, const void* act, int n_tok,
                                       int n_in, const int* n_outs, float* const* ys, void* stream);

/* matmul_tensors on f32 input (ops.cpp:283-299 with the quantize-then-
 * multiply of the convenience matmul_batch, ops.cpp:254-264): x f32
 * [n_tok][n_in] is quantized like ActBatch::quantize and multiplied by the n
 * (<= 4) tensors ws[i]. One token with n_in <= 16384 is a single launch in
 * which every workgroup quantizes x itself (no workspace; act_workspace may
 * be NULL); otherwise act_workspace (fish_hip_act_bytes(n_tok, n_in) bytes)
 * receives the quantized activations first. For the f32-path types ws[i] are
 * GGUF bytes (fish_hip_repack copies them) and x (16-byte aligned) is used as
 * it is: each weight row is dequantised with FISH's float expressions
 * (dequant_row, quant.cpp:491-527) and dotted with x in f32, no workspace;
 * n_in % 32 == 0 (256 for Q2_K, Q3_K). */
FISH_HIP_API int fish_hip_matmul_tensors(uint32_t type, int n, const void* const* ws, const float* x, int n_tok,
                                         int n_in, const int* n_outs, float* const* ys, void* act_workspace,
                                         uint64_t act_workspace_bytes, void* stream);

/* fish_hip_matmul_tensors for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, hosts that forbid
 * hipMalloc). No counterpart in the reference: FISH's CPU path allocates its
 * ActBatch per call. The activation workspace is a fixed device array of
 * this library, FISH_HIP_NOALLOC_SCRATCH_MB MiB per GPU, held until the process
 * ends; the call allocates and frees nothing. Sizes whose quantized
 * activations (fish_hip_act_bytes(n_tok, n_in)) exceed it are refused with
 * FISH_HIP_ERR_ARG. Calls on one GPU share the array: two calls that overlap
 * on a GPU (different streams, or threads without ordering) race. */
#define FISH_HIP_NOALLOC_SCRATCH_MB 32
FISH_HIP_API int fish_hip_matmul_tensors_noalloc(uint32_t type, int n, const void* const* ws, const float* x,
                                                 int n_tok, int n_in, const int* n_outs, float* const* ys,
                                                 void* stream);
/* Bytes of that array (FISH_HIP_NOALLOC_SCRATCH_MB << 20). */
FISH_HIP_API uint64_t fish_hip_noalloc_scratch_bytes(void);

/* The per-block integers of FISH's AVX2 kernels (quant_x86.cpp:280-495) for
 * every row of w against token 0 of act: Q8_0/Q4_0 one int32 per 32-block,
 * Q4_K / Q5_K two per super-block (sum sc*dot, sum m*bsum), Q6_K one per super-block. */
FISH_HIP_API int fish_hip_block_ints(uint32_t type, const void* w, const void* act, int n_in, int n_out,
                                     int32_t* out, void* stream);

/* ---------------------------------------------------------------- expert FFN (device pointers) */

/* Device bytes of the workspace fish_hip_moe_ffn needs for these sizes
 * (0 when unsupported: n_tok <= 2048, n_expert <= 256, k <= 16, widths
 * multiples of 32). */
FISH_HIP_API uint64_t fish_hip_moe_workspace_bytes(int n_tok, int n_embd, int n_ff, int n_expert, int k);

/* LlamaModel::moe_ffn (model.cpp:1523-1580) from given router logits:
 * softmax over n_expert, top-k, renormalised when norm (expert_weights_norm,
 * model.cpp:461-462); each expert's tokens as one batch through gate, up,
 * silu(gate) * up, down; out[t] = sum of w * down in ascending expert order.
 * x f32 [n_tok][n_embd], logits f32 [n_tok][n_expert], out f32 [n_tok][n_embd];
 * w_gate / w_up: repacked n_expert * n_ff rows of n_embd (fish_hip_repack of
 * the 3-D tensor, experts contiguous as expert_ptr, model.cpp:66-69);
 * w_down: n_expert * n_embd rows of n_ff; workspace 256-byte aligned. This
 * is a new device hook: FISH's own backends never receive expert matmuls
 * (model.cpp:1466-1470). */
FISH_HIP_API int fish_hip_moe_ffn(const float* x, const float* logits, int n_tok, int n_embd, int n_ff, int n_expert,
                                  int k, int norm, uint32_t t_gate, const void* w_gate, uint32_t t_up,
                                  const void* w_up, uint32_t t_down, const void* w_down, void* workspace,
                                  uint64_t workspace_bytes, float* out, void* stream);

/* Byte offsets, inside the fish_hip_moe_ffn workspace for these sizes, of
 * the intermediate buffers a call leaves behind, in this order:
 *   0 sel int32 [n_tok][k]      1 wsel f32 [n_tok][k]
 *   2 tok_slot int32 [n_tok][k] 3 slot_tok int32 [n_tok * k]
 *   4 gate f32 [n_tok * k][n_ff]  5 up f32 [n_tok * k][n_ff]
 *   6 down f32 [n_tok * k][n_embd]
 * (slot = one chosen (token, expert) pair; slots grouped by expert, tokens
 * ascending). No counterpart in FISH, whose expert FFN keeps these in local
 * vectors (model.cpp:1549-1579); here for stage-by-stage verification.
 * Returns 0, or FISH_HIP_ERR_ARG for unsupported sizes. */
#define FISH_HIP_MOE_PARTS 7
FISH_HIP_API int fish_hip_moe_workspace_layout(int n_tok, int n_embd, int n_ff, int n_expert, int k,
                                               uint64_t* offsets);

/* The routing step alone (model.cpp:1528-1547): sel int32 [n_tok][k] and
 * wsel f32 [n_tok][k] in descending probability; workspace as for
 * fish_hip_moe_workspace_bytes(n_tok, 32, 32, n_expert, k). */
FISH_HIP_API int fish_hip_moe_route(const float* logits, int n_tok, int n_expert, int k, int norm, void* workspace,
                                    uint64_t workspace_bytes, int* sel, float* wsel, void* stream);

/* Router logits for unquantized router weights: logits[t][e] = sum_k
 * x[t][k] * w[e][k] in f32, with w n_expert rows of n_embd f32 (t_router 0)
 * or f16 (t_router 1). Replaces matmul_batch(L.gate_inp->type, ...)
 * (model.cpp:1529) on its f32 dot path (ops.cpp:220-250: dequant_row +
 * dot_f32_fast); a quantized gate_inp goes through fish_hip_matmul instead.
 * Sums are in a different order than FISH's 8-lane AVX2 dot, so results agree
 * to f32 rounding. n_embd % 4 == 0; x 16-byte aligned, w 16-byte (f32) or
 * 8-byte (f16) aligned. Returns 0 or FISH_HIP_ERR_ARG. */
FISH_HIP_API int fish_hip_router_logits(const float* x, int n_tok, int n_embd, uint32_t t_router,
                                        const void* w_router, int n_expert, float* logits, void* stream);

/* silu(g) * u (silu_inplace, ops.cpp:25-30; model.cpp:1504-1508) quantized
 * like ActBatch::quantize into act (fish_hip_act_bytes(n_rows, n_ff));
 * q256_fish and h (f32 [n_rows][n_ff]) are optional copies of FISH's Q8ActK
 * bytes and of the f32 values that were quantized. */
FISH_HIP_API int fish_hip_silu_mul_quantize(const float* g, const float* u, int n_rows, int n_ff, void* act,
                                            void* q256_fish, float* h, void* stream);

/* ---------------------------------------------------------------- backend (host pointers, synchronous) */

/* gpu_backend() != NULL (backend.h:191): a gfx950 device is usable. */
FISH_HIP_API int fish_hip_backend_available(void);
/* ComputeBackend::device_name / memory_total / memory_free (backend.h:31-36) */
FISH_HIP_API const char* fish_hip_device_name(void);
FISH_HIP_API uint64_t fish_hip_memory_total(void);
FISH_HIP_API uint64_t fish_hip_memory_free(void);
/* ComputeBackend::supports (backend.h:39): 1 when matmul on this type runs here */
FISH_HIP_API int fish_hip_supports(uint32_t type);
/* ComputeBackend::upload (backend.h:41-42): copy + repack one tensor, keyed by
 * the caller's TensorInfo* (any stable pointer). data = GGUF bytes (host).
 * n_expert > 1 uploads a 3-D [n_expert][n_out][n_in] expert tensor.
 * Returns 1 on success, 0 when refused (earlier uploads stay intact). */
FISH_HIP_API int fish_hip_upload(const void* key, uint32_t type, const void* data, int n_in, int n_out, int n_expert);
/* ComputeBackend::resident / release / bytes_resident (backend.h:43, :70-71) */
FISH_HIP_API int fish_hip_resident(const void* key);
FISH_HIP_API void fish_hip_release(const void* key);
FISH_HIP_API uint64_t fish_hip_bytes_resident(void);
/* How many fish_hip_backend_matmul / _matmul_group calls this process has
 * computed on the device (each one that returned 1), so a host can confirm
 * that its matmuls ran on the GPU rather than falling back to its CPU path.
 * No counterpart in FISH's ComputeBackend; a diagnostic like the stats FISH
 * reports (c_api.h fish_stats). */
FISH_HIP_API uint64_t fish_hip_backend_served(void);
/* ComputeBackend::matmul (backend.h:73-76): y valid on return; 1 ok, 0 failed
 * (y untouched; the caller recomputes on the CPU, ops.cpp:283-291). */
FISH_HIP_API int fish_hip_backend_matmul(const void* key, const float* x, int n_tok, int n_in, int n_out, float* y);
/* ComputeBackend::matmul_group (backend.h:78-87): several tensors, one input. */
FISH_HIP_API int fish_hip_backend_matmul_group(const void* const* keys, int n, const float* x, int n_tok, int n_in,
                                               const int* n_outs, float* const* ys);
/* The expert FFN of LlamaModel::moe_ffn (model.cpp:1523-1580) on host buffers:
 * the hook FISH lacks, since mm(expert >= 0) calls matmul_batch directly
 * (model.cpp:1466-1470). key_gate / key_up / key_down are the 3-D expert
 * tensors uploaded with n_expert = ne[2] (gate, up [n_expert][n_ff][n_embd],
 * down [n_expert][n_embd][n_ff]). Router logits come from `logits` (host,
 * f32 [n_tok][n_expert], as matmul_batch(gate_inp) leaves them, model.cpp:1529)
 * or, when key_router is given (a resident F32 / F16 [n_expert][n_embd]
 * tensor), are computed on the device from x and `logits` may be NULL.
 * x f32 [n_tok][n_embd], out f32 [n_tok][n_embd] (host). Softmax, top-k,
 * renormalisation when norm, per-expert gate / up / silu * up / down and the
 * weighted sum in ascending expert order, as fish_hip_moe_ffn. 1 ok, 0 refused
 * or failed (out untouched; the caller runs its CPU loop). */
FISH_HIP_API int fish_hip_backend_moe_ffn(const void* key_gate, const void* key_up, const void* key_down,
                                          const void* key_router, const float* x, const float* logits, int n_tok,
                                          int n_embd, int n_ff, int n_expert, int k, int norm, float* out);

/* ---------------------------------------------------------------- layer spans (host pointers, synchronous) */

/* One dense layer of a span (backend.h:114-134 SpanLayer): the weight keys
 * given to fish_hip_upload (all resident) -- wq, wk, wv, or instead the fused
 * q|k|v wqkv [q_dim + 2 kv_dim][n_embd] (Phi-3) with wq / wk / wv NULL; wg
 * and wu, or wg NULL and wu the fused gate|up [2 n_ff][n_embd], gate rows
 * first (model.cpp:1481-1490) -- the two RMS-norm weight vectors [n_embd],
 * and optionally the Qwen-3 per-head q / k RMS-norm weights [head_dim], the
 * q / k / v / o projection biases ([q_dim], [kv_dim], [kv_dim], [n_embd]) or
 * the fused bias_qkv [q_dim + 2 kv_dim] instead of the first three, and the
 * Gemma-2 post norms [n_embd] of the attention and FFN outputs
 * (model.cpp:1758-1760, 1791-1793); NULL = absent. sliding_window: this
 * layer attends over the last fish_hip_span_params.window positions only.
 * Vectors are host memory, copied at fish_hip_span_prepare. */
typedef struct fish_hip_span_layer {
    const void* wq;
    const void* wk;
    const void* wv;
    const void* wo;
    const void* wg;
    const void* wu;
    const void* wd;
    const float* attn_norm;
    const float* ffn_norm;
    const float* q_norm;
    const float* k_norm;
    const float* bias_q;
    const float* bias_k;
    const float* bias_v;
    const float* bias_o;
    const void* wqkv;
    const float* bias_qkv;
    const float* post_attn_norm;
    const float* post_ffn_norm;
    int sliding_window;
} fish_hip_span_layer;

/* backend.h:136-154 SpanParams, same meaning: head_dim <= 256, n_head a
 * multiple of n_head_kv, rot_dim even and <= head_dim, RoPE tables
 * [n_ctx][rot_dim / 2] (host, copied), attn_scale 0 = 1/sqrt(head_dim). */
typedef struct fish_hip_span_params {
    int n_layers;
    int n_embd, n_head, n_head_kv, head_dim, n_ff, n_ctx;
    float eps;
    float attn_scale;
    const float* rope_cos;
    const float* rope_sin;
    int rot_dim;
    int rope_neox;
    const fish_hip_span_layer* layers;
    /* SpanParams::kv_q8 (backend.h:152-156): an int8 KV cache (one f32 scale
     * per 32 values, 2.25 bytes per K + V element) requested by FISH's planner;
     * needs kv_dim and head_dim multiples of 32, else the span is refused */
    int kv_q8;
    /* SpanParams attn_softcap (Gemma-2: scores become c tanh(s / c), 0 = none),
     * window (positions a sliding-window layer attends over) and gelu (the FFN
     * activation is FISH's tanh GELU instead of SiLU), backend.h:141-143 */
    float attn_softcap;
    int window;
    int gelu;
} fish_hip_span_params;

/* ComputeBackend::span_prepare (backend.h:156): keeps the layers' weights,
 * copies the norms, biases and RoPE tables, and allocates an f16 KV cache of
 * n_ctx positions per layer (4 bytes per position and K+V element, FISH's
 * planner budget, model.cpp:1318-1320) together with every buffer later
 * calls use, each allocation leaving FISH's VRAM headroom free
 * (vram_headroom_bytes, backend.h:171-187). Replaces an earlier span.
 * 1 ok, 0 refused (no span). */
FISH_HIP_API int fish_hip_span_prepare(const fish_hip_span_params* p);
/* ComputeBackend::span_forward (backend.h:157): x [n_tok][n_embd] (host) is the
 * residual stream entering the span's first layer; on return it leaves the
 * last one, and positions pos0 .. pos0 + n_tok - 1 are in the KV cache.
 * Batches of more than 256 tokens (FISH's largest, model.h:292) run in
 * consecutive chunks. 1 ok; 0 failed with x unmodified. */
FISH_HIP_API int fish_hip_span_forward(float* x, int n_tok, int pos0);
/* ComputeBackend::span_kv_truncate / span_release (backend.h:158-159). Positions
 * >= n_past need no clearing: every forward writes the cache rows of its own
 * positions before its attention reads them, and attends only over positions
 * up to its own, so a rewind followed by new tokens never reads a stale row. */
FISH_HIP_API void fish_hip_span_kv_truncate(int n_past);
/* The intermediate values of the last fish_hip_span_forward call (its last
 * chunk of up to 256 tokens; for a multi-layer span, those of the last layer),
 * copied to host `out` (n_floats floats), for stage-by-stage verification; no
 * counterpart in FISH, whose forward keeps them in local buffers
 * (model.cpp:1654-1801). part: 0 x (the residual stream after the call),
 * 1 attention RMS-norm output [n_tok][n_embd], 2 q, 3 k, 4 v (projection
 * outputs, before bias) [n_tok][q_dim | kv_dim], 5 q after bias, q-norm and
 * RoPE, 6 attention output [n_tok][q_dim], 7 o projection [n_tok][n_embd],
 * 8 FFN RMS-norm output, 9 silu(gate) * up [n_tok][n_ff], 10 up, 11 down
 * projection [n_tok][n_embd]; 100 / 101 rows pos0 .. pos0 + n - 1 of layer
 * `layer`'s K / V cache (f16, returned as f32) [n][kv_dim]. 1 ok, 0 refused. */
FISH_HIP_API int fish_hip_span_inspect(int part, int layer, int pos0, int n, float* out, uint64_t n_floats);
/* Tokens in the last chunk fish_hip_span_inspect returns (0 without a span call). */
FISH_HIP_API int fish_hip_span_last_tokens(void);
FISH_HIP_API void fish_hip_span_release(void);

#ifdef __cplusplus
}
#endif

#endif /* FISH_HIP_H */
