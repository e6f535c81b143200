// Drop-in harness over the reference's own host code -- TEST INFRASTRUCTURE ONLY.
//
// Linked by oracle/Makefile into _ref/libfishref_hip.so together with the
// reference's sources (where they lie), ref_shim.cpp and the HIP backend
// binding of imurun_amd/fish_side/hip_backend.cpp, which registers itself with
// FISH at load. These entry points let a test drive FISH's own routing
// (matmul_tensor / matmul_tensors, model/fish/src/ops.cpp:283-299) and its
// ComputeBackend contract (backend.h:26-163) exactly as FISH's model loader
// and forward pass do, and compare with FISH's CPU matmul_batch.
#include <fish/backend.h>
#include <fish/gguf.h>
#include <fish/ops.h>

#include "fish_hip.h"

#include <cstring>
#include <vector>

using namespace fish;

extern "C" {

// "hip" when the binding registered itself (a usable gfx950 device), else "".
const char* drop_backend_name(void) { return gpu_backend() ? gpu_backend()->name() : ""; }

// A 2-D weight tensor [n_out][n_in] over caller-owned GGUF bytes.
void* drop_tensor_new(uint32_t type, const void* data, int n_in, int n_out) {
    auto* t = new TensorInfo();
    t->name = "weight";
    t->type = static_cast<GgmlType>(type);
    t->ne = {static_cast<uint64_t>(n_in), static_cast<uint64_t>(n_out)};
    t->data = static_cast<const uint8_t*>(data);
    t->nbytes = ggml_row_size(t->type, static_cast<uint64_t>(n_in)) * static_cast<uint64_t>(n_out);
    return t;
}
void drop_tensor_free(void* t) { delete static_cast<TensorInfo*>(t); }

// A 3-D expert tensor [n_expert][n_out][n_in] (ne = {n_in, n_out, n_expert},
// FISH's ffn_*_exps layout, model.cpp:66-69) over caller-owned GGUF bytes.
void* drop_tensor3_new(uint32_t type, const void* data, int n_in, int n_out, int n_expert) {
    auto* t = new TensorInfo();
    t->name = "experts";
    t->type = static_cast<GgmlType>(type);
    t->ne = {static_cast<uint64_t>(n_in), static_cast<uint64_t>(n_out), static_cast<uint64_t>(n_expert)};
    t->data = static_cast<const uint8_t*>(data);
    t->nbytes = ggml_row_size(t->type, static_cast<uint64_t>(n_in)) * static_cast<uint64_t>(n_out) *
                static_cast<uint64_t>(n_expert);
    return t;
}

// What FISH's placement does at load: supports() then upload().
int drop_upload(void* t) {
    ComputeBackend* b = gpu_backend();
    const auto* ti = static_cast<const TensorInfo*>(t);
    return b && b->supports(ti->type) && b->upload(ti) ? 1 : 0;
}
int drop_resident(void* t) {
    ComputeBackend* b = gpu_backend();
    return b && b->resident(static_cast<const TensorInfo*>(t)) ? 1 : 0;
}
void drop_release(void* t) {
    if (ComputeBackend* b = gpu_backend()) b->release(static_cast<const TensorInfo*>(t));
}
uint64_t drop_bytes_resident(void) { return gpu_backend() ? gpu_backend()->bytes_resident() : 0; }

// The forward pass's call: x quantized into an ActBatch, then matmul_tensor.
void drop_matmul_tensor(void* t, const float* x, int n_tok, int n_in, int n_out, float* y) {
    ActBatch acts;
    acts.quantize(x, n_tok, n_in);
    matmul_tensor(static_cast<const TensorInfo*>(t), x, &acts, n_tok, n_in, n_out, y);
}

// Several tensors on the same x (q/k/v, gate/up): matmul_tensors.
void drop_matmul_tensors(void* const* ts, int n, const float* x, int n_tok, int n_in, const int* n_outs,
                         float* const* ys) {
    ActBatch acts;
    acts.quantize(x, n_tok, n_in);
    std::vector<const TensorInfo*> v(static_cast<size_t>(n));
    for (int i = 0; i < n; ++i) v[static_cast<size_t>(i)] = static_cast<const TensorInfo*>(ts[i]);
    matmul_tensors(v.data(), n, x, &acts, n_tok, n_in, n_outs, ys);
}

// The routed experts of LlamaModel::moe_ffn as the patched model.cpp runs them
// (the expert hook of INTEGRATION.md, placed right after the router matmul,
// model.cpp:1529): FISH's three 3-D expert TensorInfos, already uploaded
// through FISH's backend, are the keys; x is xb_ and logits the router_ rows
// the matmul left; out receives ffn_out_. 1 when the device ran it, 0 when the
// CPU loop of model.cpp:1549-1580 would run instead.
int drop_moe_ffn(void* gate, void* up, void* down, const float* x, const float* logits, int n_tok, int n_embd,
                 int n_ff, int n_expert, int k, int norm, float* out) {
    return fish_hip_backend_moe_ffn(gate, up, down, nullptr, x, logits, n_tok, n_embd, n_ff, n_expert, k, norm, out);
}

// FISH's CPU path for the same call (the backend hook bypassed).
void drop_matmul_cpu(void* t, const float* x, int n_tok, int n_in, int n_out, float* y) {
    const auto* ti = static_cast<const TensorInfo*>(t);
    ActBatch acts;
    acts.quantize(x, n_tok, n_in);
    matmul_batch(ti->type, ti->data, x, &acts, n_tok, n_in, n_out, y);
}

}  // extern "C"
