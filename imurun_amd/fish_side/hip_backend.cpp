// FISH's compute-backend hook implemented over libfish_hip.so: the file FISH
// would add as model/fish/src/gpu/hip_backend.cpp. It is compiled against
// FISH's own headers (fish/backend.h, backend.h:26-163), registers itself at
// load the way the Vulkan backend does (vulkan_backend.cpp:2168-2177), and
// forwards every call to the C ABI of include/fish_hip.h. FISH's routing
// (matmul_tensor / matmul_tensors, ops.cpp:283-299) then sends every matmul on
// a resident tensor to the GPU and keeps everything else on the CPU.
//
// Contracts kept (backend.h:11-17): upload() happens at load and fails
// without side effects when a type or shape is not supported; matmul() is
// synchronous; a false return makes FISH recompute on the CPU; one call at a
// time (the C ABI serialises); after a HIP error every call returns false.
#include <fish/backend.h>

#include <cstdlib>
#include <vector>

#include "fish_hip.h"

namespace fish {
namespace {

class HipComputeBackend final : public ComputeBackend {
public:
    const char* name() const override { return "hip"; }
    const char* device_name() const override { return fish_hip_device_name(); }
    uint64_t memory_total() const override { return fish_hip_memory_total(); }
    uint64_t memory_free() const override { return fish_hip_memory_free(); }
    bool supports(GgmlType t) const override { return fish_hip_supports(uint32_t(t)) != 0; }

    bool upload(const TensorInfo* t) override {
        if (!t || !t->data || t->ne.size() < 2 || !supports(t->type)) return false;
        // [ne1][ne0] rows of ne0 inputs; a 3-D expert tensor passes ne[2] experts
        const int n_expert = t->ne.size() > 2 ? int(t->ne[2]) : 1;
        return fish_hip_upload(t, uint32_t(t->type), t->data, int(t->ne[0]), int(t->ne[1]), n_expert) != 0;
    }
    bool resident(const TensorInfo* t) const override { return fish_hip_resident(t) != 0; }
    void release(const TensorInfo* t) override { fish_hip_release(t); }
    uint64_t bytes_resident() const override { return fish_hip_bytes_resident(); }

    // `acts` is not used: the device quantizer writes the same int8 bytes as ActBatch
    bool matmul(const TensorInfo* t, const float* x, const ActBatch*, int n_tok, int n_in, int n_out,
                float* y) override {
        return fish_hip_backend_matmul(t, x, n_tok, n_in, n_out, y) != 0;
    }
    bool matmul_group(const TensorInfo* const* ts, int n, const float* x, const ActBatch*, int n_tok, int n_in,
                      const int* n_outs, float* const* ys) override {
        return fish_hip_backend_matmul_group(reinterpret_cast<const void* const*>(ts), n, x, n_tok, n_in, n_outs,
                                             ys) != 0;
    }

    // Layer spans (backend.h:89-162): every field of SpanParams and SpanLayer is
    // passed on (fused q|k|v and gate|up, biases, q/k norms, post norms,
    // soft-caps, sliding windows, GELU, the int8 KV cache); a span the device
    // cannot run is refused there, and FISH then keeps routing per matmul.
    bool span_prepare(const SpanParams& p) override {
        const int n = p.layer_end - p.layer_begin;
        if (n <= 0 || !p.layers) return false;
        std::vector<fish_hip_span_layer> ls(static_cast<size_t>(n));
        for (int i = 0; i < n; ++i) {
            const SpanLayer& L = p.layers[i];
            fish_hip_span_layer& h = ls[size_t(i)];
            h = fish_hip_span_layer{};
            h.wq = L.wq;
            h.wk = L.wk;
            h.wv = L.wv;
            h.wo = L.wo;
            h.wg = L.wg;
            h.wu = L.wu;
            h.wd = L.wd;
            h.attn_norm = L.attn_norm;
            h.ffn_norm = L.ffn_norm;
            h.q_norm = L.q_norm;
            h.k_norm = L.k_norm;
            h.bias_q = L.bias_q;
            h.bias_k = L.bias_k;
            h.bias_v = L.bias_v;
            h.bias_o = L.bias_o;
            h.wqkv = L.wqkv;
            h.bias_qkv = L.bias_qkv;
            h.post_attn_norm = L.post_attn_norm;
            h.post_ffn_norm = L.post_ffn_norm;
            h.sliding_window = L.sliding_window ? 1 : 0;
            // a fused q|k|v comes with wq / wk / wv unset (model.cpp:1665-1674)
            if (h.wqkv) h.wq = h.wk = h.wv = nullptr;
        }
        fish_hip_span_params hp{};
        hp.n_layers = n;
        hp.n_embd = p.n_embd;
        hp.n_head = p.n_head;
        hp.n_head_kv = p.n_head_kv;
        hp.head_dim = p.head_dim;
        hp.n_ff = p.n_ff;
        hp.n_ctx = p.n_ctx;
        hp.eps = p.eps;
        hp.attn_scale = p.attn_scale;
        hp.rope_cos = p.rope_cos;
        hp.rope_sin = p.rope_sin;
        hp.rot_dim = p.rot_dim;
        hp.rope_neox = p.rope_neox ? 1 : 0;
        hp.layers = ls.data();
        hp.kv_q8 = p.kv_q8 ? 1 : 0;
        hp.attn_softcap = p.attn_softcap;
        hp.window = p.window;
        hp.gelu = p.gelu ? 1 : 0;
        return fish_hip_span_prepare(&hp) != 0;
    }
    bool span_forward(float* x, int n_tok, int pos0) override { return fish_hip_span_forward(x, n_tok, pos0) != 0; }
    void span_kv_truncate(int n_past) override { fish_hip_span_kv_truncate(n_past); }
    void span_release() override { fish_hip_span_release(); }
};

struct Registrar {
    Registrar() {
        const char* e = std::getenv("FISH_HIP");  // FISH_HIP=0 keeps FISH on the CPU
        if (e && *e == '0') return;
        if (fish_hip_backend_available()) set_gpu_backend(new HipComputeBackend());  // lives until exit
    }
} g_hip_registrar;

}  // namespace
}  // namespace fish
