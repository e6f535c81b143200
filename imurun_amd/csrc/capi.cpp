// C ABI of libfish_hip.so and the host-side backend object.
//
// HipBackend mirrors FISH's ComputeBackend (include/fish/backend.h:26-163):
// weights are uploaded once (copied, then repacked on the device), keyed by
// the caller's TensorInfo pointer; matmul is synchronous; one call at a time
// (a mutex, like vulkan_backend.cpp:316); any HIP error disables the backend
// for the rest of the process (the sticky broken_ flag of
// vulkan_backend.cpp:1139-1156), after which every call returns "failed" so
// that the caller computes on the CPU (ops.cpp:283-291). The device is
// opened lazily on first use, never from a static initializer.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/fish_hip.h"
#include "common.h"
#include "kernels.h"

using namespace fishhip;

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(FISH_HIP_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// Types with an int8 path (repacked device planes, quantized activations).
bool int8_type(uint32_t type) {
    return type == kQ8_0 || type == kQ4_0 || type == kQ4_K || type == kQ5_K || type == kQ6_K;
}
// Everything the backend multiplies: the int8 types and FISH's f32-path types
// (kept on the device as their GGUF bytes).
bool type_ok(uint32_t type) { return int8_type(type) || f32path_type(type); }

// GGUF bytes of an f32-path tensor, 0 when n_in is not whole 32-value sub-blocks
// (256 for Q2_K / Q3_K) or the type is not an f32-path type.
size_t f32path_bytes(uint32_t type, int n_in, int n_out) {
    if (!f32path_type(type) || n_in <= 0 || n_out <= 0 || n_in % 32) return 0;
    if ((type == kQ2_K || type == kQ3_K) && n_in % 256) return 0;
    return gguf_row_bytes(type, n_in) * size_t(n_out);
}

// Matmul dispatch on an already quantized activation buffer: up to
// kGemvMaxTok tokens -> the bandwidth-bound GEMV; up to kBatchMaxTok tokens
// (any count for Q8_0 / Q4_0) -> the 16x16 MFMA batch kernel; more tokens of a
// K-quant -> the large-tile MFMA GEMM.
constexpr int kGemvMaxTok = 4;
constexpr int kBatchMaxTok = 64;

bool uses_gemm(const WeightLayout& L, int n_tok) { return n_tok > kBatchMaxTok && is_kquant(L.type); }

hipError_t dispatch_matmul(const void* w, const WeightLayout& L, const void* act, int n_tok, float* y, int ldy,
                           hipStream_t s) {
    if (uses_gemm(L, n_tok)) return launch_gemm(w, L, act, n_tok, y, ldy, s);
    if (n_tok > kGemvMaxTok && batch_mfma_supported(L)) return launch_batch_mfma(w, L, act, n_tok, n_tok, y, ldy, s);
    return launch_gemv(w, L, act, n_tok, n_tok, y, ldy, s);
}

// Workspace of one expert-FFN call: routing arrays, the quantized input, the
// per-slot gate/up/down rows and the quantized hidden rows (slot = one chosen
// (token, expert) pair, grouped by expert).
struct MoeWork {
    int slots = 0, item_tokens = 1, max_items = 0;
    bool mfma = false;  // expert products on the MFMA batch kernel (else the GEMV)
    size_t sel = 0, wsel = 0, counts = 0, offsets = 0, slot_tok = 0, tok_slot = 0, items = 0, n_items = 0;
    size_t act_x = 0, g = 0, u = 0, act_h = 0, h = 0, dn = 0, total = 0;
};

MoeWork moe_work(int n_tok, int n_embd, int n_ff, int n_expert, int k) {
    MoeWork w;
    if (n_tok <= 0 || n_tok > 2048 || n_embd <= 0 || n_ff <= 0 || n_expert <= 0 || k <= 0 || k > n_expert ||
        k > 16 || n_expert > 256 || n_embd % 32 || n_ff % 32)
        return w;
    w.slots = n_tok * k;
    // Work-list items: one token per item at decode sizes (every expert
    // streams its rows once anyway), else 16- or 32-token MFMA items sized to
    // the mean tokens per expert (each extra item of an expert re-reads its
    // weights: at 16 tokens per expert 32-token items measure faster).
    const int avg = (w.slots + n_expert - 1) / n_expert;
    w.mfma = avg > 1 && n_embd % 256 == 0 && n_ff % 256 == 0;
    if (w.mfma) w.item_tokens = avg <= 12 ? 16 : kBatchItemTokens;
    else w.item_tokens = avg <= 1 ? 1 : (avg <= 2 ? 2 : kGemvItemTokens);
    w.max_items = std::min(n_expert, w.slots) + w.slots / w.item_tokens + 1;
    const ActLayout ax = act_layout(n_tok, n_embd), ah = act_layout(w.slots, n_ff);
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off = align256(off + bytes);
        return at;
    };
    w.sel = take(size_t(w.slots) * 4);
    w.wsel = take(size_t(w.slots) * 4);
    w.counts = take(size_t(n_expert) * 4);
    w.offsets = take(size_t(n_expert + 1) * 4);
    w.slot_tok = take(size_t(w.slots) * 4);
    w.tok_slot = take(size_t(w.slots) * 4);
    w.items = take(size_t(w.max_items) * 12);
    w.n_items = take(4);
    w.act_x = take(ax.total);
    w.g = take(size_t(w.slots) * n_ff * 4);
    w.u = take(size_t(w.slots) * n_ff * 4);
    w.act_h = take(ah.total);
    w.h = take(size_t(w.slots) * n_ff * 4);
    w.dn = take(size_t(w.slots) * n_embd * 4);
    w.total = off;
    return w;
}

MoeRouting moe_routing(void* ws, const MoeWork& w) {
    uint8_t* b = static_cast<uint8_t*>(ws);
    MoeRouting r;
    r.sel = reinterpret_cast<int*>(b + w.sel);
    r.wsel = reinterpret_cast<float*>(b + w.wsel);
    r.counts = reinterpret_cast<int*>(b + w.counts);
    r.offsets = reinterpret_cast<int*>(b + w.offsets);
    r.slot_tok = reinterpret_cast<int*>(b + w.slot_tok);
    r.tok_slot = reinterpret_cast<int*>(b + w.tok_slot);
    r.items = reinterpret_cast<int*>(b + w.items);
    r.n_items = reinterpret_cast<int*>(b + w.n_items);
    return r;
}

// The whole expert FFN on device buffers (weights already repacked:
// gate/up n_expert * n_ff rows of n_embd, down n_expert * n_embd rows of n_ff).
hipError_t moe_ffn(const float* x, const float* logits, int n_tok, int n_embd, int n_ff, int n_expert, int k,
                   int norm, uint32_t tg, const void* wg, uint32_t tu, const void* wu, uint32_t td, const void* wd,
                   void* ws, const MoeWork& w, float* out, hipStream_t s) {
    uint8_t* b = static_cast<uint8_t*>(ws);
    const MoeRouting r = moe_routing(ws, w);
    const WeightLayout Lg = weight_layout(tg, n_embd, n_expert * n_ff);
    const WeightLayout Lu = weight_layout(tu, n_embd, n_expert * n_ff);
    const WeightLayout Ld = weight_layout(td, n_ff, n_expert * n_embd);
    if (!Lg.total || !Lu.total || !Ld.total) return hipErrorInvalidValue;
    float* g = reinterpret_cast<float*>(b + w.g);
    float* u = reinterpret_cast<float*>(b + w.u);
    float* dn = reinterpret_cast<float*>(b + w.dn);
    if (n_tok == 1 && moe1_supported(tg, tu, n_embd, n_ff, n_expert, k)) {
        float* h = reinterpret_cast<float*>(b + w.h);
        return launch_moe1(x, logits, n_embd, n_ff, n_expert, k, norm, tg, wg, tu, wu, td, wd, r, g, u, h,
                           b + w.act_h, dn, out, s);
    }
    hipError_t e = launch_moe_route(logits, n_tok, n_expert, k, norm, w.item_tokens, r, s);
    const unsigned planes = w.mfma ? (kPlanesBatch32 | kPlanesBatch256) : kPlanesGemv;
    if (e == hipSuccess) e = launch_quantize(x, n_tok, n_embd, n_embd, b + w.act_x, nullptr, nullptr, s, planes);
    auto grouped = [&](const void* wt, const WeightLayout& L, const void* act, int act_rows, float* y, int ldy,
                       const TokenMap& map) {
        if (w.mfma) return launch_batch_mfma(wt, L, act, act_rows, w.slots, y, ldy, s, &map, w.item_tokens, w.max_items);
        return launch_gemv(wt, L, act, act_rows, w.slots, y, ldy, s, &map, w.item_tokens, w.max_items);
    };
    const TokenMap up_map{r.items, r.n_items, r.slot_tok, n_ff};
    if (e == hipSuccess) e = grouped(wg, Lg, b + w.act_x, n_tok, g, n_ff, up_map);
    if (e == hipSuccess) e = grouped(wu, Lu, b + w.act_x, n_tok, u, n_ff, up_map);
    if (e == hipSuccess)
        e = launch_quantize(g, w.slots, n_ff, n_ff, b + w.act_h, nullptr, nullptr, s, planes, u, nullptr);
    const TokenMap down_map{r.items, r.n_items, nullptr, n_embd};
    if (e == hipSuccess) e = grouped(wd, Ld, b + w.act_h, w.slots, dn, n_embd, down_map);
    if (e == hipSuccess) e = launch_moe_combine(dn, r, n_tok, k, n_embd, out, s);
    return e;
}

struct Resident {
    void* dev = nullptr;
    WeightLayout layout;
    int n_expert = 1;
    size_t bytes = 0;
};

class HipBackend {
public:
    static HipBackend& instance() {
        static HipBackend* b = new HipBackend();  // deliberately leaked: no driver calls at exit
        return *b;
    }

    bool available() {
        std::lock_guard<std::mutex> lk(mu_);
        return ensure_init();
    }

    const char* device_name() {
        std::lock_guard<std::mutex> lk(mu_);
        ensure_init();
        return name_.c_str();
    }

    uint64_t memory(bool total) {
        std::lock_guard<std::mutex> lk(mu_);
        if (!ensure_init()) return 0;
        size_t f = 0, t = 0;
        if (hipMemGetInfo(&f, &t) != hipSuccess) return 0;
        return total ? t : f;
    }

    bool upload(const void* key, uint32_t type, const void* data, int n_in, int n_out, int n_expert) {
        std::lock_guard<std::mutex> lk(mu_);
        if (!ensure_init() || !key || !data || !type_ok(type) || n_expert < 1) return false;
        if (map_.count(key)) return true;
        WeightLayout L = weight_layout(type, n_in, n_out * n_expert);
        if (f32path_type(type)) {
            // f32-path types stay in their GGUF bytes
            L = WeightLayout{};
            L.type = type;
            L.n_in = n_in;
            L.n_out = n_out * n_expert;
            L.total = f32path_bytes(type, n_in, n_out * n_expert);
        }
        if (!L.total) return false;
        const size_t src_bytes = gguf_row_bytes(type, n_in) * size_t(n_out) * size_t(n_expert);
        Resident r;
        r.layout = L;
        r.n_expert = n_expert;
        r.bytes = L.total;
        void* staging = nullptr;
        if (hipMalloc(&r.dev, L.total) != hipSuccess) { r.dev = nullptr; return false; }
        if (hipMalloc(&staging, src_bytes) != hipSuccess) { (void)hipFree(r.dev); return false; }
        hipError_t e = hipMemcpyAsync(staging, data, src_bytes, hipMemcpyHostToDevice, stream_);
        if (e == hipSuccess && f32path_type(type))
            e = hipMemcpyAsync(r.dev, staging, src_bytes, hipMemcpyDeviceToDevice, stream_);
        else if (e == hipSuccess)
            e = launch_repack(type, staging, n_in, n_out * n_expert, r.dev, stream_);
        if (e == hipSuccess) e = hipStreamSynchronize(stream_);
        (void)hipFree(staging);
        if (e != hipSuccess) {
            (void)hipFree(r.dev);
            mark_broken(e, "upload");
            return false;
        }
        bytes_ += r.bytes;
        map_[key] = r;
        return true;
    }

    bool resident(const void* key) {
        std::lock_guard<std::mutex> lk(mu_);
        return !broken_ && map_.count(key) != 0;
    }

    void release(const void* key) {
        std::lock_guard<std::mutex> lk(mu_);
        auto it = map_.find(key);
        if (it == map_.end()) return;
        (void)hipFree(it->second.dev);
        bytes_ -= it->second.bytes;
        map_.erase(it);
    }

    uint64_t bytes_resident() {
        std::lock_guard<std::mutex> lk(mu_);
        return bytes_;
    }

    // Synchronous matmul group on host buffers; y untouched on failure.
    bool matmul_group(const void* const* keys, int n, const float* x, int n_tok, int n_in, const int* n_outs,
                      float* const* ys) {
        std::lock_guard<std::mutex> lk(mu_);
        if (!ensure_init() || broken_ || n <= 0 || n_tok <= 0 || !x) return false;
        std::vector<const Resident*> rs(static_cast<size_t>(n));
        size_t y_total = 0;
        for (int i = 0; i < n; ++i) {
            auto it = map_.find(keys[i]);
            if (it == map_.end()) return false;
            const Resident& r = it->second;
            if (r.layout.n_in != n_in || r.layout.n_out != n_outs[i] * r.n_expert || r.n_expert != 1) return false;
            rs[size_t(i)] = &r;
            y_total += size_t(n_tok) * size_t(n_outs[i]);
        }
        const ActLayout AL = act_layout(n_tok, n_in);
        if (!AL.total) return false;
        bool any_int8 = false;
        for (int i = 0; i < n; ++i) {
            if (is_kquant(rs[size_t(i)]->layout.type) && !AL.has256) return false;
            any_int8 = any_int8 || int8_type(rs[size_t(i)]->layout.type);
        }
        const size_t x_bytes = size_t(n_tok) * size_t(n_in) * 4;
        if (!reserve(x_bytes, AL.total, y_total * 4)) return false;
        // y_i at consecutive offsets of the staging buffer
        std::vector<float*> dys(static_cast<size_t>(n));
        size_t off = 0;
        for (int i = 0; i < n; ++i) {
            dys[size_t(i)] = static_cast<float*>(d_y_) + off;
            off += size_t(n_tok) * size_t(n_outs[i]);
        }
        hipError_t e = hipMemcpyAsync(d_x_, x, x_bytes, hipMemcpyHostToDevice, stream_);
        if (e == hipSuccess)
            e = run_group(rs.data(), n, static_cast<const float*>(d_x_), n_tok, n_in, n_outs, dys.data(), d_act_);
        if (e == hipSuccess) e = hipStreamSynchronize(stream_);
        if (e != hipSuccess) {
            mark_broken(e, "matmul");
            return false;
        }
        off = 0;
        for (int i = 0; i < n; ++i) {
            const size_t cnt = size_t(n_tok) * size_t(n_outs[i]);
            e = hipMemcpy(ys[i], static_cast<float*>(d_y_) + off, cnt * 4, hipMemcpyDeviceToHost);
            if (e != hipSuccess) {
                mark_broken(e, "readback");
                return false;
            }
            off += cnt;
        }
        ++served_;
        return true;
    }

    uint64_t served() {
        std::lock_guard<std::mutex> lk(mu_);
        return served_;
    }

    // ---------------------------------------------------------- layer spans

    bool span_prepare(const fish_hip_span_params& p) {
        std::lock_guard<std::mutex> lk(mu_);
        span_free();
        if (!ensure_init() || broken_ || p.n_layers <= 0 || !p.layers || p.n_embd <= 0 || p.n_head <= 0 ||
            p.n_head_kv <= 0 || p.n_head % p.n_head_kv || p.head_dim <= 0 || p.head_dim > 256 || p.n_ff <= 0 ||
            p.n_ctx <= 0 || p.rot_dim < 0 || p.rot_dim > p.head_dim || p.rot_dim % 2 || !p.rope_cos || !p.rope_sin)
            return false;
        const int E = p.n_embd, Q = p.n_head * p.head_dim, KV = p.n_head_kv * p.head_dim, F = p.n_ff;
        // every weight resident, unsplit, with the shapes of a dense layer
        for (int l = 0; l < p.n_layers; ++l) {
            const fish_hip_span_layer& L = p.layers[l];
            const void* keys[7] = {L.wq, L.wk, L.wv, L.wo, L.wg, L.wu, L.wd};
            const int n_in[7] = {E, E, E, Q, E, E, F}, n_out[7] = {Q, KV, KV, E, F, F, E};
            for (int i = 0; i < 7; ++i) {
                auto it = map_.find(keys[i]);
                if (it == map_.end() || it->second.n_expert != 1 || it->second.layout.n_in != n_in[i] ||
                    it->second.layout.n_out != n_out[i])
                    return false;
                span_keys_.push_back(keys[i]);
            }
            if (!L.attn_norm || !L.ffn_norm) return false;
        }
        sp_ = p;
        sp_.layers = nullptr;
        const size_t half = size_t(p.rot_dim / 2), ctx = size_t(p.n_ctx);
        const size_t norm_b = size_t(p.n_layers) * 2 * E * 4, rope_b = ctx * half * 4,
                     kv_b = size_t(p.n_layers) * ctx * KV * 4;
        hipError_t e = hipMalloc(&d_span_fixed_, norm_b + 2 * rope_b + 2 * kv_b + 256);
        if (e != hipSuccess) {
            d_span_fixed_ = nullptr;
            span_keys_.clear();
            return false;
        }
        char* b = static_cast<char*>(d_span_fixed_);
        d_norms_ = reinterpret_cast<float*>(b);
        d_cos_ = reinterpret_cast<float*>(b + norm_b);
        d_sin_ = reinterpret_cast<float*>(b + norm_b + rope_b);
        d_kc_ = reinterpret_cast<float*>(b + norm_b + 2 * rope_b);
        d_vc_ = reinterpret_cast<float*>(b + norm_b + 2 * rope_b + kv_b);
        for (int l = 0; l < p.n_layers && e == hipSuccess; ++l) {
            e = hipMemcpy(d_norms_ + size_t(2 * l) * E, p.layers[l].attn_norm, size_t(E) * 4, hipMemcpyHostToDevice);
            if (e == hipSuccess)
                e = hipMemcpy(d_norms_ + size_t(2 * l + 1) * E, p.layers[l].ffn_norm, size_t(E) * 4,
                              hipMemcpyHostToDevice);
        }
        if (e == hipSuccess && rope_b) e = hipMemcpy(d_cos_, p.rope_cos, rope_b, hipMemcpyHostToDevice);
        if (e == hipSuccess && rope_b) e = hipMemcpy(d_sin_, p.rope_sin, rope_b, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            span_free();
            mark_broken(e, "span_prepare");
            return false;
        }
        span_on_ = true;
        return true;
    }

    void span_release() {
        std::lock_guard<std::mutex> lk(mu_);
        span_free();
    }

    // One forward of the span's layers over x (host) for positions pos0.. (model.cpp:1650-1801).
    bool span_forward(float* x, int n_tok, int pos0) {
        std::lock_guard<std::mutex> lk(mu_);
        if (!span_on_ || broken_ || !x || n_tok <= 0 || pos0 < 0 || pos0 + n_tok > sp_.n_ctx) return false;
        const int E = sp_.n_embd, Q = sp_.n_head * sp_.head_dim, F = sp_.n_ff;
        std::vector<const Resident*> rs(span_keys_.size());
        for (size_t i = 0; i < rs.size(); ++i) {
            auto it = map_.find(span_keys_[i]);
            if (it == map_.end()) return false;
            rs[i] = &it->second;
        }
        if (n_tok == 1) return span_decode(x, pos0, rs);
        size_t act = 0;
        for (int n_in : {E, Q, F}) act = std::max(act, act_layout(n_tok, n_in).total);
        if (!act || !reserve(0, act, 0) || !grow_span_ws(span_ws_bytes(n_tok, pos0 + n_tok))) return false;
        SpanBufs B = span_bufs(d_span_ws_, n_tok, pos0 + n_tok);
        hipError_t e = hipMemcpyAsync(B.x, x, size_t(n_tok) * E * 4, hipMemcpyHostToDevice, stream_);
        if (e == hipSuccess) e = span_layers(rs, B, n_tok, pos0, nullptr, d_act_);
        // x is written only once everything has run
        if (e == hipSuccess) e = hipStreamSynchronize(stream_);
        if (e == hipSuccess) e = hipMemcpy(x, B.x, size_t(n_tok) * E * 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) {
            mark_broken(e, "span_forward");
            return false;
        }
        ++served_;
        return true;
    }

private:
    // Device scratch of one span call: x, xb, q, k, v, q_rot, attn, proj, g, u,
    // attention partials (positions < ld), each 256-byte aligned; then the position.
    struct SpanBufs {
        float *x, *xb, *q, *k, *v, *qr, *att, *proj, *g, *u, *sc;
        int* pos;
        int ld;
    };
    void span_sizes(int n_tok, int ld, size_t (&z)[11]) const {
        const size_t T = size_t(n_tok), E = size_t(sp_.n_embd), Q = size_t(sp_.n_head) * sp_.head_dim,
                     KV = size_t(sp_.n_head_kv) * sp_.head_dim, F = size_t(sp_.n_ff);
        const size_t v[11] = {T * E, T * E, T * Q, T * KV, T * KV, T * Q, T * Q, T * E, T * F, T * F,
                              attention_scratch_floats(n_tok, sp_.n_head, sp_.head_dim, ld)};
        for (int i = 0; i < 11; ++i) z[i] = (v[i] * 4 + 255) / 256 * 256;
    }
    size_t span_ws_bytes(int n_tok, int ld) const {
        size_t z[11], total = 256;
        span_sizes(n_tok, ld, z);
        for (size_t b : z) total += b;
        return total;
    }
    SpanBufs span_bufs(void* base, int n_tok, int ld) const {
        size_t z[11];
        span_sizes(n_tok, ld, z);
        char* b = static_cast<char*>(base);
        float* p[11];
        for (int i = 0; i < 11; ++i) {
            p[i] = reinterpret_cast<float*>(b);
            b += z[i];
        }
        return SpanBufs{p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8], p[9], p[10],
                        reinterpret_cast<int*>(b), ld};
    }

    // The span's layers on B.x (model.cpp:1650-1801), asynchronous on stream_;
    // the position comes from pos_dev when it is given.
    hipError_t span_layers(const std::vector<const Resident*>& rs, const SpanBufs& B, int n_tok, int pos0,
                           const int* pos_dev, void* act) {
        const int E = sp_.n_embd, H = sp_.n_head, HKV = sp_.n_head_kv, D = sp_.head_dim, F = sp_.n_ff;
        const int Q = H * D, KV = HKV * D;
        const size_t T = size_t(n_tok);
        const float scale = sp_.attn_scale > 0.0f ? sp_.attn_scale : 1.0f / std::sqrt(float(D));
        hipError_t e = hipSuccess;
        // the FFN residual of layer l - 1 is added by layer l's first rmsnorm
        const float* pending = nullptr;
        for (int l = 0; l < sp_.n_layers && e == hipSuccess; ++l) {
            const Resident* const* W = rs.data() + size_t(7 * l);
            float* kc = d_kc_ + size_t(l) * sp_.n_ctx * KV;
            float* vc = d_vc_ + size_t(l) * sp_.n_ctx * KV;
            const int n_qkv[3] = {Q, KV, KV}, n_e[1] = {E}, n_f[2] = {F, F};
            float* y_qkv[3] = {B.q, B.k, B.v};
            float* y_o[1] = {B.proj};
            float* y_gu[2] = {B.g, B.u};
            e = launch_rmsnorm(B.x, pending, d_norms_ + size_t(2 * l) * E, B.xb, n_tok, E, sp_.eps, stream_);
            if (e == hipSuccess) e = run_group(W, 3, B.xb, n_tok, E, n_qkv, y_qkv, act);
            if (e == hipSuccess)
                e = launch_rope_store(B.q, B.k, B.v, B.qr, kc, vc, n_tok, H, HKV, D, sp_.rot_dim, sp_.rope_neox != 0,
                                      pos0, d_cos_, d_sin_, stream_, pos_dev);
            if (e == hipSuccess)
                e = launch_attention(B.qr, kc, vc, B.att, B.sc, B.ld, n_tok, H, HKV, D, pos0, scale, stream_, pos_dev);
            if (e == hipSuccess) e = run_group(W + 3, 1, B.att, n_tok, Q, n_e, y_o, act);
            if (e == hipSuccess)
                e = launch_rmsnorm(B.x, B.proj, d_norms_ + size_t(2 * l + 1) * E, B.xb, n_tok, E, sp_.eps, stream_);
            if (e == hipSuccess) e = run_group(W + 4, 2, B.xb, n_tok, E, n_f, y_gu, act);
            if (e == hipSuccess) e = launch_silu_mul(B.g, B.u, T * F, stream_);
            if (e == hipSuccess) e = run_group(W + 6, 1, B.g, n_tok, F, n_e, y_o, act);
            pending = B.proj;
        }
        if (e == hipSuccess) e = launch_add(B.x, pending, T * E, stream_);
        return e;
    }

    // One decode token: the layer sequence is captured once into a HIP graph
    // over fixed scratch (its own activation buffer, attention partials for n_ctx,
    // the position in device memory) and replayed per token, so the launches of
    // all layers cost one graph launch.
    bool span_decode(float* x, int pos0, const std::vector<const Resident*>& rs) {
        const int E = sp_.n_embd;
        hipError_t e = hipSuccess;
        // the graph holds the weights' device addresses: rebuild it if any changed
        std::vector<const void*> devs(rs.size());
        for (size_t i = 0; i < rs.size(); ++i) devs[i] = rs[i]->dev;
        if (dec_exec_ && devs != dec_devs_) {
            (void)hipGraphExecDestroy(dec_exec_);
            dec_exec_ = nullptr;
            (void)hipFree(d_dec_);
            d_dec_ = nullptr;
        }
        if (!dec_exec_) {
            size_t act = 0;
            for (int n_in : {E, sp_.n_head * sp_.head_dim, sp_.n_ff}) act = std::max(act, act_layout(1, n_in).total);
            const size_t ws = span_ws_bytes(1, sp_.n_ctx);
            if (!act || hipMalloc(&d_dec_, ws + act) != hipSuccess) {
                d_dec_ = nullptr;
                return false;
            }
            dec_ = span_bufs(d_dec_, 1, sp_.n_ctx);
            void* dact = static_cast<char*>(d_dec_) + ws;
            hipGraph_t g = nullptr;
            e = hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal);
            if (e == hipSuccess) {
                const hipError_t le = span_layers(rs, dec_, 1, 0, dec_.pos, dact);
                e = hipStreamEndCapture(stream_, &g);
                if (e == hipSuccess) e = le;
            }
            if (e == hipSuccess) e = hipGraphInstantiate(&dec_exec_, g, nullptr, nullptr, 0);
            if (g) (void)hipGraphDestroy(g);
            if (e != hipSuccess) {
                dec_exec_ = nullptr;
                mark_broken(e, "span graph");
                return false;
            }
            dec_devs_ = devs;
        }
        const int pos_host = pos0;
        e = hipMemcpyAsync(dec_.x, x, size_t(E) * 4, hipMemcpyHostToDevice, stream_);
        if (e == hipSuccess) e = hipMemcpyAsync(dec_.pos, &pos_host, sizeof(int), hipMemcpyHostToDevice, stream_);
        if (e == hipSuccess) e = hipGraphLaunch(dec_exec_, stream_);
        if (e == hipSuccess) e = hipStreamSynchronize(stream_);
        if (e == hipSuccess) e = hipMemcpy(x, dec_.x, size_t(E) * 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) {
            mark_broken(e, "span_forward");
            return false;
        }
        ++served_;
        return true;
    }

    // The matmuls of n resident tensors on one device input (f32 [n_tok][n_in]):
    // y_i [n_tok][n_out_i] (device). Asynchronous on stream_; d_act_ must hold
    // act_layout(n_tok, n_in).total bytes.
    hipError_t run_group(const Resident* const* rs, int n, const float* dx, int n_tok, int n_in, const int* n_outs,
                         float* const* dys, void* act) {
        bool any_int8 = false;
        for (int i = 0; i < n; ++i) any_int8 = any_int8 || int8_type(rs[i]->layout.type);
        // one token, one type: each workgroup quantizes x itself (one launch)
        bool fused = n_tok == 1 && n <= kGemmGroupMax && int8_type(rs[0]->layout.type) &&
                     gemv_x_supported(rs[0]->layout);
        for (int i = 1; i < n && fused; ++i) fused = rs[i]->layout.type == rs[0]->layout.type;
        // one token, int8 types mixed (q/k in Q4_K, v in Q6_K): one fused launch per type
        bool per_type = !fused && n_tok == 1 && n <= kGemmGroupMax;
        for (int i = 0; i < n && per_type; ++i)
            per_type = int8_type(rs[i]->layout.type) && gemv_x_supported(rs[i]->layout);
        if (per_type) {
            hipError_t e = hipSuccess;
            bool done[kGemmGroupMax] = {};
            for (int i = 0; i < n && e == hipSuccess; ++i) {
                if (done[i]) continue;
                const void* ws[kGemmGroupMax];
                WeightLayout Ls[kGemmGroupMax];
                float* ys[kGemmGroupMax];
                int m = 0;
                for (int j = i; j < n; ++j) {
                    if (done[j] || rs[j]->layout.type != rs[i]->layout.type) continue;
                    done[j] = true;
                    ws[m] = rs[j]->dev;
                    Ls[m] = rs[j]->layout;
                    ys[m] = dys[j];
                    ++m;
                }
                e = launch_gemv_x(m, ws, Ls, dx, ys, stream_);
            }
            return e;
        }
        hipError_t e = hipSuccess;
        if (!fused && any_int8)
            e = launch_quantize(dx, n_tok, n_in, n_in, act, nullptr, nullptr, stream_, planes_for_tokens(n_tok, n_in));
        // tensors of one K-quant type go out as one grouped launch when the batch is GEMM-sized
        bool one_group = n <= kGemmGroupMax;
        for (int i = 0; i < n; ++i)
            one_group = one_group && rs[i]->layout.type == rs[0]->layout.type && int8_type(rs[i]->layout.type) &&
                        uses_gemm(rs[i]->layout, n_tok);
        if (e == hipSuccess && fused) {
            const void* ws[kGemmGroupMax];
            WeightLayout Ls[kGemmGroupMax];
            for (int i = 0; i < n; ++i) {
                ws[i] = rs[size_t(i)]->dev;
                Ls[i] = rs[size_t(i)]->layout;
            }
            e = launch_gemv_x(n, ws, Ls, dx, dys, stream_);
        } else if (e == hipSuccess && one_group) {
            const void* ws[kGemmGroupMax];
            WeightLayout Ls[kGemmGroupMax];
            int ldy[kGemmGroupMax];
            for (int i = 0; i < n; ++i) {
                ws[i] = rs[size_t(i)]->dev;
                Ls[i] = rs[size_t(i)]->layout;
                ldy[i] = n_outs[i];
            }
            e = launch_gemm_group(n, ws, Ls, act, n_tok, dys, ldy, stream_);
        } else {
            for (int i = 0; i < n && e == hipSuccess; ++i) {
                const Resident& r = *rs[i];
                e = f32path_type(r.layout.type)
                        ? launch_dq_matmul(r.layout.type, r.dev, dx, n_tok, n_in, n_outs[i], dys[i], stream_)
                        : dispatch_matmul(r.dev, r.layout, act, n_tok, dys[i], n_outs[i], stream_);
            }
        }
        return e;
    }

    bool grow_span_ws(size_t need) {
        if (need <= cap_span_ws_) return true;
        if (d_span_ws_) (void)hipFree(d_span_ws_);
        d_span_ws_ = nullptr;
        cap_span_ws_ = 0;
        if (hipMalloc(&d_span_ws_, need) != hipSuccess) return false;
        cap_span_ws_ = need;
        return true;
    }

    void span_free() {
        if (dec_exec_) (void)hipGraphExecDestroy(dec_exec_);
        dec_exec_ = nullptr;
        if (d_dec_) (void)hipFree(d_dec_);
        d_dec_ = nullptr;
        if (d_span_fixed_) (void)hipFree(d_span_fixed_);
        d_span_fixed_ = nullptr;
        span_keys_.clear();
        span_on_ = false;
    }

    HipBackend() = default;

    bool ensure_init() {
        if (init_done_) return ok_;
        init_done_ = true;
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return ok_ = false;
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, 0) != hipSuccess) return ok_ = false;
        name_ = p.name;
        if (std::string(p.gcnArchName).rfind("gfx950", 0) != 0) return ok_ = false;
        if (hipStreamCreate(&stream_) != hipSuccess) return ok_ = false;
        return ok_ = true;
    }

    bool reserve(size_t xb, size_t ab, size_t yb) {
        auto grow = [&](void*& p, size_t& cap, size_t need) {
            if (need <= cap) return true;
            if (p) (void)hipFree(p);
            p = nullptr;
            cap = 0;
            if (hipMalloc(&p, need) != hipSuccess) return false;
            cap = need;
            return true;
        };
        return grow(d_x_, cap_x_, xb) && grow(d_act_, cap_act_, ab) && grow(d_y_, cap_y_, yb);
    }

    void mark_broken(hipError_t e, const char* what) {
        broken_ = true;
        g_err = std::string("hip backend disabled after ") + what + ": " + hipGetErrorString(e);
        std::fprintf(stderr, "[fish_hip] %s\n", g_err.c_str());
    }

    std::mutex mu_;
    bool init_done_ = false, ok_ = false, broken_ = false;
    uint64_t served_ = 0;  // matmul groups computed on the device
    std::string name_ = "";
    hipStream_t stream_ = nullptr;
    std::unordered_map<const void*, Resident> map_;
    uint64_t bytes_ = 0;
    void *d_x_ = nullptr, *d_act_ = nullptr, *d_y_ = nullptr;
    size_t cap_x_ = 0, cap_act_ = 0, cap_y_ = 0;
    // layer span: parameters, weight keys (7 per layer), norms / RoPE tables /
    // KV cache in one allocation, per-call scratch
    bool span_on_ = false;
    fish_hip_span_params sp_{};
    std::vector<const void*> span_keys_;
    void* d_span_fixed_ = nullptr;
    float *d_norms_ = nullptr, *d_cos_ = nullptr, *d_sin_ = nullptr, *d_kc_ = nullptr, *d_vc_ = nullptr;
    void* d_span_ws_ = nullptr;
    size_t cap_span_ws_ = 0;
    // decode graph over fixed scratch (built at the first one-token call)
    hipGraphExec_t dec_exec_ = nullptr;
    void* d_dec_ = nullptr;
    SpanBufs dec_{};
    std::vector<const void*> dec_devs_;
};

}  // namespace

namespace fishhip {
void set_last_error(const std::string& msg) { g_err = msg; }
}  // namespace fishhip

extern "C" {

int fish_hip_abi_version(void) { return FISH_HIP_ABI_VERSION; }
const char* fish_hip_kernel_name(void) { return "hip-gfx950"; }
const char* fish_hip_last_error(void) { return g_err.c_str(); }

uint64_t fish_hip_weight_bytes(uint32_t type, int n_in, int n_out) {
    return f32path_type(type) ? f32path_bytes(type, n_in, n_out) : weight_layout(type, n_in, n_out).total;
}
uint64_t fish_hip_act_bytes(int n_tok, int n_in) { return act_layout(n_tok, n_in).total; }

int fish_hip_quantize(const float* x, int n_tok, int n_in, void* act, void* q32_fish, void* q256_fish, void* stream) {
    if (!x || !act || n_tok <= 0 || n_in <= 0 || n_in % 32) return fail(FISH_HIP_ERR_ARG, "quantize: bad arguments");
    const hipError_t e =
        launch_quantize(x, n_tok, n_in, n_in, act, q32_fish, q256_fish, as_stream(stream), planes_for_tokens(n_tok, n_in));
    return e == hipSuccess ? 0 : hip_fail(e, "quantize");
}

int fish_hip_repack(uint32_t type, const void* gguf, int n_in, int n_out, void* w, void* stream) {
    if (f32path_type(type)) {  // kept as GGUF bytes: a device copy
        const size_t bytes = f32path_bytes(type, n_in, n_out);
        if (!gguf || !w || !bytes) return fail(FISH_HIP_ERR_ARG, "repack: bad arguments");
        const hipError_t e = hipMemcpyAsync(w, gguf, bytes, hipMemcpyDeviceToDevice, as_stream(stream));
        return e == hipSuccess ? 0 : hip_fail(e, "repack");
    }
    if (!gguf || !w || !weight_layout(type, n_in, n_out).total) return fail(FISH_HIP_ERR_ARG, "repack: bad arguments");
    const hipError_t e = launch_repack(type, gguf, n_in, n_out, w, as_stream(stream));
    return e == hipSuccess ? 0 : hip_fail(e, "repack");
}

int fish_hip_matmul(uint32_t type, const void* w, const void* act, int n_tok, int n_in, int n_out, float* y,
                    void* stream) {
    const WeightLayout L = weight_layout(type, n_in, n_out);
    if (!w || !act || !y || !L.total || n_tok <= 0) return fail(FISH_HIP_ERR_ARG, "matmul: bad arguments");
    if (is_kquant(type) && n_in % 256) return fail(FISH_HIP_ERR_ARG, "matmul: K-quant needs n_in % 256 == 0");
    const hipError_t e = dispatch_matmul(w, L, act, n_tok, y, n_out, as_stream(stream));
    return e == hipSuccess ? 0 : hip_fail(e, "matmul");
}

int fish_hip_matmul_group(uint32_t type, int n, const void* const* ws, const void* act, int n_tok, int n_in,
                          const int* n_outs, float* const* ys, void* stream) {
    if (n <= 0 || n > kGemmGroupMax || !ws || !act || !n_outs || !ys || n_tok <= 0)
        return fail(FISH_HIP_ERR_ARG, "matmul_group: bad arguments");
    if (is_kquant(type) && n_in % 256) return fail(FISH_HIP_ERR_ARG, "matmul_group: K-quant needs n_in % 256 == 0");
    WeightLayout L[kGemmGroupMax];
    int ldy[kGemmGroupMax];
    for (int i = 0; i < n; ++i) {
        L[i] = weight_layout(type, n_in, n_outs[i]);
        ldy[i] = n_outs[i];
        if (!ws[i] || !ys[i] || !L[i].total) return fail(FISH_HIP_ERR_ARG, "matmul_group: bad tensor");
    }
    hipError_t e = hipSuccess;
    if (uses_gemm(L[0], n_tok)) {
        e = launch_gemm_group(n, ws, L, act, n_tok, ys, ldy, as_stream(stream));
    } else {
        for (int i = 0; i < n && e == hipSuccess; ++i)
            e = dispatch_matmul(ws[i], L[i], act, n_tok, ys[i], ldy[i], as_stream(stream));
    }
    return e == hipSuccess ? 0 : hip_fail(e, "matmul_group");
}

int fish_hip_matmul_tensors(uint32_t type, int n, const void* const* ws, const float* x, int n_tok, int n_in,
                            const int* n_outs, float* const* ys, void* act_workspace, uint64_t act_workspace_bytes,
                            void* stream) {
    if (n <= 0 || n > kGemmGroupMax || !ws || !x || !n_outs || !ys || n_tok <= 0 || n_in <= 0 || n_in % 32)
        return fail(FISH_HIP_ERR_ARG, "matmul_tensors: bad arguments");
    if (is_kquant(type) && n_in % 256) return fail(FISH_HIP_ERR_ARG, "matmul_tensors: K-quant needs n_in % 256 == 0");
    if (f32path_type(type)) {
        // FISH's f32 path: dequantised weights times the f32 x, no quantization
        if (reinterpret_cast<uintptr_t>(x) % 16) return fail(FISH_HIP_ERR_ARG, "matmul_tensors: x not 16-byte aligned");
        hipError_t e = hipSuccess;
        for (int i = 0; i < n && e == hipSuccess; ++i) {
            if (!ws[i] || !ys[i] || !f32path_bytes(type, n_in, n_outs[i]))
                return fail(FISH_HIP_ERR_ARG, "matmul_tensors: bad tensor");
            e = launch_dq_matmul(type, ws[i], x, n_tok, n_in, n_outs[i], ys[i], as_stream(stream));
        }
        return e == hipSuccess ? 0 : hip_fail(e, "matmul_tensors");
    }
    WeightLayout L[kGemmGroupMax];
    for (int i = 0; i < n; ++i) {
        L[i] = weight_layout(type, n_in, n_outs[i]);
        if (!ws[i] || !ys[i] || !L[i].total) return fail(FISH_HIP_ERR_ARG, "matmul_tensors: bad tensor");
    }
    hipError_t e;
    if (n_tok == 1 && gemv_x_supported(L[0])) {
        e = launch_gemv_x(n, ws, L, x, ys, as_stream(stream));
    } else {
        if (!act_workspace || act_workspace_bytes < act_layout(n_tok, n_in).total)
            return fail(FISH_HIP_ERR_ARG, "matmul_tensors: act_workspace missing or too small");
        e = launch_quantize(x, n_tok, n_in, n_in, act_workspace, nullptr, nullptr, as_stream(stream),
                            planes_for_tokens(n_tok, n_in));
        if (e == hipSuccess) {
            const int rc = fish_hip_matmul_group(type, n, ws, act_workspace, n_tok, n_in, n_outs, ys, stream);
            if (rc != 0) return rc;
        }
    }
    return e == hipSuccess ? 0 : hip_fail(e, "matmul_tensors");
}

int fish_hip_block_ints(uint32_t type, const void* w, const void* act, int n_in, int n_out, int32_t* out,
                        void* stream) {
    const WeightLayout L = weight_layout(type, n_in, n_out);
    if (!w || !act || !out || !L.total) return fail(FISH_HIP_ERR_ARG, "block_ints: bad arguments");
    const hipError_t e = launch_block_ints(w, L, act, out, as_stream(stream));
    return e == hipSuccess ? 0 : hip_fail(e, "block_ints");
}

uint64_t fish_hip_moe_workspace_bytes(int n_tok, int n_embd, int n_ff, int n_expert, int k) {
    return moe_work(n_tok, n_embd, n_ff, n_expert, k).total;
}

int fish_hip_moe_ffn(const float* x, const float* logits, int n_tok, int n_embd, int n_ff, int n_expert, int k,
                     int norm, uint32_t t_gate, const void* w_gate, uint32_t t_up, const void* w_up, uint32_t t_down,
                     const void* w_down, void* workspace, uint64_t workspace_bytes, float* out, void* stream) {
    const MoeWork w = moe_work(n_tok, n_embd, n_ff, n_expert, k);
    if (!w.total || !x || !logits || !w_gate || !w_up || !w_down || !workspace || !out)
        return fail(FISH_HIP_ERR_ARG, "moe_ffn: bad arguments");
    if (workspace_bytes < w.total) return fail(FISH_HIP_ERR_ARG, "moe_ffn: workspace too small");
    if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(FISH_HIP_ERR_ARG, "moe_ffn: workspace not 256-byte aligned");
    if (!int8_type(t_gate) || !int8_type(t_up) || !int8_type(t_down) ||
        ((is_kquant(t_gate) || is_kquant(t_up)) && n_embd % 256) || (is_kquant(t_down) && n_ff % 256))
        return fail(FISH_HIP_ERR_ARG, "moe_ffn: unsupported weight type/shape");
    const hipError_t e = moe_ffn(x, logits, n_tok, n_embd, n_ff, n_expert, k, norm, t_gate, w_gate, t_up, w_up,
                                 t_down, w_down, workspace, w, out, as_stream(stream));
    return e == hipSuccess ? 0 : hip_fail(e, "moe_ffn");
}

int fish_hip_moe_workspace_layout(int n_tok, int n_embd, int n_ff, int n_expert, int k, uint64_t* offsets) {
    const MoeWork w = moe_work(n_tok, n_embd, n_ff, n_expert, k);
    if (!w.total || !offsets) return fail(FISH_HIP_ERR_ARG, "moe_workspace_layout: bad arguments");
    const size_t parts[FISH_HIP_MOE_PARTS] = {w.sel, w.wsel, w.tok_slot, w.slot_tok, w.g, w.u, w.dn};
    for (int i = 0; i < FISH_HIP_MOE_PARTS; ++i) offsets[i] = parts[i];
    return 0;
}

int fish_hip_moe_route(const float* logits, int n_tok, int n_expert, int k, int norm, void* workspace,
                       uint64_t workspace_bytes, int* sel, float* wsel, void* stream) {
    const MoeWork w = moe_work(n_tok, 32, 32, n_expert, k);
    if (!w.total || !logits || !workspace || !sel || !wsel) return fail(FISH_HIP_ERR_ARG, "moe_route: bad arguments");
    if (workspace_bytes < w.total) return fail(FISH_HIP_ERR_ARG, "moe_route: workspace too small");
    MoeRouting r = moe_routing(workspace, w);
    r.sel = sel;
    r.wsel = wsel;
    const hipError_t e = launch_moe_route(logits, n_tok, n_expert, k, norm, w.item_tokens, r, as_stream(stream));
    return e == hipSuccess ? 0 : hip_fail(e, "moe_route");
}

int fish_hip_router_logits(const float* x, int n_tok, int n_embd, uint32_t t_router, const void* w_router,
                           int n_expert, float* logits, void* stream) {
    if (!x || !w_router || !logits || n_tok <= 0 || n_embd <= 0 || n_expert <= 0)
        return fail(FISH_HIP_ERR_ARG, "router_logits: bad arguments");
    if (t_router != kF32 && t_router != kF16) return fail(FISH_HIP_ERR_ARG, "router_logits: weights not f32 or f16");
    if (n_embd % 4) return fail(FISH_HIP_ERR_ARG, "router_logits: n_embd not a multiple of 4");
    if (n_embd > (1 << 30) || int64_t(n_tok) * n_expert > (int64_t(1) << 30))
        return fail(FISH_HIP_ERR_ARG, "router_logits: too large");
    const uintptr_t walign = t_router == kF32 ? 16 : 8;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w_router) % walign ||
        reinterpret_cast<uintptr_t>(logits) % 4)
        return fail(FISH_HIP_ERR_ARG, "router_logits: misaligned pointer");
    const hipError_t e = launch_router(x, n_tok, n_embd, t_router, w_router, n_expert, logits, as_stream(stream));
    return e == hipSuccess ? 0 : hip_fail(e, "router_logits");
}

int fish_hip_silu_mul_quantize(const float* g, const float* u, int n_rows, int n_ff, void* act, void* q256_fish,
                               float* h, void* stream) {
    if (!g || !u || !act || n_rows <= 0 || n_ff <= 0 || n_ff % 32)
        return fail(FISH_HIP_ERR_ARG, "silu_mul_quantize: bad arguments");
    const hipError_t e =
        launch_quantize(g, n_rows, n_ff, n_ff, act, nullptr, q256_fish, as_stream(stream), kPlanesAll, u, h);
    return e == hipSuccess ? 0 : hip_fail(e, "silu_mul_quantize");
}

int fish_hip_backend_available(void) { return HipBackend::instance().available() ? 1 : 0; }
const char* fish_hip_device_name(void) { return HipBackend::instance().device_name(); }
uint64_t fish_hip_memory_total(void) { return HipBackend::instance().memory(true); }
uint64_t fish_hip_memory_free(void) { return HipBackend::instance().memory(false); }
int fish_hip_supports(uint32_t type) { return type_ok(type) ? 1 : 0; }

int fish_hip_upload(const void* key, uint32_t type, const void* data, int n_in, int n_out, int n_expert) {
    return HipBackend::instance().upload(key, type, data, n_in, n_out, n_expert) ? 1 : 0;
}
int fish_hip_resident(const void* key) { return HipBackend::instance().resident(key) ? 1 : 0; }
void fish_hip_release(const void* key) { HipBackend::instance().release(key); }
uint64_t fish_hip_bytes_resident(void) { return HipBackend::instance().bytes_resident(); }
uint64_t fish_hip_backend_served(void) { return HipBackend::instance().served(); }

int fish_hip_backend_matmul(const void* key, const float* x, int n_tok, int n_in, int n_out, float* y) {
    const void* keys[1] = {key};
    float* ys[1] = {y};
    return HipBackend::instance().matmul_group(keys, 1, x, n_tok, n_in, &n_out, ys) ? 1 : 0;
}

int fish_hip_span_prepare(const fish_hip_span_params* p) {
    return p && HipBackend::instance().span_prepare(*p) ? 1 : 0;
}
int fish_hip_span_forward(float* x, int n_tok, int pos0) {
    return HipBackend::instance().span_forward(x, n_tok, pos0) ? 1 : 0;
}
void fish_hip_span_kv_truncate(int n_past) { (void)n_past; }  // positions >= n_past are rewritten before use
void fish_hip_span_release(void) { HipBackend::instance().span_release(); }

int fish_hip_backend_matmul_group(const void* const* keys, int n, const float* x, int n_tok, int n_in,
                                  const int* n_outs, float* const* ys) {
    return HipBackend::instance().matmul_group(keys, n, x, n_tok, n_in, n_outs, ys) ? 1 : 0;
}

}  // extern "C"
