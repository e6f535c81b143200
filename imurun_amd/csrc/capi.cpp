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
#include <cstdint>
#include <cmath>
#include <cstdio>
#include <cstdlib>
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

// VRAM the backend leaves free for other programs, applied to each of its
// allocations (the rule of vram_headroom_bytes, backend.h:171-187, which FISH's
// planner applies to its budget too): max(256 MB, 5 % of the heap); with
// FISH_VRAM_HEADROOM_PCT = p (0..90) p % of the heap instead; with
// FISH_VRAM_HEADROOM_MB = m (wins when both are set) m MB.
uint64_t vram_headroom_bytes(uint64_t heap) {
    uint64_t h = std::max<uint64_t>(heap / 20, uint64_t(256) << 20);
    if (const char* e = std::getenv("FISH_VRAM_HEADROOM_PCT"); e && *e) {
        const double pct = std::atof(e);
        if (pct >= 0.0 && pct <= 90.0) h = uint64_t(double(heap) * pct / 100.0);
    }
    if (const char* e = std::getenv("FISH_VRAM_HEADROOM_MB"); e && *e) {
        const long long mb = std::atoll(e);
        if (mb >= 0) h = uint64_t(mb) << 20;
    }
    return h;
}

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

// The activation planes the kernel that dispatch_matmul picks for this tensor
// reads (kernels.h): a quantization for one consumer writes only those.
unsigned planes_of(const WeightLayout& L, int n_tok) {
    if (uses_gemm(L, n_tok)) return kPlanesGemm;
    if (n_tok > kGemvMaxTok && batch_mfma_supported(L)) return is_kquant(L.type) ? kPlanesBatch256 : kPlanesBatch32;
    return kPlanesGemv;
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
        if (!ensure_init() || broken_ || !key || !data || !type_ok(type) || n_in <= 0 || n_out <= 0 || n_expert < 1)
            return false;
        if (map_.count(key)) return true;
        if (int64_t(n_out) * n_expert > (int64_t(1) << 30)) return false;
        const int rows = n_out * n_expert;
        WeightLayout L = weight_layout(type, n_in, rows);
        if (f32path_type(type)) {
            // f32-path types stay in their GGUF bytes
            L = WeightLayout{};
            L.type = type;
            L.n_in = n_in;
            L.n_out = rows;
            L.total = f32path_bytes(type, n_in, rows);
        }
        if (!L.total) return false;
        const size_t row_b = gguf_row_bytes(type, n_in);
        // whole rows through one bounded staging buffer, so a large (3-D expert)
        // tensor never needs a second device copy of its own size
        const int chunk = int(std::max<size_t>(1, std::min<size_t>(kStageBytes / row_b, size_t(rows))));
        Resident r;
        r.layout = L;
        r.n_expert = n_expert;
        r.bytes = L.total;
        if (!grow_buffer(d_stage_, cap_stage_, size_t(chunk) * row_b)) return false;
        if (dev_alloc(&r.dev, L.total) != hipSuccess) return false;
        hipError_t e = hipSuccess;
        for (int r0 = 0; r0 < rows && e == hipSuccess; r0 += chunk) {
            const int nr = std::min(chunk, rows - r0);
            e = hipMemcpyAsync(d_stage_, static_cast<const uint8_t*>(data) + size_t(r0) * row_b, size_t(nr) * row_b,
                               hipMemcpyHostToDevice, stream_);
            if (e != hipSuccess) break;
            if (f32path_type(type))
                e = hipMemcpyAsync(static_cast<uint8_t*>(r.dev) + size_t(r0) * row_b, d_stage_, size_t(nr) * row_b,
                                   hipMemcpyDeviceToDevice, stream_);
            else
                e = launch_repack_rows(type, d_stage_, n_in, rows, r0, nr, r.dev, stream_);
        }
        if (e == hipSuccess) e = hipStreamSynchronize(stream_);
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
        // every output comes back into one host staging buffer before any y_i is
        // written, so a failed readback leaves all of them untouched
        if (!grow_host(y_total * 4)) return false;
        e = hipMemcpy(h_y_, d_y_, y_total * 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) {
            mark_broken(e, "readback");
            return false;
        }
        off = 0;
        for (int i = 0; i < n; ++i) {
            const size_t cnt = size_t(n_tok) * size_t(n_outs[i]);
            std::memcpy(ys[i], static_cast<const float*>(h_y_) + off, cnt * 4);
            off += cnt;
        }
        ++served_;
        return true;
    }

    // The expert FFN on host buffers over 3-D resident expert tensors (uploaded
    // with n_expert = ne[2]); router logits from the host, or computed here from
    // a resident f32 / f16 router tensor. out written only on success.
    bool moe_ffn_host(const void* kg, const void* ku, const void* kd, const void* kr, const float* x,
                      const float* logits, int n_tok, int n_embd, int n_ff, int n_expert, int k, int norm, float* out) {
        std::lock_guard<std::mutex> lk(mu_);
        if (!ensure_init() || broken_ || !x || !out || (!logits && !kr)) return false;
        const MoeWork w = moe_work(n_tok, n_embd, n_ff, n_expert, k);
        if (!w.total) return false;
        auto find = [&](const void* key, int n_in, int n_rows, int n_exp) -> const Resident* {
            auto it = map_.find(key);
            if (it == map_.end()) return nullptr;
            const Resident& r = it->second;
            return (r.n_expert == n_exp && r.layout.n_in == n_in && r.layout.n_out == n_rows * n_exp) ? &r : nullptr;
        };
        const Resident* rg = find(kg, n_embd, n_ff, n_expert);
        const Resident* ru = find(ku, n_embd, n_ff, n_expert);
        const Resident* rd = find(kd, n_ff, n_embd, n_expert);
        const Resident* rr = kr ? find(kr, n_embd, n_expert, 1) : nullptr;
        if (!rg || !ru || !rd || (kr && !rr)) return false;
        const uint32_t tg = rg->layout.type, tu = ru->layout.type, td = rd->layout.type;
        if (!int8_type(tg) || !int8_type(tu) || !int8_type(td) || ((is_kquant(tg) || is_kquant(tu)) && n_embd % 256) ||
            (is_kquant(td) && n_ff % 256))
            return false;
        if (rr && ((rr->layout.type != kF32 && rr->layout.type != kF16) || n_embd % 4)) return false;
        const size_t xb = align256(size_t(n_tok) * n_embd * 4), lb = align256(size_t(n_tok) * n_expert * 4);
        if (!grow_buffer(d_moe_, cap_moe_, w.total + 2 * xb + lb)) return false;
        uint8_t* base = static_cast<uint8_t*>(d_moe_);
        float* dx = reinterpret_cast<float*>(base + w.total);
        float* dout = reinterpret_cast<float*>(base + w.total + xb);
        float* dl = reinterpret_cast<float*>(base + w.total + 2 * xb);
        hipError_t e = hipMemcpyAsync(dx, x, size_t(n_tok) * n_embd * 4, hipMemcpyHostToDevice, stream_);
        if (e == hipSuccess && rr)
            e = launch_router(dx, n_tok, n_embd, rr->layout.type, rr->dev, n_expert, dl, stream_);
        else if (e == hipSuccess)
            e = hipMemcpyAsync(dl, logits, size_t(n_tok) * n_expert * 4, hipMemcpyHostToDevice, stream_);
        if (e == hipSuccess)
            e = moe_ffn(dx, dl, n_tok, n_embd, n_ff, n_expert, k, norm, tg, rg->dev, tu, ru->dev, td, rd->dev, base, w,
                        dout, stream_);
        if (e == hipSuccess) e = hipStreamSynchronize(stream_);
        if (e == hipSuccess) e = hipMemcpy(out, dout, size_t(n_tok) * n_embd * 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) {
            mark_broken(e, "moe_ffn");
            return false;
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
            p.n_head_kv <= 0 || p.n_head % p.n_head_kv || p.head_dim <= 0 || p.head_dim > 256 || p.head_dim % 2 || p.n_ff <= 0 ||
            p.n_ctx <= 0 || p.rot_dim < 0 || p.rot_dim > p.head_dim || p.rot_dim % 2 || !p.rope_cos || !p.rope_sin)
            return false;
        const int E = p.n_embd, Q = p.n_head * p.head_dim, KV = p.n_head_kv * p.head_dim, F = p.n_ff;
        // the int8 cache keeps one scale per 32 values of a head (FISH sets kv_q8 only then)
        if (p.kv_q8 && (KV % 32 || p.head_dim % 32)) return false;
        if (p.attn_softcap < 0.0f || p.window < 0) return false;
        // every weight resident, unsplit, with the shapes of a dense layer; a fused q|k|v
        // (wq, wk, wv null) or a fused gate|up (wg null) in the first and sixth slot
        span_fused_qkv_.assign(size_t(p.n_layers), 0);
        span_fused_gu_.assign(size_t(p.n_layers), 0);
        span_window_.assign(size_t(p.n_layers), 0);
        span_any_fused_ = false;
        for (int l = 0; l < p.n_layers; ++l) {
            const fish_hip_span_layer& L = p.layers[l];
            const bool fq = L.wqkv != nullptr, fg = L.wg == nullptr;
            if ((fq && (L.wq || L.wk || L.wv || L.bias_q || L.bias_k || L.bias_v)) || (!fq && L.bias_qkv) ||
                !L.attn_norm || !L.ffn_norm || (!L.q_norm) != (!L.k_norm) || (L.sliding_window && p.window <= 0)) {
                span_keys_.clear();
                return false;
            }
            const void* keys[7] = {fq ? L.wqkv : L.wq, L.wk, L.wv, L.wo, L.wg, L.wu, L.wd};
            const int n_in[7] = {E, E, E, Q, E, E, F};
            const int n_out[7] = {fq ? Q + 2 * KV : Q, KV, KV, E, F, fg ? 2 * F : F, E};
            for (int i = 0; i < 7; ++i) {
                if ((fq && (i == 1 || i == 2)) || (fg && i == 4)) {  // absent in the fused form
                    span_keys_.push_back(nullptr);
                    continue;
                }
                auto it = map_.find(keys[i]);
                if (!keys[i] || it == map_.end() || it->second.n_expert != 1 || it->second.layout.n_in != n_in[i] ||
                    it->second.layout.n_out != n_out[i]) {
                    span_keys_.clear();
                    return false;
                }
                span_keys_.push_back(keys[i]);
            }
            span_fused_qkv_[size_t(l)] = fq;
            span_fused_gu_[size_t(l)] = fg;
            span_window_[size_t(l)] = L.sliding_window != 0;
            span_any_fused_ = span_any_fused_ || fq || fg;
        }
        sp_ = p;
        sp_.layers = nullptr;
        // per-layer vectors: attn_norm, ffn_norm, q_norm, k_norm, bias_q, bias_k, bias_v, bias_o,
        // post_attn_norm, post_ffn_norm (a fused bias_qkv is kept as its three parts)
        const int D = p.head_dim;
        const size_t vlen[kSpanVecs] = {size_t(E), size_t(E), size_t(D), size_t(D), size_t(Q), size_t(KV), size_t(KV),
                                        size_t(E), size_t(E), size_t(E)};
        size_t voff[kSpanVecs], per_layer = 0;
        for (int i = 0; i < kSpanVecs; ++i) {
            voff[i] = per_layer;
            per_layer += align256(vlen[i] * 4);
        }
        const size_t half = size_t(p.rot_dim / 2), ctx = size_t(p.n_ctx);
        const size_t vec_b = size_t(p.n_layers) * per_layer, rope_b = align256(ctx * half * 4),
                     kv_c = size_t(p.n_layers) * ctx * KV * (p.kv_q8 ? 1 : 2),
                     kv_s = p.kv_q8 ? size_t(p.n_layers) * ctx * (KV / 32) * 4 : 0,
                     kv_b = align256(kv_c) + align256(kv_s);
        // buffers of later calls, sized once here so that no call grows them: a
        // prefill chunk of up to kSpanChunk tokens, the decode graph's one token
        // (attention partials over the whole context), the activation buffer
        size_t act = 0;
        for (int n_in : {E, Q, F}) act = std::max(act, act_layout(kSpanChunk, n_in).total);
        const size_t ws_b = span_ws_bytes(kSpanChunk, p.n_ctx), dec_b = span_ws_bytes(1, p.n_ctx);
        size_t dec_act = 0;
        for (int n_in : {E, Q, F}) dec_act = std::max(dec_act, act_layout(1, n_in).total);
        const size_t total = vec_b + 2 * rope_b + 2 * kv_b + ws_b + align256(dec_b) + dec_act + 256;
        if (!act || !reserve(0, act, 0) || dev_alloc(&d_span_fixed_, total) != hipSuccess ||
            hipHostMalloc(&h_dec_, size_t(E) * 4 + 256, hipHostMallocDefault) != hipSuccess) {
            span_free();
            return false;
        }
        char* b = static_cast<char*>(d_span_fixed_);
        d_vecs_ = reinterpret_cast<float*>(b);
        d_cos_ = reinterpret_cast<float*>(b + vec_b);
        d_sin_ = reinterpret_cast<float*>(b + vec_b + rope_b);
        // K, then V: values (f16 or int8), then (int8) the scales
        d_kc_ = b + vec_b + 2 * rope_b;
        d_vc_ = b + vec_b + 2 * rope_b + kv_b;
        d_ks_ = p.kv_q8 ? reinterpret_cast<float*>(b + vec_b + 2 * rope_b + align256(kv_c)) : nullptr;
        d_vs_ = p.kv_q8 ? reinterpret_cast<float*>(b + vec_b + 2 * rope_b + kv_b + align256(kv_c)) : nullptr;
        d_span_ws_ = b + vec_b + 2 * rope_b + 2 * kv_b;
        d_dec_ = b + vec_b + 2 * rope_b + 2 * kv_b + ws_b;
        d_dec_act_ = b + vec_b + 2 * rope_b + 2 * kv_b + ws_b + align256(dec_b);
        span_vec_off_.assign(size_t(p.n_layers) * kSpanVecs, SIZE_MAX);
        hipError_t e = hipSuccess;
        for (int l = 0; l < p.n_layers && e == hipSuccess; ++l) {
            const fish_hip_span_layer& L = p.layers[l];
            const float* bq = L.bias_qkv ? L.bias_qkv : L.bias_q;
            const float* bk = L.bias_qkv ? L.bias_qkv + Q : L.bias_k;
            const float* bv = L.bias_qkv ? L.bias_qkv + Q + KV : L.bias_v;
            const float* src[kSpanVecs] = {L.attn_norm, L.ffn_norm, L.q_norm, L.k_norm,         bq,
                                           bk,          bv,         L.bias_o, L.post_attn_norm, L.post_ffn_norm};
            for (int i = 0; i < kSpanVecs && e == hipSuccess; ++i) {
                if (!src[i]) continue;
                const size_t at = size_t(l) * per_layer + voff[i];
                e = hipMemcpy(reinterpret_cast<char*>(d_vecs_) + at, src[i], vlen[i] * 4, hipMemcpyHostToDevice);
                span_vec_off_[size_t(l) * kSpanVecs + i] = at;
            }
        }
        if (e == hipSuccess && half) e = hipMemcpy(d_cos_, p.rope_cos, ctx * half * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess && half) e = hipMemcpy(d_sin_, p.rope_sin, ctx * half * 4, hipMemcpyHostToDevice);
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
        const size_t E = size_t(sp_.n_embd);
        std::vector<const Resident*> rs(span_keys_.size(), nullptr);
        for (size_t i = 0; i < rs.size(); ++i) {
            if (!span_keys_[i]) continue;  // a fused layer's absent slot
            auto it = map_.find(span_keys_[i]);
            if (it == map_.end()) return false;
            rs[i] = &it->second;
        }
        if (n_tok == 1) return span_decode(x, pos0, rs);
        // chunks of at most kSpanChunk tokens, in order (each attends over the
        // cache rows the earlier ones wrote); the results gather in pinned host
        // memory and reach x only once every chunk has run
        if (!grow_host(size_t(n_tok) * E * 4)) return false;
        const SpanBufs B = span_bufs(d_span_ws_, kSpanChunk, sp_.n_ctx);
        last_bufs_ = B;
        last_tok_ = std::min(kSpanChunk, n_tok - (n_tok - 1) / kSpanChunk * kSpanChunk);
        last_pos0_ = pos0 + (n_tok - 1) / kSpanChunk * kSpanChunk;
        hipError_t e = hipSuccess;
        for (int c0 = 0; c0 < n_tok && e == hipSuccess; c0 += kSpanChunk) {
            const int n = std::min(kSpanChunk, n_tok - c0);
            e = hipMemcpyAsync(B.x, x + size_t(c0) * E, size_t(n) * E * 4, hipMemcpyHostToDevice, stream_);
            if (e == hipSuccess) e = span_layers(rs, B, n, pos0 + c0, nullptr, d_act_);
            if (e == hipSuccess)
                e = hipMemcpyAsync(static_cast<float*>(h_y_) + size_t(c0) * E, B.x, size_t(n) * E * 4,
                                   hipMemcpyDeviceToHost, stream_);
        }
        if (e == hipSuccess) e = hipStreamSynchronize(stream_);
        if (e != hipSuccess) {
            mark_broken(e, "span_forward");
            return false;
        }
        std::memcpy(x, h_y_, size_t(n_tok) * E * 4);
        ++served_;
        return true;
    }

    // A buffer of the last span call's last chunk (part ids in span_sizes'
    // order, 0..11), or rows [pos0, pos0 + n) of layer `layer`'s f16 K (part 100)
    // or V (part 101) cache as f32, copied to host `out` of n_floats floats.
    bool span_inspect(int part, int layer, int pos0, int n, float* out, uint64_t n_floats) {
        std::lock_guard<std::mutex> lk(mu_);
        if (!span_on_ || broken_ || !out) return false;
        hipError_t e = hipSuccess;
        if (part == 100 || part == 101) {
            const size_t KV = size_t(sp_.n_head_kv) * sp_.head_dim;
            if (layer < 0 || layer >= sp_.n_layers || pos0 < 0 || n <= 0 || pos0 + n > sp_.n_ctx ||
                n_floats < size_t(n) * KV)
                return false;
            const size_t first = (size_t(layer) * sp_.n_ctx + pos0) * KV;  // element index
            const float* scales = part == 100 ? d_ks_ : d_vs_;
            if (scales) {
                // int8: value = code * d of its 32-value block, as the attention kernels read it
                std::vector<int8_t> codes(size_t(n) * KV);
                std::vector<float> d(size_t(n) * KV / 32);
                e = hipMemcpy(codes.data(), static_cast<const int8_t*>(part == 100 ? d_kc_ : d_vc_) + first,
                              codes.size(), hipMemcpyDeviceToHost);
                if (e == hipSuccess)
                    e = hipMemcpy(d.data(), scales + first / 32, d.size() * 4, hipMemcpyDeviceToHost);
                if (e == hipSuccess)
                    for (size_t i = 0; i < codes.size(); ++i) out[i] = float(codes[i]) * d[i / 32];
            } else {
                const _Float16* src = static_cast<const _Float16*>(part == 100 ? d_kc_ : d_vc_) + first;
                std::vector<_Float16> tmp(size_t(n) * KV);
                e = hipMemcpy(tmp.data(), src, tmp.size() * 2, hipMemcpyDeviceToHost);
                if (e == hipSuccess)
                    for (size_t i = 0; i < tmp.size(); ++i) out[i] = float(tmp[i]);
            }
        } else {
            if (last_tok_ <= 0 || part < 0 || part >= kSpanParts) return false;
            size_t z[kSpanBufs], cnt[kSpanBufs];
            span_sizes(last_tok_, last_bufs_.ld, z, cnt);
            float* const bufs[kSpanParts] = {last_bufs_.x,   last_bufs_.xb, last_bufs_.q,   last_bufs_.k,
                                             last_bufs_.v,   last_bufs_.qr, last_bufs_.att, last_bufs_.proj,
                                             last_bufs_.xb2, last_bufs_.g,  last_bufs_.u,   last_bufs_.dn};
            if (n_floats < cnt[part]) return false;
            e = hipMemcpy(out, bufs[part], cnt[part] * 4, hipMemcpyDeviceToHost);
        }
        if (e != hipSuccess) {
            mark_broken(e, "span_inspect");
            return false;
        }
        return true;
    }

    int span_last_tokens() {
        std::lock_guard<std::mutex> lk(mu_);
        return span_on_ ? last_tok_ : 0;
    }

private:
    static constexpr int kSpanChunk = 256;  // FISH's largest forward batch (model.h:292)
    static constexpr int kSpanVecs = 10;    // per-layer vectors kept on the device

    // Device scratch of one span call, each buffer 256-byte aligned, in this
    // order (the fish_hip_span_inspect part ids): x, xb (attention norm out),
    // q, k, v (projections), qr (q after bias, norm and RoPE), att, proj (o
    // projection), xb2 (FFN norm out), g (silu(g) * u after the FFN), u, dn
    // (down projection), fz (a fused projection's output before its split;
    // empty when no layer is fused), attention partials (positions < ld); then
    // the position.
    static constexpr int kSpanBufs = 14;
    static constexpr int kSpanParts = 12;  // inspectable: x .. dn
    struct SpanBufs {
        float *x, *xb, *q, *k, *v, *qr, *att, *proj, *xb2, *g, *u, *dn, *fz, *sc;
        int* pos;
        int ld;
    };
    void span_sizes(int n_tok, int ld, size_t (&z)[kSpanBufs], size_t (&cnt)[kSpanBufs]) const {
        const size_t T = size_t(n_tok), E = size_t(sp_.n_embd), Q = size_t(sp_.n_head) * sp_.head_dim,
                     KV = size_t(sp_.n_head_kv) * sp_.head_dim, F = size_t(sp_.n_ff);
        // partials for the largest call that splits attention (at most kAttnSplitTok tokens)
        const size_t part = attention_scratch_floats(std::min(n_tok, kAttnSplitTok), sp_.n_head, sp_.head_dim, ld);
        const size_t fz = span_any_fused_ ? T * std::max(Q + 2 * KV, 2 * F) : 0;
        const size_t v[kSpanBufs] = {T * E, T * E, T * Q, T * KV, T * KV, T * Q, T * Q,
                                     T * E, T * E, T * F, T * F, T * E, fz, part};
        for (int i = 0; i < kSpanBufs; ++i) {
            cnt[i] = v[i];
            z[i] = (v[i] * 4 + 255) / 256 * 256;
        }
    }
    size_t span_ws_bytes(int n_tok, int ld) const {
        size_t z[kSpanBufs], cnt[kSpanBufs], total = 256;
        span_sizes(n_tok, ld, z, cnt);
        for (size_t b : z) total += b;
        return total;
    }
    SpanBufs span_bufs(void* base, int n_tok, int ld) const {
        size_t z[kSpanBufs], cnt[kSpanBufs];
        span_sizes(n_tok, ld, z, cnt);
        char* b = static_cast<char*>(base);
        float* p[kSpanBufs];
        for (int i = 0; i < kSpanBufs; ++i) {
            p[i] = reinterpret_cast<float*>(b);
            b += z[i];
        }
        return SpanBufs{p[0], p[1], p[2],  p[3],  p[4],  p[5],  p[6], p[7],
                        p[8], p[9], p[10], p[11], p[12], p[13], reinterpret_cast<int*>(b), ld};
    }
    // device copy of per-layer vector i of layer l, or nullptr when the layer has none
    const float* span_vec(int l, int i) const {
        const size_t at = span_vec_off_[size_t(l) * kSpanVecs + i];
        return at == SIZE_MAX ? nullptr : reinterpret_cast<const float*>(reinterpret_cast<const char*>(d_vecs_) + at);
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
        // the FFN residual of an unfolded layer l - 1 is added by layer l's first rmsnorm
        const float* pending = nullptr;
        for (int l = 0; l < sp_.n_layers && e == hipSuccess; ++l) {
            const Resident* const* W = rs.data() + size_t(7 * l);
            // layer l's caches: f16, or int8 codes with one scale per 32 values
            const size_t lay = size_t(l) * sp_.n_ctx * KV, esz = d_ks_ ? 1 : 2;
            const KvCache kc{static_cast<char*>(d_kc_) + lay * esz, d_ks_ ? d_ks_ + lay / 32 : nullptr};
            const KvCache vc{static_cast<char*>(d_vc_) + lay * esz, d_vs_ ? d_vs_ + lay / 32 : nullptr};
            const SpanVecs vecs{span_vec(l, 2), span_vec(l, 3), span_vec(l, 4), span_vec(l, 5), span_vec(l, 6)};
            const bool fq = span_fused_qkv_[size_t(l)] != 0, fg = span_fused_gu_[size_t(l)] != 0;
            const float* post_a = span_vec(l, 8);
            const float* post_f = span_vec(l, 9);
            const int window = span_window_[size_t(l)] ? sp_.window : 0;
            const int n_qkv[3] = {Q, KV, KV}, n_e[1] = {E}, n_f[2] = {F, F}, n_fq[1] = {Q + 2 * KV}, n_fg[1] = {2 * F};
            float* y_qkv[3] = {B.q, B.k, B.v};
            float* y_o[1] = {B.proj};
            float* y_gu[2] = {B.g, B.u};
            float* y_d[1] = {B.dn};
            float* y_fz[1] = {B.fz};
            // one token: each norm is the prologue of its projections' fused launch and each
            // residual add the epilogue of the projection it follows, so x is rewritten only
            // by the o and down launches, row by row, and no other launch runs for them
            // (layers with a fused projection or a post norm take the general sequence)
            const bool fold = n_tok == 1 && E <= 8192 && !fq && !fg && !post_a && !post_f && foldable(W, 7);
            if (fold && pending) {
                e = launch_add(B.x, pending, T * E, stream_);
                pending = nullptr;
            }
            if (e == hipSuccess && fold) {
                const RowNorm an{span_vec(l, 0), B.xb, sp_.eps};
                e = run_group(W, 3, B.x, n_tok, E, n_qkv, y_qkv, act, &an);
            } else if (e == hipSuccess && n_tok > 1) {
                // the attention norm formed by the projections' quantization (one launch)
                const PreNorm an{B.x, pending, nullptr, span_vec(l, 0), sp_.eps};
                if (fq) {
                    // fused q|k|v (model.cpp:1665-1674): one matmul, then its columns split
                    e = run_group(W, 1, B.xb, n_tok, E, n_fq, y_fz, act, nullptr, nullptr, kActNone, nullptr, &an);
                    if (e == hipSuccess) e = launch_split_rows(B.fz, n_tok, B.q, Q, B.k, KV, B.v, KV, stream_);
                } else {
                    e = run_group(W, 3, B.xb, n_tok, E, n_qkv, y_qkv, act, nullptr, nullptr, kActNone, nullptr, &an);
                }
            } else if (e == hipSuccess) {
                e = launch_rmsnorm(B.x, pending, nullptr, span_vec(l, 0), B.xb, n_tok, E, sp_.eps, stream_);
                if (e == hipSuccess && fq) {
                    // fused q|k|v (model.cpp:1665-1674): one matmul, then its columns split
                    e = run_group(W, 1, B.xb, n_tok, E, n_fq, y_fz, act);
                    if (e == hipSuccess) e = launch_split_rows(B.fz, n_tok, B.q, Q, B.k, KV, B.v, KV, stream_);
                } else if (e == hipSuccess) {
                    e = run_group(W, 3, B.xb, n_tok, E, n_qkv, y_qkv, act);
                }
            }
            if (e == hipSuccess && n_tok == 1) {
                // one token: the attention workgroups prepare q and the new k / v rows themselves
                e = launch_attention_prep(B.q, B.k, B.v, vecs, B.qr, kc, vc, B.att, B.sc, B.ld, H, HKV, D, sp_.rot_dim,
                                          sp_.rope_neox != 0, sp_.eps, pos0, d_cos_, d_sin_, scale, stream_, pos_dev,
                                          sp_.attn_softcap, window);
            } else if (e == hipSuccess) {
                e = launch_qkv_prep(B.q, B.k, B.v, vecs, B.qr, kc, vc, n_tok, H, HKV, D, sp_.rot_dim,
                                    sp_.rope_neox != 0, sp_.eps, pos0, d_cos_, d_sin_, stream_, pos_dev);
                if (e == hipSuccess)
                    e = launch_attention(B.qr, kc, vc, B.att, B.sc, B.ld, n_tok, H, HKV, D, pos0, scale, stream_,
                                         pos_dev, sp_.attn_softcap, window);
            }
            if (e == hipSuccess && fold) {
                const RowResid ro{B.x, span_vec(l, 7)};
                const RowNorm fn{span_vec(l, 1), B.xb2, sp_.eps};
                e = run_group(W + 3, 1, B.att, n_tok, Q, n_e, y_o, act, nullptr, &ro);
                // gate and up of one type and shape: the activation is the launch's epilogue
                const WeightLayout gu[2] = {W[4]->layout, W[5]->layout};
                const int pair = gemv_x_pair_supported(gu) ? (sp_.gelu ? kActGelu : kActSilu) : kActNone;
                if (e == hipSuccess) e = run_group(W + 4, 2, B.x, n_tok, E, n_f, y_gu, act, &fn, nullptr, pair);
                if (e == hipSuccess && pair == kActNone) e = launch_silu_mul(B.g, B.u, T * F, stream_, sp_.gelu != 0);
                const RowResid rd{B.x, nullptr};
                if (e == hipSuccess) e = run_group(W + 6, 1, B.g, n_tok, F, n_e, y_d, act, nullptr, &rd);
                continue;
            }
            if (e == hipSuccess) e = run_group(W + 3, 1, B.att, n_tok, Q, n_e, y_o, act);
            // the FFN norm (x += proj (+ bias_o) first), formed by the gate / up quantization;
            // Gemma-2 norms proj + bias_o itself before the residual add (model.cpp:1756-1760)
            if (e == hipSuccess && post_a)
                e = launch_rmsnorm(B.proj, nullptr, span_vec(l, 7), post_a, B.proj, n_tok, E, sp_.eps, stream_);
            const PreNorm fnorm{B.x, B.proj, post_a ? nullptr : span_vec(l, 7), span_vec(l, 1), sp_.eps};
            const PreNorm* fpre = n_tok > 1 ? &fnorm : nullptr;  // one token: a launch of its own
            if (e == hipSuccess && !fpre)
                e = launch_rmsnorm(fnorm.x, fnorm.y, fnorm.b, fnorm.w, B.xb2, n_tok, E, sp_.eps, stream_);
            if (e == hipSuccess && fg) {
                // fused gate|up, gate rows first (model.cpp:1481-1490)
                e = run_group(W + 5, 1, B.xb2, n_tok, E, n_fg, y_fz, act, nullptr, nullptr, kActNone, nullptr, fpre);
                if (e == hipSuccess) e = launch_split_rows(B.fz, n_tok, B.g, F, B.u, F, nullptr, 0, stream_);
            } else if (e == hipSuccess) {
                e = run_group(W + 4, 2, B.xb2, n_tok, E, n_f, y_gu, act, nullptr, nullptr, kActNone, nullptr, fpre);
            }
            // act(g) * u: formed by the down projection's quantization when that reads only
            // the quantized h (one launch fewer, g read once), else a launch of its own
            const GateUp gu{B.u, B.g, sp_.gelu != 0};
            const bool gu_q = quantizes_input(W + 6, 1, n_tok);
            if (e == hipSuccess && !gu_q) e = launch_silu_mul(B.g, B.u, T * F, stream_, sp_.gelu != 0);
            if (e == hipSuccess)
                e = run_group(W + 6, 1, B.g, n_tok, F, n_e, y_d, act, nullptr, nullptr, kActNone, gu_q ? &gu : nullptr);
            // Gemma-2: the FFN output normed before the residual add (model.cpp:1791-1793)
            if (e == hipSuccess && post_f)
                e = launch_rmsnorm(B.dn, nullptr, nullptr, post_f, B.dn, n_tok, E, sp_.eps, stream_);
            pending = B.dn;
        }
        if (e == hipSuccess && pending) e = launch_add(B.x, pending, T * E, stream_);
        return e;
    }

    // One decode token: the layer sequence is captured once into a HIP graph
    // over fixed scratch (allocated at span_prepare: attention partials for
    // n_ctx, its own activation buffer, the position in device memory) and
    // replayed per token, so the launches of all layers cost one graph launch.
    bool span_decode(float* x, int pos0, const std::vector<const Resident*>& rs) {
        const int E = sp_.n_embd;
        hipError_t e = hipSuccess;
        // the graph holds the weights' device addresses: rebuild it if any changed
        std::vector<const void*> devs(rs.size());
        for (size_t i = 0; i < rs.size(); ++i) devs[i] = rs[i] ? rs[i]->dev : nullptr;  // null: a fused layer's gap
        if (dec_exec_ && devs != dec_devs_) {
            (void)hipGraphExecDestroy(dec_exec_);
            dec_exec_ = nullptr;
        }
        if (!dec_exec_) {
            dec_ = span_bufs(d_dec_, 1, sp_.n_ctx);
            // the token's x and position go in and x comes out through one pinned staging
            // buffer (h_dec_, allocated by span_prepare), as copy nodes of the graph itself:
            // one launch and one wait per token
            char* hx = static_cast<char*>(h_dec_);
            hipGraph_t g = nullptr;
            e = hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal);
            if (e == hipSuccess) {
                hipError_t le = hipMemcpyAsync(dec_.x, hx, size_t(E) * 4, hipMemcpyHostToDevice, stream_);
                if (le == hipSuccess)
                    le = hipMemcpyAsync(dec_.pos, hx + size_t(E) * 4, sizeof(int), hipMemcpyHostToDevice, stream_);
                if (le == hipSuccess) le = span_layers(rs, dec_, 1, 0, dec_.pos, d_dec_act_);
                if (le == hipSuccess)
                    le = hipMemcpyAsync(hx, dec_.x, size_t(E) * 4, hipMemcpyDeviceToHost, stream_);
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
        last_bufs_ = dec_;
        last_tok_ = 1;
        last_pos0_ = pos0;
        char* hx = static_cast<char*>(h_dec_);
        std::memcpy(hx, x, size_t(E) * 4);
        std::memcpy(hx + size_t(E) * 4, &pos0, sizeof(int));
        e = hipGraphLaunch(dec_exec_, stream_);
        if (e == hipSuccess) e = hipStreamSynchronize(stream_);
        if (e != hipSuccess) {
            mark_broken(e, "span_forward");
            return false;
        }
        std::memcpy(x, hx, size_t(E) * 4);
        ++served_;
        return true;
    }

    // The matmuls of n resident tensors on one device input (f32 [n_tok][n_in]):
    // y_i [n_tok][n_out_i] (device). Asynchronous on stream_; d_act_ must hold
    // act_layout(n_tok, n_in).total bytes.
    // tensors whose one-token matmul is a fused launch (launch_gemv_x), which can also
    // take a RowNorm prologue
    static bool foldable(const Resident* const* rs, int n) {
        for (int i = 0; i < n; ++i)
            if (!int8_type(rs[i]->layout.type) || !gemv_x_supported(rs[i]->layout)) return false;
        return true;
    }

    // A group of more than one token whose every tensor is int8 reads only the
    // quantized activations, so an activation applied by the quantization reaches
    // all of them.
    static bool quantizes_input(const Resident* const* rs, int n, int n_tok) {
        if (n_tok < 2) return false;
        for (int i = 0; i < n; ++i)
            if (!int8_type(rs[i]->layout.type)) return false;
        return true;
    }

    // norm (one token, foldable tensors only): the RowNorm prologue of every fused launch;
    // pair_act (gate and up of one type and shape, with a norm): dys[0] = act(gate) * up;
    // gu (int8 tensors of more than one token): the input is act(dx) * gu->u, formed by the
    // quantization and written to gu->h; pre (more than one token): the input dx is
    // rmsnorm(pre->x) * pre->w, formed first, by the group's quantization when it has one
    hipError_t run_group(const Resident* const* rs, int n, const float* dx, int n_tok, int n_in, const int* n_outs,
                         float* const* dys, void* act, const RowNorm* norm = nullptr,
                         const RowResid* resid = nullptr, int pair_act = kActNone, const GateUp* gu = nullptr,
                         const PreNorm* pre = nullptr) {
        if ((norm || resid) && (n_tok != 1 || n > kGemmGroupMax || !foldable(rs, n))) return hipErrorInvalidValue;
        if (gu && !quantizes_input(rs, n, n_tok)) return hipErrorInvalidValue;
        if (pre && (gu || n_tok < 2)) return hipErrorInvalidValue;
        if (resid && n != 1) return hipErrorInvalidValue;
        bool any_int8 = false;
        for (int i = 0; i < n; ++i) any_int8 = any_int8 || int8_type(rs[i]->layout.type);
        // one token, one type: each workgroup quantizes x itself (one launch)
        bool fused = n_tok == 1 && n <= kGemmGroupMax && int8_type(rs[0]->layout.type) &&
                     gemv_x_supported(rs[0]->layout);
        for (int i = 1; i < n && fused; ++i) fused = rs[i]->layout.type == rs[0]->layout.type;
        if (pair_act != kActNone && !fused) return hipErrorInvalidValue;
        // one token, int8 types mixed (q/k in Q4_K, v in Q6_K): one fused launch per type
        bool per_type = !fused && n_tok == 1 && n <= kGemmGroupMax;
        for (int i = 0; i < n && per_type; ++i)
            per_type = int8_type(rs[i]->layout.type) && gemv_x_supported(rs[i]->layout);
        if (per_type) {
            // two K-quant types in one launch when instantiated, else one launch per type
            WeightLayout Lm[kGemmGroupMax];
            const void* wm[kGemmGroupMax];
            for (int i = 0; i < n; ++i) {
                Lm[i] = rs[i]->layout;
                wm[i] = rs[i]->dev;
            }
            if (gemv_x_mixed_supported(n, Lm)) return launch_gemv_x(n, wm, Lm, dx, dys, stream_, norm, resid);
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
                e = launch_gemv_x(m, ws, Ls, dx, ys, stream_, norm, resid);
            }
            return e;
        }
        hipError_t e = hipSuccess;
        float* const xn = const_cast<float*>(dx);  // the norm's output (pre): the group's input
        if (!fused && any_int8) {
            unsigned planes = 0;  // what this group's int8 tensors read, nothing else
            for (int i = 0; i < n; ++i)
                if (int8_type(rs[i]->layout.type)) planes |= planes_of(rs[i]->layout, n_tok);
            if (pre)
                e = launch_rmsnorm_quantize(pre->x, pre->y, pre->b, pre->w, xn, n_tok, n_in, pre->eps, act, planes,
                                            stream_);
            else if (gu)
                e = launch_quantize(dx, n_tok, n_in, n_in, act, nullptr, nullptr, stream_, planes, gu->u, gu->h, gu->gelu);
            else
                e = launch_quantize(dx, n_tok, n_in, n_in, act, nullptr, nullptr, stream_, planes);
        } else if (pre) {
            e = launch_rmsnorm(pre->x, pre->y, pre->b, pre->w, xn, n_tok, n_in, pre->eps, stream_);
        }
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
            e = launch_gemv_x(n, ws, Ls, dx, dys, stream_, norm, resid, pair_act);
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
            // mixed types (a Q4_K_M layer's q, k in Q4_K and v in Q6_K): the GEMM-sized tensors
            // of each type still share one grouped launch (q with k), the rest go one by one
            bool done[kGemmGroupMax] = {};
            for (int i = 0; i < n && e == hipSuccess; ++i) {
                const Resident& r = *rs[i];
                if (i < kGemmGroupMax && done[i]) continue;
                if (n <= kGemmGroupMax && int8_type(r.layout.type) && uses_gemm(r.layout, n_tok)) {
                    const void* ws[kGemmGroupMax];
                    WeightLayout Ls[kGemmGroupMax];
                    float* ys[kGemmGroupMax];
                    int ldy[kGemmGroupMax];
                    int m = 0;
                    for (int j = i; j < n; ++j) {
                        if (done[j] || rs[j]->layout.type != r.layout.type) continue;
                        done[j] = true;
                        ws[m] = rs[j]->dev;
                        Ls[m] = rs[j]->layout;
                        ys[m] = dys[j];
                        ldy[m] = n_outs[j];
                        ++m;
                    }
                    e = launch_gemm_group(m, ws, Ls, act, n_tok, ys, ldy, stream_);
                    continue;
                }
                e = f32path_type(r.layout.type)
                        ? launch_dq_matmul(r.layout.type, r.dev, dx, n_tok, n_in, n_outs[i], dys[i], stream_)
                        : dispatch_matmul(r.dev, r.layout, act, n_tok, dys[i], n_outs[i], stream_);
            }
        }
        return e;
    }

    void span_free() {
        if (dec_exec_) (void)hipGraphExecDestroy(dec_exec_);
        dec_exec_ = nullptr;
        if (h_dec_) (void)hipHostFree(h_dec_);  // after the graph whose copy nodes use it
        h_dec_ = nullptr;
        if (d_span_fixed_) (void)hipFree(d_span_fixed_);
        d_span_fixed_ = nullptr;
        d_vecs_ = d_cos_ = d_sin_ = nullptr;
        d_kc_ = d_vc_ = nullptr;
        d_ks_ = d_vs_ = nullptr;
        d_span_ws_ = d_dec_ = d_dec_act_ = nullptr;
        span_keys_.clear();
        span_vec_off_.clear();
        span_on_ = false;
        last_tok_ = 0;
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

    // hipMalloc within the headroom rule (vram_headroom_bytes): refused, not an
    // error, when the allocation would leave less than the headroom free
    hipError_t dev_alloc(void** p, size_t bytes) {
        *p = nullptr;
        size_t f = 0, t = 0;
        if (hipMemGetInfo(&f, &t) != hipSuccess) return hipErrorOutOfMemory;
        if (bytes > f || f - bytes < vram_headroom_bytes(t)) return hipErrorOutOfMemory;
        const hipError_t e = hipMalloc(p, bytes);
        if (e != hipSuccess) *p = nullptr;
        return e;
    }

    bool grow_buffer(void*& p, size_t& cap, size_t need) {
        if (need <= cap) return true;
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
        if (dev_alloc(&p, need) != hipSuccess) return false;
        cap = need;
        return true;
    }

    bool grow_host(size_t need) {
        if (need <= cap_h_y_) return true;
        if (h_y_) (void)hipHostFree(h_y_);
        h_y_ = nullptr;
        cap_h_y_ = 0;
        if (hipHostMalloc(&h_y_, need, hipHostMallocDefault) != hipSuccess) {
            h_y_ = nullptr;
            return false;
        }
        cap_h_y_ = need;
        return true;
    }

    bool reserve(size_t xb, size_t ab, size_t yb) {
        return grow_buffer(d_x_, cap_x_, xb) && grow_buffer(d_act_, cap_act_, ab) && grow_buffer(d_y_, cap_y_, yb);
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
    // upload staging (whole rows, at most kStageBytes), expert-FFN workspace,
    // pinned host staging of matmul outputs
    static constexpr size_t kStageBytes = size_t(64) << 20;
    void* d_stage_ = nullptr;
    size_t cap_stage_ = 0;
    void* d_moe_ = nullptr;
    size_t cap_moe_ = 0;
    void* h_y_ = nullptr;
    size_t cap_h_y_ = 0;
    void* h_dec_ = nullptr;  // pinned x / position staging of the decode graph's copy nodes
    // layer span: parameters, weight keys (7 per layer); one allocation holds the
    // per-layer vectors, RoPE tables, f16 KV cache and every per-call buffer
    bool span_on_ = false;
    fish_hip_span_params sp_{};
    std::vector<const void*> span_keys_;  // 7 per layer; null: a fused layer's absent slot
    std::vector<uint8_t> span_fused_qkv_, span_fused_gu_, span_window_;  // per layer
    bool span_any_fused_ = false;
    std::vector<size_t> span_vec_off_;  // [layer][kSpanVecs] byte offset in d_vecs_, SIZE_MAX = absent
    void* d_span_fixed_ = nullptr;
    float *d_vecs_ = nullptr, *d_cos_ = nullptr, *d_sin_ = nullptr;
    void *d_kc_ = nullptr, *d_vc_ = nullptr;  // K / V caches: f16, or int8 codes
    float *d_ks_ = nullptr, *d_vs_ = nullptr;  // int8 caches: one scale per 32 values (else null)
    void *d_span_ws_ = nullptr, *d_dec_ = nullptr, *d_dec_act_ = nullptr;
    // buffers of the last span call's last chunk (fish_hip_span_inspect)
    SpanBufs last_bufs_{};
    int last_tok_ = 0, last_pos0_ = 0;
    // decode graph over the fixed decode buffers (built at the first one-token call)
    hipGraphExec_t dec_exec_ = nullptr;
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

int fish_hip_quantize_for(uint32_t type, const float* x, int n_tok, int n_in, void* act, void* stream) {
    if (!x || !act || n_tok <= 0 || n_in <= 0 || n_in % 32) return fail(FISH_HIP_ERR_ARG, "quantize_for: bad arguments");
    const WeightLayout L = weight_layout(type, n_in, 1);
    if (!L.total || !int8_type(type)) return fail(FISH_HIP_ERR_ARG, "quantize_for: not an int8-path type");
    const hipError_t e =
        launch_quantize(x, n_tok, n_in, n_in, act, nullptr, nullptr, as_stream(stream), planes_of(L, n_tok));
    return e == hipSuccess ? 0 : hip_fail(e, "quantize_for");
}

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
                            planes_of(L[0], n_tok));
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

int fish_hip_backend_moe_ffn(const void* key_gate, const void* key_up, const void* key_down, const void* key_router,
                             const float* x, const float* logits, int n_tok, int n_embd, int n_ff, int n_expert, int k,
                             int norm, float* out) {
    return HipBackend::instance().moe_ffn_host(key_gate, key_up, key_down, key_router, x, logits, n_tok, n_embd, n_ff,
                                               n_expert, k, norm, out)
               ? 1
               : 0;
}

int fish_hip_span_prepare(const fish_hip_span_params* p) {
    return p && HipBackend::instance().span_prepare(*p) ? 1 : 0;
}
int fish_hip_span_forward(float* x, int n_tok, int pos0) {
    return HipBackend::instance().span_forward(x, n_tok, pos0) ? 1 : 0;
}
int fish_hip_span_inspect(int part, int layer, int pos0, int n, float* out, uint64_t n_floats) {
    return HipBackend::instance().span_inspect(part, layer, pos0, n, out, n_floats) ? 1 : 0;
}
int fish_hip_span_last_tokens(void) { return HipBackend::instance().span_last_tokens(); }
void fish_hip_span_kv_truncate(int n_past) { (void)n_past; }  // positions >= n_past are rewritten before use
void fish_hip_span_release(void) { HipBackend::instance().span_release(); }

int fish_hip_backend_matmul_group(const void* const* keys, int n, const float* x, int n_tok, int n_in,
                                  const int* n_outs, float* const* ys) {
    return HipBackend::instance().matmul_group(keys, n, x, n_tok, n_in, n_outs, ys) ? 1 : 0;
}

}  // extern "C"
