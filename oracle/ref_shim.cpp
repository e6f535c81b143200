// C entry points over the reference's own CPU path -- TEST INFRASTRUCTURE ONLY.
//
// Built by oracle/Makefile together with the reference's sources where they
// lie (model/fish/src/{gguf,quant,quantize,quant_x86,ops,threadpool,specs}.cpp)
// into oracle/_ref/libfishref.so. Used to write golden fixtures and as the
// timed CPU baseline ("kind": "reference"). This file only calls the
// reference's public functions; the MoE composition follows the order of
// model/fish/src/model.cpp:1523-1580 because LlamaModel::moe_ffn is a member
// of a model object that needs a GGUF file to exist.
#include <fish/ops.h>
#include <fish/quant.h>
#include <fish/threadpool.h>

#include <algorithm>
#include <cstring>
#include <utility>
#include <vector>

using namespace fish;

namespace {
const QuantKernels& table(int scalar) { return scalar ? scalar_kernels() : quant_kernels(); }
}  // namespace

extern "C" {

const char* ref_kernel_name(void) { return quant_kernels().name; }
int ref_threads(void) { return ThreadPool::instance().active_threads(); }

float ref_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h); }
uint16_t ref_fp32_to_fp16(float f) { return fp32_to_fp16(f); }

void ref_quantize_acts(const float* x, uint64_t n, void* out, int scalar) {
    table(scalar).quantize(x, n, static_cast<Q8Act*>(out));
}
void ref_quantize_acts_k(const float* x, uint64_t n, void* out, int scalar) {
    table(scalar).quantize_k(x, n, static_cast<Q8ActK*>(out));
}

int ref_dequant_row(uint32_t type, const void* src, float* dst, uint64_t n) {
    return dequant_row(static_cast<GgmlType>(type), src, dst, n) ? 1 : 0;
}

int ref_quantize_row(uint32_t type, const float* x, void* dst, uint64_t n) {
    return quantize_row(static_cast<GgmlType>(type), x, dst, n) ? 1 : 0;
}

// One weight row times int8 activations through the installed (AVX2) or the
// scalar table.
float ref_vec_dot_q8(uint32_t type, const void* row, const void* acts, uint64_t n, int scalar) {
    const QuantKernels& k = table(scalar);
    const auto* a32 = static_cast<const Q8Act*>(acts);
    const auto* a256 = static_cast<const Q8ActK*>(acts);
    switch (static_cast<GgmlType>(type)) {
        case GgmlType::Q8_0: return k.q8_0_q8(row, a32, n);
        case GgmlType::Q4_0: return k.q4_0_q8(row, a32, n);
        case GgmlType::Q4_K: return k.q4_K_q8k(row, a256, n);
        case GgmlType::Q5_K: return k.q5_K_q8k(row, a256, n);
        case GgmlType::Q6_K: return k.q6_K_q8k(row, a256, n);
        default: return 0.0f;
    }
}

// FISH's whole int8 matmul from f32 input: ActBatch::quantize, then the
// threaded matmul_batch (ops.cpp:158-216).
void ref_matmul_f32(uint32_t type, const void* w, const float* x, int n_tok, int n_in, int n_out, float* y) {
    ActBatch acts;
    acts.quantize(x, n_tok, n_in);
    matmul_batch(static_cast<GgmlType>(type), w, x, &acts, n_tok, n_in, n_out, y);
}

// matmul_batch on activations quantised beforehand (ActBatch's two layouts as
// packed bytes; acts256 may be null when n_in % 256 != 0).
void ref_matmul_acts(uint32_t type, const void* w, const void* acts32, const void* acts256,
                     int n_tok, int n_in, int n_out, float* y) {
    ActBatch acts;
    acts.n_tok = n_tok;
    acts.n_in = n_in;
    acts.q32.resize(static_cast<size_t>(n_tok) * (n_in / kQ8ActBlock));
    std::memcpy(acts.q32.data(), acts32, acts.q32.size() * sizeof(Q8Act));
    if (acts256 && n_in % kQ8ActKBlock == 0) {
        acts.q256.resize(static_cast<size_t>(n_tok) * (n_in / kQ8ActKBlock));
        std::memcpy(acts.q256.data(), acts256, acts.q256.size() * sizeof(Q8ActK));
    }
    matmul_batch(static_cast<GgmlType>(type), w, nullptr, &acts, n_tok, n_in, n_out, y);
}

// Expert FFN with given router logits, composed from FISH's primitives in the
// order of model.cpp:1528-1580 (softmax, partial_sort top-k, renormalise;
// experts ascending, tokens ascending; gate, up, silu*up, requantise, down,
// out[t] += w * down). gate/up: [NE][F rows of E], down: [NE][E rows of F].
void ref_moe_ffn(const float* x, const float* logits, int n_tok, int E, int F, int NE, int K, int norm,
                 uint32_t t_gate, const void* w_gate, uint32_t t_up, const void* w_up,
                 uint32_t t_down, const void* w_down, float* out, int* sel_out, float* wsel_out) {
    const auto tg = static_cast<GgmlType>(t_gate), tu = static_cast<GgmlType>(t_up), td = static_cast<GgmlType>(t_down);
    std::vector<int> sel(static_cast<size_t>(n_tok) * K);
    std::vector<float> wsel(static_cast<size_t>(n_tok) * K);
    std::vector<std::pair<float, int>> scores(static_cast<size_t>(NE));
    std::vector<float> lg(static_cast<size_t>(NE));
    for (int t = 0; t < n_tok; ++t) {
        std::memcpy(lg.data(), logits + static_cast<size_t>(t) * NE, sizeof(float) * NE);
        softmax_inplace(lg.data(), NE);
        for (int e = 0; e < NE; ++e) scores[static_cast<size_t>(e)] = {lg[static_cast<size_t>(e)], e};
        std::partial_sort(scores.begin(), scores.begin() + K, scores.end(),
                          [](const auto& a, const auto& b) { return a.first > b.first; });
        float sum = 0.0f;
        for (int k = 0; k < K; ++k) {
            sel[static_cast<size_t>(t) * K + k] = scores[static_cast<size_t>(k)].second;
            wsel[static_cast<size_t>(t) * K + k] = scores[static_cast<size_t>(k)].first;
            sum += scores[static_cast<size_t>(k)].first;
        }
        if (norm && sum > 0.0f)
            for (int k = 0; k < K; ++k) wsel[static_cast<size_t>(t) * K + k] /= sum;
    }
    if (sel_out) std::memcpy(sel_out, sel.data(), sel.size() * sizeof(int));
    if (wsel_out) std::memcpy(wsel_out, wsel.data(), wsel.size() * sizeof(float));
    std::fill(out, out + static_cast<size_t>(n_tok) * E, 0.0f);

    const size_t gsz = ggml_row_size(tg, static_cast<uint64_t>(E)) * static_cast<size_t>(F);
    const size_t usz = ggml_row_size(tu, static_cast<uint64_t>(E)) * static_cast<size_t>(F);
    const size_t dsz = ggml_row_size(td, static_cast<uint64_t>(F)) * static_cast<size_t>(E);
    std::vector<int> toks;
    std::vector<float> wts, xin, g, u, dn;
    ActBatch xq, hq;
    for (int e = 0; e < NE; ++e) {
        toks.clear();
        wts.clear();
        for (int t = 0; t < n_tok; ++t)
            for (int k = 0; k < K; ++k)
                if (sel[static_cast<size_t>(t) * K + k] == e) {
                    toks.push_back(t);
                    wts.push_back(wsel[static_cast<size_t>(t) * K + k]);
                }
        if (toks.empty()) continue;
        const int cnt = static_cast<int>(toks.size());
        xin.resize(static_cast<size_t>(cnt) * E);
        g.resize(static_cast<size_t>(cnt) * F);
        u.resize(static_cast<size_t>(cnt) * F);
        dn.resize(static_cast<size_t>(cnt) * E);
        for (int j = 0; j < cnt; ++j)
            std::memcpy(xin.data() + static_cast<size_t>(j) * E, x + static_cast<size_t>(toks[static_cast<size_t>(j)]) * E,
                        sizeof(float) * E);
        xq.quantize(xin.data(), cnt, E);
        matmul_batch(tg, static_cast<const uint8_t*>(w_gate) + gsz * e, xin.data(), &xq, cnt, E, F, g.data());
        matmul_batch(tu, static_cast<const uint8_t*>(w_up) + usz * e, xin.data(), &xq, cnt, E, F, u.data());
        for (int j = 0; j < cnt; ++j) {
            float* gr = g.data() + static_cast<size_t>(j) * F;
            const float* ur = u.data() + static_cast<size_t>(j) * F;
            silu_inplace(gr, F);
            for (int i = 0; i < F; ++i) gr[i] *= ur[i];
        }
        hq.quantize(g.data(), cnt, F);
        matmul_batch(td, static_cast<const uint8_t*>(w_down) + dsz * e, g.data(), &hq, cnt, F, E, dn.data());
        for (int j = 0; j < cnt; ++j) {
            float* o = out + static_cast<size_t>(toks[static_cast<size_t>(j)]) * E;
            const float* d = dn.data() + static_cast<size_t>(j) * E;
            const float w = wts[static_cast<size_t>(j)];
            for (int i = 0; i < E; ++i) o[i] += w * d[i];
        }
    }
}

}  // extern "C"
