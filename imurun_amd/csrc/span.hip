// The non-matmul steps of a dense transformer layer, for layer spans: a range
// of layers run entirely on the device per forward call (the ComputeBackend
// span contract, backend.h:89-162), with the projections on the matmul kernels.
//
// Each kernel restates FISH's CPU step for one layer (model.cpp:1650-1790):
//   rmsnorm      ops.cpp:18-23   (double sum of squares, f32 scale, x * scale * w)
//   q/k/v prep   the projection biases (add_bias, model.cpp:1704-1706), the
//                Qwen-3 per-head q/k RMS norms (model.cpp:1712-1719), RoPE
//                (ops.cpp:126-152, neox or adjacent pairs) and the KV-cache
//                store (model.cpp:1721-1729), in one kernel
//   attention    ops.cpp:303-357 (causal, GQA head groups, max-subtracted exp,
//                softmax-weighted sum of V; a decode token split over position
//                chunks, more tokens in one pass per (token, head))
//   silu * up    ops.cpp:25-30, model.cpp:1504-1508
//   residual add model.cpp:1772-1776, :1797-1801, with the o bias
//                (model.cpp:1749) (fused into the next rmsnorm)
// The KV cache holds f16 K and V (4 bytes per position and K+V element), as
// FISH's own device span does (vulkan_backend.cpp:1650) and as its planner
// budgets (model.cpp:1318-1320); values round to nearest even when stored.
// The file is compiled without floating-point contraction, so every
// expression rounds as FISH's baseline x86-64 build does; exp is the device's
// expf, within a few ulp of the C library's.
#include "common.h"
#include "kernels.h"
#include "qact.h"

namespace fishhip {

namespace {

constexpr int kTh = 256;

constexpr int kNormTh = 1024;

__device__ __forceinline__ double block_sum_d(double v, double* red) {
    const int tid = threadIdx.x;
    red[tid] = v;
    __syncthreads();
    for (int s = kNormTh / 2; s > 0; s >>= 1) {
        if (tid < s) red[tid] += red[tid + s];
        __syncthreads();
    }
    const double r = red[0];
    __syncthreads();
    return r;
}

__device__ __forceinline__ float block_reduce_f(float v, float* red, bool is_max) {
    const int tid = threadIdx.x;
    red[tid] = v;
    __syncthreads();
    for (int s = kTh / 2; s > 0; s >>= 1) {
        if (tid < s) red[tid] = is_max ? fmaxf(red[tid], red[tid + s]) : red[tid] + red[tid + s];
        __syncthreads();
    }
    const float r = red[0];
    __syncthreads();
    return r;
}

// one workgroup of kNormTh threads per token; with y, first x += y (the
// residual add, written back to x; with b, y + b is added: the projection's
// bias, then the residual); with b and no y, x += b (a projection's bias
// before its own norm, model.cpp:1756-1760); then out = rmsnorm(x), which
// may be x itself
__global__ __launch_bounds__(kNormTh) void rmsnorm_kernel(float* __restrict__ x, const float* __restrict__ y,
                                                          const float* __restrict__ b, const float* __restrict__ w,
                                                          float* __restrict__ out, int n, float eps) {
    __shared__ double red[kNormTh];
    float* xr = x + size_t(blockIdx.x) * n;
    const float* yr = y ? y + size_t(blockIdx.x) * n : nullptr;
    float* orow = out + size_t(blockIdx.x) * n;
    double s = 0.0;
#pragma unroll 4
    for (int i = threadIdx.x; i < n; i += kNormTh) {
        float v = xr[i];
        if (yr) {
            v = v + (b ? yr[i] + b[i] : yr[i]);
            xr[i] = v;
        } else if (b) {
            v = v + b[i];
            xr[i] = v;
        }
        s += double(v) * double(v);
    }
    const double sum = block_sum_d(s, red);
    const float scale = 1.0f / sqrtf(float(sum / n) + eps);
    for (int i = threadIdx.x; i < n; i += kNormTh) orow[i] = xr[i] * scale * w[i];
}

// One head of a token, thread d owning element d (D <= kTh): its inputs, loaded
// first (head_load), then prepared by the whole workgroup (head_prep): value +
// bias, the per-head RMS norm when given (the rmsnorm of ops.cpp:18-23 over the
// head's D values, the squares summed in double over a fixed tree), then RoPE
// (ops.cpp:126-152: pairs (i, i + half) with NEOX, else (2i, 2i + 1); elements
// past 2 half unchanged). The loads and the arithmetic are apart so that a
// caller can issue other loads in between without waiting for them.
struct HeadIn {
    float x, b, w, c, s;  // value, bias, norm weight, RoPE cos / sin of the element's pair
};

__device__ __forceinline__ HeadIn head_load(const float* __restrict__ src_row, const float* __restrict__ bias,
                                            const float* __restrict__ nw, int head, int D, int half, int neox,
                                            const float* __restrict__ c, const float* __restrict__ s) {
    const int d = threadIdx.x;
    HeadIn r{0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (d < D) {
        r.x = src_row[head * D + d];
        if (bias) r.b = bias[head * D + d];
        if (nw) r.w = nw[d];
        if (d < 2 * half) {
            const int i = neox ? (d < half ? d : d - half) : d >> 1;
            r.c = c[i];
            r.s = s[i];
        }
    }
    return r;
}

// Element d of the prepared head (d < D). row and red are LDS of kTh entries;
// every thread of the workgroup calls this.
__device__ __forceinline__ float head_prep(const HeadIn& in, bool has_bias, bool has_norm, int D, int half, int neox,
                                           float eps, float* row, double* red) {
    const int d = threadIdx.x;
    float val = 0.0f;
    if (d < D) val = has_bias ? in.x + in.b : in.x;
    if (has_norm) {  // uniform over the workgroup
        red[d] = d < D ? double(val) * double(val) : 0.0;
        __syncthreads();
        for (int st = kTh / 2; st > 0; st >>= 1) {
            if (d < st) red[d] += red[d + st];
            __syncthreads();
        }
        const float scale = 1.0f / sqrtf(float(red[0] / D) + eps);
        if (d < D) val = val * scale * in.w;
    }
    row[d] = val;
    __syncthreads();
    float r = 0.0f;
    if (d < D) {
        if (d >= 2 * half) {
            r = row[d];
        } else if (neox) {
            const int i = d < half ? d : d - half;
            const float x0 = row[i], x1 = row[i + half];
            r = d < half ? x0 * in.c - x1 * in.s : x0 * in.s + x1 * in.c;
        } else {
            const int i = d >> 1;
            const float x0 = row[2 * i], x1 = row[2 * i + 1];
            r = (d & 1) ? x0 * in.s + x1 * in.c : x0 * in.c - x1 * in.s;
        }
    }
    __syncthreads();  // row is free again on return
    return r;
}

// The int8 code of element x of a 32-value block held by the 32 lanes of one
// half wavefront (all of them active), and the block's d = amax / 127: the
// activation quantizer's arithmetic (qact.h).
__device__ __forceinline__ int kv_code(float x, float& d) {
    float a = fabsf(x);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off));
    d = block_d(a);
    return code(x, block_id(d));
}

// Element x of a K or V row into the cache at element index `at`, by the thread
// that owns element at % D of the head (thread index == element index within
// the head): f16, or (Q8) the int8 code plus the block's d from the block's
// first thread. Every thread of the 32-value block calls this.
template <bool Q8>
__device__ __forceinline__ void kv_store(const KvCache& c, size_t at, float x) {
    if constexpr (Q8) {
        float d;
        const int q = kv_code(x, d);
        static_cast<int8_t*>(c.c)[at] = int8_t(q);
        if ((threadIdx.x & 31) == 0) c.d[at >> 5] = d;
    } else {
        static_cast<_Float16*>(c.c)[at] = _Float16(x);
    }
}

// One workgroup per (token t, head): q heads first, then k heads (whose
// workgroup also stores the v head of the same index); prep_head, then q ->
// q_out, k and v -> cache rows of position pos0 + t.
template <bool Q8>
__global__ __launch_bounds__(kTh) void qkv_prep_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                       const float* __restrict__ v, SpanVecs vecs,
                                                       float* __restrict__ q_out, KvCache kc, KvCache vc, int Q,
                                                       int KV, int D, int half,
                                                       int neox, float eps, int pos0, const int* __restrict__ pos_dev,
                                                       const float* __restrict__ cosv,
                                                       const float* __restrict__ sinv) {
    __shared__ float row[kTh];
    __shared__ double red[kTh];
    if (pos_dev) pos0 = *pos_dev;
    const int t = blockIdx.x, hh = blockIdx.y, pos = pos0 + t, H = Q / D, d = threadIdx.x;
    const bool is_q = hh < H;
    const int head = is_q ? hh : hh - H;
    const float* src = is_q ? q + size_t(t) * Q : k + size_t(t) * KV;
    const float* bias = is_q ? vecs.bias_q : vecs.bias_k;
    const float* nw = is_q ? vecs.q_norm : vecs.k_norm;
    const HeadIn in = head_load(src, bias, nw, head, D, half, neox, cosv + size_t(pos) * half,
                                sinv + size_t(pos) * half);
    const float r = head_prep(in, bias != nullptr, nw != nullptr, D, half, neox, eps, row, red);
    if (d >= D) return;
    if (is_q) {
        q_out[size_t(t) * Q + head * D + d] = r;
    } else {
        const size_t at = size_t(pos) * KV + head * D + d;
        kv_store<Q8>(kc, at, r);
        float vv = v[size_t(t) * KV + head * D + d];
        if (vecs.bias_v) vv = vv + vecs.bias_v[head * D + d];
        kv_store<Q8>(vc, at, vv);
    }
}

// Attention in two steps, split over the positions so that one decode token
// still spreads over many workgroups (flash-decoding):
//   attn_part_kernel: one workgroup (four wavefronts) per (token, head, chunk
//     of kCh positions). Lanes run over the head's D values (DL per lane), so
//     each K or V row is one coalesced load; every wavefront issues the loads
//     of its kCh / 4 positions before using them. It writes the chunk's max
//     score m, its sum l of exp(s - m), and o = sum exp(s - m) v.
//   attn_combine_kernel: one workgroup per (token, head): M = max m,
//     L = sum l exp(m - M), out = (sum o exp(m - M)) * (1 / L).
// Chunks that start past the token's position, or end before a sliding window's
// first position, hold m = -inf, l = 0, o = 0.
// Mathematically FISH's single-pass softmax (ops.cpp:331-350); the rounding
// order differs. Needs D <= 256.
constexpr int kCh = 64;

// The f16 K / V caches are read as element pairs, one dword per lane (2-byte
// loads become half-register loads that the compiler waits on one by one):
// lane l owns the pairs 2 (l + 64 j), j < NP, of a head of D (even) values.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float2 f16x2(uint32_t u) {
    const half2_t h = __builtin_bit_cast(half2_t, u);
    return make_float2(float(h.x), float(h.y));
}

// A lane's pair of elements (e, e + 1) of one cache row as loaded: the f16 pair,
// or (Q8) the two int8 codes in the low 16 bits and their block's d.
struct KvRaw {
    uint32_t w;
    float d;
};
template <bool Q8>
__device__ __forceinline__ KvRaw kv_raw(const KvCache& c, size_t elem) {
    KvRaw r;
    if constexpr (Q8) {
        r.w = *reinterpret_cast<const uint16_t*>(static_cast<const int8_t*>(c.c) + elem);
        r.d = c.d[elem >> 5];
    } else {
        r.w = *reinterpret_cast<const uint32_t*>(static_cast<const _Float16*>(c.c) + elem);
        r.d = 0.0f;
    }
    return r;
}
template <bool Q8>
__device__ __forceinline__ float2 kv_val(const KvRaw& r) {
    if constexpr (Q8)
        return make_float2(float(int8_t(r.w & 0xFFu)) * r.d, float(int8_t((r.w >> 8) & 0xFFu)) * r.d);
    else
        return f16x2(r.w);
}

// The raw pair (e, e + 1) of a row held in LDS: f16 pairs as dwords, or int8
// codes with one d per 32 values.
template <bool Q8>
__device__ __forceinline__ KvRaw lds_raw(const uint32_t* w, const float* d, int e) {
    if constexpr (Q8)
        return KvRaw{uint32_t(reinterpret_cast<const uint16_t*>(w)[e >> 1]), d[e >> 5]};
    else
        return KvRaw{w[e >> 1], 0.0f};
}

// A position's score: dot * scale, then Gemma-2's soft cap c tanh(s / c) when c > 0
// (ops.cpp:334-335)
__device__ __forceinline__ float score(float dot, float scale, float softcap) {
    const float s = dot * scale;
    return softcap > 0.0f ? softcap * tanhf(s / softcap) : s;
}

// PREP (one token): the workgroup prepares its q head from the raw projection
// itself (prep_head, as qkv_prep_kernel), and the workgroups of the chunk that
// holds the token's position also prepare that position's k and v rows (the
// same values the cache gets) and use them in place of the cache rows; of
// those, the first q head of each KV group stores the rows into the caches and
// every one stores its q head into q_out. No separate preparation launch.
struct AttnPrep {
    const float *q, *k, *v;  // raw projections of the token
    SpanVecs vecs;
    float* q_out;
    KvCache kc, vc;          // the caches, for the position's rows
    const float *cosv, *sinv;
    int half, neox;
    float eps;
};

template <int NP, bool PREP, bool Q8>
__global__ __launch_bounds__(kTh) void attn_part_kernel(const float* __restrict__ q, KvCache kc, KvCache vc,
                                                        float* __restrict__ part,
                                                        int S, int H, int HKV, int D, int pos0,
                                                        const int* __restrict__ pos_dev, float scale, float softcap,
                                                        int window, AttnPrep P) {
    constexpr int PB = kCh / 4;
    __shared__ float s_e[kCh];
    __shared__ float s_o[4][128 * NP];
    __shared__ float s_ml[2];
    // PREP: the prepared q head, the position's k / v rows (f16 pairs, or int8 codes
    // and their d per 32), scratch
    __shared__ float s_q[PREP ? 128 * NP : 1];
    __shared__ uint32_t s_kn[PREP ? 64 * NP : 1], s_vn[PREP ? 64 * NP : 1];
    __shared__ float s_knd[PREP && Q8 ? 4 * NP : 1], s_vnd[PREP && Q8 ? 4 * NP : 1];
    __shared__ float s_row[PREP ? kTh : 1];
    __shared__ double s_red[PREP ? kTh : 1];
    if (pos_dev) pos0 = *pos_dev;
    const int item = blockIdx.x, chunk = blockIdx.y, t = item / H, h = item % H;
    const int pos = pos0 + t, kvh = h / (H / HKV), KV = HKV * D, Q = H * D;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int j0 = chunk * kCh;
    // a sliding window attends over positions jlo..pos (ops.cpp:327-328)
    const int jlo = window > 0 ? max(0, pos - window + 1) : 0;
    float* pp = part + (size_t(item) * S + chunk) * size_t(D + 2);
    if (j0 > pos || j0 + kCh <= jlo) {  // uniform over the workgroup
        for (int d = tid; d < D; d += kTh) pp[d] = 0.0f;
        if (tid == 0) {
            pp[D] = -INFINITY;
            pp[D + 1] = 0.0f;
        }
        return;
    }
    const int jn = min(pos, j0 + kCh - 1);
    const size_t hoff = size_t(kvh) * D;  // the KV head's first element in a cache row

    // PREP: the inputs of the q head (and of the position's k / v rows) are loaded
    // first, then the cache rows; the preparation waits only for its own loads
    const bool own = PREP && jn == pos;  // this chunk holds the position (uniform)
    HeadIn qin{}, kin{};
    float v_x = 0.0f, v_b = 0.0f;
    if constexpr (PREP) {
        const float* c = P.cosv + size_t(pos) * P.half;
        const float* sn = P.sinv + size_t(pos) * P.half;
        qin = head_load(P.q + size_t(t) * Q, P.vecs.bias_q, P.vecs.q_norm, h, D, P.half, P.neox, c, sn);
        if (own) {
            kin = head_load(P.k + size_t(t) * KV, P.vecs.bias_k, P.vecs.k_norm, kvh, D, P.half, P.neox, c, sn);
            if (tid < D) {
                v_x = P.v[size_t(t) * KV + size_t(kvh) * D + tid];
                if (P.vecs.bias_v) v_b = P.vecs.bias_v[size_t(kvh) * D + tid];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    // scores of positions j0 + w + 4 b; their V rows are loaded with the K rows, so the
    // chunk waits for the cache once
    KvRaw kv[PB][NP], vv[PB][NP];
#pragma unroll
    for (int b = 0; b < PB; ++b) {
        const size_t rb = size_t(min(j0 + w + 4 * b, jn)) * KV + hoff;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int e = 2 * (lane + 64 * i);
            kv[b][i] = e < D ? kv_raw<Q8>(kc, rb + e) : KvRaw{0u, 0.0f};
        }
    }
#pragma unroll
    for (int b = 0; b < PB; ++b) {
        const size_t rb = size_t(min(j0 + w + 4 * b, jn)) * KV + hoff;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int e = 2 * (lane + 64 * i);
            vv[b][i] = e < D ? kv_raw<Q8>(vc, rb + e) : KvRaw{0u, 0.0f};
        }
    }
    float2 qv[NP];
    if constexpr (PREP) {
        __builtin_amdgcn_sched_barrier(0);
        const float r = head_prep(qin, P.vecs.bias_q != nullptr, P.vecs.q_norm != nullptr, D, P.half, P.neox, P.eps,
                                  s_row, s_red);
        if (tid < D) {
            s_q[tid] = r;
            if (own) P.q_out[size_t(t) * Q + size_t(h) * D + tid] = r;
        }
        if (own) {
            const float rk = head_prep(kin, P.vecs.bias_k != nullptr, P.vecs.k_norm != nullptr, D, P.half, P.neox,
                                       P.eps, s_row, s_red);
            if (tid < D) {  // whole 32-value blocks (D % 32 == 0 for Q8)
                const float vx = P.vecs.bias_v ? v_x + v_b : v_x;
                const size_t at = size_t(pos) * KV + size_t(kvh) * D + tid;
                if constexpr (Q8) {
                    float dk, dv;
                    const int qk = kv_code(rk, dk), qv8 = kv_code(vx, dv);
                    reinterpret_cast<int8_t*>(s_kn)[tid] = int8_t(qk);
                    reinterpret_cast<int8_t*>(s_vn)[tid] = int8_t(qv8);
                    if ((tid & 31) == 0) {
                        s_knd[tid >> 5] = dk;
                        s_vnd[tid >> 5] = dv;
                    }
                    if (h % (H / HKV) == 0) {
                        static_cast<int8_t*>(P.kc.c)[at] = int8_t(qk);
                        static_cast<int8_t*>(P.vc.c)[at] = int8_t(qv8);
                        if ((tid & 31) == 0) {
                            P.kc.d[at >> 5] = dk;
                            P.vc.d[at >> 5] = dv;
                        }
                    }
                } else {
                    const _Float16 k16 = _Float16(rk), v16 = _Float16(vx);
                    reinterpret_cast<_Float16*>(s_kn)[tid] = k16;
                    reinterpret_cast<_Float16*>(s_vn)[tid] = v16;
                    if (h % (H / HKV) == 0) {
                        static_cast<_Float16*>(P.kc.c)[at] = k16;
                        static_cast<_Float16*>(P.vc.c)[at] = v16;
                    }
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int e = 2 * (lane + 64 * i);
            qv[i] = e < D ? make_float2(s_q[e], s_q[e + 1]) : make_float2(0.f, 0.f);
        }
        if (own) {
#pragma unroll
            for (int b = 0; b < PB; ++b)
                if (min(j0 + w + 4 * b, jn) == pos)
#pragma unroll
                    for (int i = 0; i < NP; ++i)
                        if (2 * (lane + 64 * i) < D) kv[b][i] = lds_raw<Q8>(s_kn, s_knd, 2 * (lane + 64 * i));
        }
    } else {
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int e = 2 * (lane + 64 * i);
            qv[i] = e < D ? *reinterpret_cast<const float2*>(q + size_t(t) * Q + size_t(h) * D + e)
                          : make_float2(0.f, 0.f);
        }
    }
#pragma unroll
    for (int b = 0; b < PB; ++b) {
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const float2 k2 = kv_val<Q8>(kv[b][i]);
            sum += qv[i].x * k2.x;
            sum += qv[i].y * k2.y;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
        if (lane == 0) {
            const int j = j0 + w + 4 * b;
            s_e[w + 4 * b] = (j <= jn && j >= jlo) ? score(sum, scale, softcap) : -INFINITY;
        }
    }
    __syncthreads();
    if (w == 0) {
        float m = s_e[lane];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        const float e = (lane <= jn - j0 && j0 + lane >= jlo) ? expf(s_e[lane] - m) : 0.0f;
        float l = e;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
        s_e[lane] = e;
        if (lane == 0) {
            s_ml[0] = m;
            s_ml[1] = l;
        }
    }
    __syncthreads();
    if constexpr (PREP) {
        if (own) {
#pragma unroll
            for (int b = 0; b < PB; ++b)
                if (min(j0 + w + 4 * b, jn) == pos)
#pragma unroll
                    for (int i = 0; i < NP; ++i)
                        if (2 * (lane + 64 * i) < D) vv[b][i] = lds_raw<Q8>(s_vn, s_vnd, 2 * (lane + 64 * i));
        }
    }
    float2 acc[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) acc[i] = make_float2(0.f, 0.f);
#pragma unroll
    for (int b = 0; b < PB; ++b) {
        const float e = s_e[w + 4 * b];  // 0 past jn
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const float2 v2 = kv_val<Q8>(vv[b][i]);
            acc[i].x += e * v2.x;
            acc[i].y += e * v2.y;
        }
    }
#pragma unroll
    for (int i = 0; i < NP; ++i) *reinterpret_cast<float2*>(&s_o[w][2 * (lane + 64 * i)]) = acc[i];
    __syncthreads();
    for (int d = tid; d < D; d += kTh) pp[d] = (s_o[0][d] + s_o[1][d]) + (s_o[2][d] + s_o[3][d]);
    if (tid == 0) {
        pp[D] = s_ml[0];
        pp[D + 1] = s_ml[1];
    }
}

// Chunks past the token's position hold nothing and are not read. Every load of
// the first kTh chunks' (m, l) and of the first kCombineRegs chunks' o is issued
// before the first wait, so a decode token's combine waits on memory once.
constexpr int kCombineRegs = 16;
__global__ __launch_bounds__(kTh) void attn_combine_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                           int S, int H, int D, int pos0,
                                                           const int* __restrict__ pos_dev) {
    __shared__ float s_red[2][kTh / 64];
    __shared__ float s_w[kTh];
    if (pos_dev) pos0 = *pos_dev;
    const int item = blockIdx.x, t = item / H, h = item % H, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int sv = min(S, (pos0 + t) / kCh + 1);  // chunks holding positions up to the token's
    const size_t st = size_t(D + 2);
    const float* pp = part + size_t(item) * S * st;
    float o_r[kCombineRegs];
#pragma unroll
    for (int c = 0; c < kCombineRegs; ++c) o_r[c] = (tid < D && c < sv) ? pp[size_t(c) * st + tid] : 0.0f;
    const float mc = tid < sv ? pp[size_t(tid) * st + D] : -INFINITY;
    const float lc = tid < sv ? pp[size_t(tid) * st + D + 1] : 0.0f;
    float m = mc;
    for (int c = tid + kTh; c < sv; c += kTh) m = fmaxf(m, pp[size_t(c) * st + D]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane == 0) s_red[0][wv] = m;
    __syncthreads();
    float M = s_red[0][0];
#pragma unroll
    for (int i = 1; i < kTh / 64; ++i) M = fmaxf(M, s_red[0][i]);
    // chunk weights exp(m - M); an empty chunk (m = -inf) weighs 0
    const float wc = mc == -INFINITY ? 0.0f : expf(mc - M);
    s_w[tid] = wc;
    float l = lc * wc;
    for (int c = tid + kTh; c < sv; c += kTh) {
        const float mx = pp[size_t(c) * st + D];
        l += pp[size_t(c) * st + D + 1] * (mx == -INFINITY ? 0.0f : expf(mx - M));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
    if (lane == 0) s_red[1][wv] = l;
    __syncthreads();
    float L = 0.0f;
#pragma unroll
    for (int i = 0; i < kTh / 64; ++i) L += s_red[1][i];
    if (tid >= D) return;
    float o = 0.0f;
#pragma unroll
    for (int c = 0; c < kCombineRegs; ++c) o += o_r[c] * s_w[c];
    for (int c = kCombineRegs; c < min(sv, kTh); ++c) o += pp[size_t(c) * st + tid] * s_w[c];
    for (int c = kTh; c < sv; ++c) {
        const float mx = pp[size_t(c) * st + D];
        o += pp[size_t(c) * st + tid] * (mx == -INFINITY ? 0.0f : expf(mx - M));
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    out[size_t(t) * H * D + size_t(h) * D + tid] = o * inv;
}

// Attention of more tokens (prefill): one workgroup per (token, head) walks
// the chunks of kCh positions up to the token's own, each chunk as in
// attn_part_kernel, and merges them into a running (max, sum, output) --
// no partials in memory, so the scratch does not grow with tokens x context.
template <int NP, bool Q8>
__global__ __launch_bounds__(kTh) void attn_full_kernel(const float* __restrict__ q, KvCache kc, KvCache vc,
                                                        float* __restrict__ out,
                                                        int H, int HKV, int D, int pos0,
                                                        const int* __restrict__ pos_dev, float scale, float softcap,
                                                        int window) {
    constexpr int PB = kCh / 4;
    __shared__ float s_e[kCh];
    __shared__ float s_o[4][128 * NP];
    __shared__ float s_ml[2];
    if (pos_dev) pos0 = *pos_dev;
    const int item = blockIdx.x, t = item / H, h = item % H;
    const int pos = pos0 + t, kvh = h / (H / HKV), KV = HKV * D, Q = H * D;
    const int jlo = window > 0 ? max(0, pos - window + 1) : 0;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    float2 qv[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int e = 2 * (lane + 64 * i);
        qv[i] = e < D ? *reinterpret_cast<const float2*>(q + size_t(t) * Q + size_t(h) * D + e) : make_float2(0.f, 0.f);
    }
    const size_t hoff = size_t(kvh) * D;
    float o_run = 0.0f, m_run = -INFINITY, l_run = 0.0f;
    for (int j0 = jlo / kCh * kCh; j0 <= pos; j0 += kCh) {
        const int jn = min(pos, j0 + kCh - 1);
        KvRaw kv[PB][NP];
#pragma unroll
        for (int b = 0; b < PB; ++b) {
            const size_t rb = size_t(min(j0 + w + 4 * b, jn)) * KV + hoff;
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int e = 2 * (lane + 64 * i);
                kv[b][i] = e < D ? kv_raw<Q8>(kc, rb + e) : KvRaw{0u, 0.0f};
            }
        }
        // V rows of the chunk in flight while the scores are formed
        KvRaw vv[PB][NP];
#pragma unroll
        for (int b = 0; b < PB; ++b) {
            const size_t rb = size_t(min(j0 + w + 4 * b, jn)) * KV + hoff;
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int e = 2 * (lane + 64 * i);
                vv[b][i] = e < D ? kv_raw<Q8>(vc, rb + e) : KvRaw{0u, 0.0f};
            }
        }
#pragma unroll
        for (int b = 0; b < PB; ++b) {
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const float2 k2 = kv_val<Q8>(kv[b][i]);
                sum += qv[i].x * k2.x;
                sum += qv[i].y * k2.y;
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
            if (lane == 0) {
                const int j = j0 + w + 4 * b;
                s_e[w + 4 * b] = (j <= jn && j >= jlo) ? score(sum, scale, softcap) : -INFINITY;
            }
        }
        __syncthreads();
        if (w == 0) {
            float m = s_e[lane];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
            const float e = (lane <= jn - j0 && j0 + lane >= jlo) ? expf(s_e[lane] - m) : 0.0f;
            float l = e;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
            s_e[lane] = e;
            if (lane == 0) {
                s_ml[0] = m;
                s_ml[1] = l;
            }
        }
        __syncthreads();
        float2 acc[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) acc[i] = make_float2(0.f, 0.f);
#pragma unroll
        for (int b = 0; b < PB; ++b) {
            const float e = s_e[w + 4 * b];  // 0 past jn
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const float2 v2 = kv_val<Q8>(vv[b][i]);
                acc[i].x += e * v2.x;
                acc[i].y += e * v2.y;
            }
        }
#pragma unroll
        for (int i = 0; i < NP; ++i) *reinterpret_cast<float2*>(&s_o[w][2 * (lane + 64 * i)]) = acc[i];
        __syncthreads();
        // merge the chunk (mc, lc, oc) into the running softmax
        const float mc = s_ml[0], lc = s_ml[1], mn = fmaxf(m_run, mc);
        const float a = m_run == -INFINITY ? 0.0f : expf(m_run - mn), bc = expf(mc - mn);
        if (tid < D) {
            const float oc = (s_o[0][tid] + s_o[1][tid]) + (s_o[2][tid] + s_o[3][tid]);
            o_run = o_run * a + oc * bc;
        }
        l_run = l_run * a + lc * bc;
        m_run = mn;
        __syncthreads();  // the next chunk overwrites s_e, s_o, s_ml
    }
    if (tid < D) out[size_t(t) * Q + size_t(h) * D + tid] = o_run * (1.0f / l_run);
}

// Attention of more tokens on MFMA, for head dims D of 64, 128 or 256. One
// workgroup (four wavefronts) per (block of 32
// tokens, head); wavefront w takes the key blocks of 32 positions
// b = b_lo + w, b_lo + w + 4, ... that the block's tokens can see, keeps a
// running max, sum and output per token, and the four are merged at the end
// (exact max, then the four sums and outputs rescaled and added in wavefront
// order). The tiles are transposed so that tokens run along lanes:
//   S^T = K Q^T   (32 keys x 32 tokens; k = the D head values),
//   O^T += V^T P^T (D values x 32 tokens in D / 32 tiles; k = the 32 keys).
// In the 32x32 MFMA output a lane holds one column (its token) and 16 rows:
// register r of lane half h is row 8 (r / 4) + 4 h + r % 4. So a token's
// softmax statistics stay in its own two lanes (l, l + 32), and the
// probabilities of S^T are already the B operand of the second product when
// its k order is taken to be that row order. K and V rows are staged through LDS per
// wavefront, rows past the block's last position as zeros (so a masked
// probability of 0 never meets a never-written cache row). Mathematically
// FISH's softmax (ops.cpp:331-350); the rounding order differs.
constexpr int kAttnMfmaTok = 32;
// The tiles run on f16 MFMA (v_mfma_f32_32x32x16_f16, 8x the rate of the f32
// form v_mfma_f32_32x32x2_f32) at f32 accuracy: K and V are f16 in the cache
// already, so only q and p are split, x = hi + lo with hi = f16(x),
// lo = f16(x - hi), and each product takes two MFMAs (K q hi + K q lo,
// V p hi + V p lo). f16 x f16 products are exact in the f32 accumulator, and
// what the split drops is below 2^-22 of |x| (2^-25 absolute where the lo part
// is subnormal). A token's q is first scaled by a power of two (its scores by
// the inverse) when its largest value exceeds 2^14, so hi never overflows.
// Operand lanes of the 32x32x16 form: A row = lane % 32, k = 8 (lane / 32) + e;
// B k likewise, column = lane % 32; the output as in the f32 form (register r
// of lane half h is row 8 (r / 4) + 4 h + r % 4). For O^T += V^T P^T the 8 k
// slots of a lane are the keys its S^T registers r = 8 u .. 8 u + 7 hold
// (16 u + 8 (e / 4) + 4 hf + e % 4), so p is the B operand straight from
// registers and V^T is gathered from the staged rows in that key order.
template <int D>
__global__ __launch_bounds__(256) void attn_mfma16_kernel(const float* __restrict__ q, const _Float16* __restrict__ kc,
                                                          const _Float16* __restrict__ vc, float* __restrict__ out,
                                                          int n_tok, int ld, int H, int HKV, int pos0, float scale,
                                                          float softcap, int window) {
    typedef float v16f __attribute__((ext_vector_type(16)));
    typedef _Float16 v8h __attribute__((ext_vector_type(8)));
    constexpr int NK = D / 16;     // k-steps of S^T
    constexpr int DT = D / 32;     // 32-row tiles of O^T
    constexpr int KROW = D + 8;    // LDS row stride in halves (16 bytes of padding)
    constexpr int STAGE = 2 * 4 * 32 * KROW * 2;                // K and V rows of the four wavefronts
    constexpr int MERGE = 4 * (D * 32 + 64) * 4;                // per wavefront: O^T, m, l
    __shared__ __align__(16) unsigned char s_mem[STAGE > MERGE ? STAGE : MERGE];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hf = lane >> 5, col = lane & 31;
    const int head = int(blockIdx.x) % H, qb = int(blockIdx.x) / H;
    const int kvh = head / (H / HKV), Q = H * D, KV = HKV * D;
    const int t0 = qb * kAttnMfmaTok, t = t0 + col;
    const int tc = min(t, n_tok - 1);                 // tokens past the call read the last one, unused
    const int pos = pos0 + tc;
    const int jlo = window > 0 ? max(0, pos - window + 1) : 0;  // this token's first position
    const int pos_last = pos0 + min(t0 + kAttnMfmaTok - 1, n_tok - 1);
    const int first_lo = window > 0 ? max(0, pos0 + t0 - window + 1) : 0;
    const int kb_lo = first_lo / 32, kb_hi = pos_last / 32;

    // Q^T operand: step kk uses q[t][16 kk + 8 hf + e], split into hi + lo
    const float* qr = q + size_t(tc) * Q + size_t(head) * D;
    float qf[NK][8];
    float qmax = 0.0f;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
        const float4 a = *reinterpret_cast<const float4*>(qr + 16 * kk + 8 * hf);
        const float4 b = *reinterpret_cast<const float4*>(qr + 16 * kk + 8 * hf + 4);
        qf[kk][0] = a.x; qf[kk][1] = a.y; qf[kk][2] = a.z; qf[kk][3] = a.w;
        qf[kk][4] = b.x; qf[kk][5] = b.y; qf[kk][6] = b.z; qf[kk][7] = b.w;
#pragma unroll
        for (int e = 0; e < 8; ++e) qmax = fmaxf(qmax, fabsf(qf[kk][e]));
    }
    qmax = fmaxf(qmax, __shfl_xor(qmax, 32));
    // the token's power-of-two scale: 2^-sh brings its largest value to at most 2^14
    int sh = 0;
    if (qmax > 16384.0f) {
        int ex;
        (void)frexpf(qmax, &ex);  // qmax = f 2^ex, 0.5 <= f < 1
        sh = ex - 14;
    }
    const float sc_out = sh ? ldexpf(scale, sh) : scale;
    v8h qh[NK], ql[NK];
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float x = sh ? ldexpf(qf[kk][e], -sh) : qf[kk][e];
            const _Float16 h = _Float16(x);
            qh[kk][e] = h;
            ql[kk][e] = _Float16(x - float(h));
        }

    _Float16* sk = reinterpret_cast<_Float16*>(s_mem) + size_t(w) * 32 * KROW;
    _Float16* sv = reinterpret_cast<_Float16*>(s_mem) + size_t(4 + w) * 32 * KROW;
    v16f o[DT];
#pragma unroll
    for (int c = 0; c < DT; ++c) o[c] = v16f{};
    float m_run = -INFINITY, l_run = 0.0f;
    // rows j0 .. j0 + 31 of K and V, 16 bytes per lane per piece; the next block's
    // pieces are loaded while the current block computes
    constexpr int PCS = 32 * (D / 8) / 64;  // pieces per lane
    uint4 nk[PCS], nv[PCS];
    auto load_block = [&](int kb) {
#pragma unroll
        for (int pc = 0; pc < PCS; ++pc) {
            const int i = lane + 64 * pc, r = i / (D / 8), c8 = i % (D / 8);
            const size_t at = size_t(min(kb * 32 + r, ld - 1)) * KV + size_t(kvh) * D + size_t(c8) * 8;
            nk[pc] = *reinterpret_cast<const uint4*>(kc + at);
            nv[pc] = *reinterpret_cast<const uint4*>(vc + at);
        }
    };
    // (head dim 256: no registers to spare, each block loaded when it is staged)
    constexpr bool PF = D <= 128;
    if (PF && kb_lo + w <= kb_hi) load_block(kb_lo + w);
    for (int kb = kb_lo + w; kb <= kb_hi; kb += 4) {  // uniform over the wavefront
        const int j0 = kb * 32;
        if (!PF) load_block(kb);
        // stage the block (rows past the block's last position as zeros)
#pragma unroll
        for (int pc = 0; pc < PCS; ++pc) {
            const int i = lane + 64 * pc, r = i / (D / 8), c8 = i % (D / 8);
            const bool live = j0 + r <= pos_last;
            *reinterpret_cast<uint4*>(sk + r * KROW + c8 * 8) = live ? nk[pc] : make_uint4(0, 0, 0, 0);
            *reinterpret_cast<uint4*>(sv + r * KROW + c8 * 8) = live ? nv[pc] : make_uint4(0, 0, 0, 0);
        }
        if (PF && kb + 4 <= kb_hi) load_block(kb + 4);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // S^T = K Q^T: rows = the block's keys (A from LDS), columns = tokens
        v16f s0 = v16f{}, s1 = v16f{};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
            const v8h ka = *reinterpret_cast<const v8h*>(sk + col * KROW + 16 * kk + 8 * hf);
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qh[kk], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, ql[kk], s1, 0, 0, 0);
        }
        // scores of this lane's token over its 16 keys (the other 16 are in lane l ^ 32)
        float p[16];
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int j = j0 + 8 * (r >> 2) + 4 * hf + (r & 3);
            const float sc = score(s0[r] + s1[r], sc_out, softcap);
            p[r] = (j <= pos && j >= jlo) ? sc : -INFINITY;
            mx = fmaxf(mx, p[r]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m_run, mx);
        const float a = mn == -INFINITY ? 1.0f : expf(m_run - mn);
        float ls = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            p[r] = p[r] == -INFINITY ? 0.0f : expf(p[r] - mn);
            ls += p[r];
        }
        ls += __shfl_xor(ls, 32);
        l_run = l_run * a + ls;
        m_run = mn;
#pragma unroll
        for (int c = 0; c < DT; ++c) o[c] *= a;
        // O^T += V^T P^T over the keys of registers 8 u .. 8 u + 7
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            v8h ph, pl;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const _Float16 h = _Float16(p[8 * u + e]);
                ph[e] = h;
                pl[e] = _Float16(p[8 * u + e] - float(h));
            }
#pragma unroll
            for (int c = 0; c < DT; ++c) {
                v8h va;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int kr = 16 * u + 8 * (e >> 2) + 4 * hf + (e & 3);
                    va[e] = sv[kr * KROW + 32 * c + col];
                }
                o[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, ph, o[c], 0, 0, 0);
                o[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pl, o[c], 0, 0, 0);
            }
        }
        __builtin_amdgcn_wave_barrier();  // the next block overwrites this wavefront's rows
    }
    // merge the four wavefronts: O^T rows (dims) of register r of tile c are 32 c + 8 (r / 4) + 4 hf + r % 4
    __syncthreads();
    float* mo = reinterpret_cast<float*>(s_mem) + size_t(w) * (D * 32 + 64);
#pragma unroll
    for (int c = 0; c < DT; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) mo[(32 * c + 8 * (r >> 2) + 4 * hf + (r & 3)) * 32 + col] = o[c][r];
    if (hf == 0) {
        mo[D * 32 + col] = m_run;
        mo[D * 32 + 32 + col] = l_run;
    }
    __syncthreads();
    const float* mb = reinterpret_cast<const float*>(s_mem);
    for (int i = tid; i < D * 32; i += 256) {
        const int d = i >> 5, tk = i & 31;
        if (t0 + tk >= n_tok) continue;
        float mw[4], M = -INFINITY;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            mw[v] = mb[size_t(v) * (D * 32 + 64) + D * 32 + tk];
            M = fmaxf(M, mw[v]);
        }
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float f = mw[v] == -INFINITY ? 0.0f : expf(mw[v] - M);
            L = L + mb[size_t(v) * (D * 32 + 64) + D * 32 + 32 + tk] * f;
            O = O + mb[size_t(v) * (D * 32 + 64) + d * 32 + tk] * f;
        }
        out[size_t(t0 + tk) * Q + size_t(head) * D + d] = O * (1.0f / L);
    }
}

// g = silu(g) * u
// g = act(g) * u: SiLU v / (1 + exp(-v)) (silu_inplace, ops.cpp:25-30), or with
// gelu FISH's tanh GELU 0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3)))
// (gelu_inplace, ops.cpp:32-38), each step rounded as there (no contraction)
__global__ __launch_bounds__(kTh) void act_mul_kernel(float* __restrict__ g, const float* __restrict__ u, size_t n,
                                                      int gelu) {
    const size_t i = size_t(blockIdx.x) * kTh + threadIdx.x;
    if (i >= n) return;
    g[i] = act_mul(g[i], u[i], gelu != 0);
}

// Row t of src [n_tok][w0 + w1 + w2] split into d0 [n_tok][w0], d1, d2 (a fused
// projection's output, model.cpp:1666-1673 and 1481-1490); w2 may be 0.
__global__ __launch_bounds__(kTh) void split_rows_kernel(const float* __restrict__ src, float* __restrict__ d0,
                                                         float* __restrict__ d1, float* __restrict__ d2, int w0,
                                                         int w1, int w2) {
    const int t = blockIdx.y, W = w0 + w1 + w2;
    const float* r = src + size_t(t) * W;
    for (int i = int(blockIdx.x) * kTh + threadIdx.x; i < W; i += int(gridDim.x) * kTh) {
        const float v = r[i];
        if (i < w0) d0[size_t(t) * w0 + i] = v;
        else if (i < w0 + w1) d1[size_t(t) * w1 + (i - w0)] = v;
        else d2[size_t(t) * w2 + (i - w0 - w1)] = v;
    }
}

// x += y
__global__ __launch_bounds__(kTh) void add_kernel(float* __restrict__ x, const float* __restrict__ y, size_t n) {
    const size_t i = size_t(blockIdx.x) * kTh + threadIdx.x;
    if (i < n) x[i] = x[i] + y[i];
}

unsigned blocks_for(size_t n) { return unsigned((n + kTh - 1) / kTh); }

}  // namespace

hipError_t launch_rmsnorm(float* x, const float* y, const float* b, const float* w, float* out, int n_tok, int n,
                          float eps, hipStream_t s) {
    if (n_tok <= 0 || n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(unsigned(n_tok)), dim3(kNormTh), 0, s, x, y, b, w, out, n, eps);
    return hipGetLastError();
}

namespace {

// int8 caches: kv_dim and head_dim multiples of 32 (whole 32-value blocks per head)
bool kv_ok(const KvCache& c, int D) { return c.c && (!c.d || D % 32 == 0); }

template <bool Q8>
void attention_split(const float* q, const KvCache& kc, const KvCache& vc, float* out, float* part, int ld, int n_tok,
                     int H, int HKV, int D, int pos0, float scale, hipStream_t s, const int* pos_dev, float softcap,
                     int window) {
    const dim3 block(kTh);
    if (n_tok > kAttnSplitTok) {
        const dim3 grid(unsigned(n_tok * H));
        if (D <= 128)
            hipLaunchKernelGGL((attn_full_kernel<1, Q8>), grid, block, 0, s, q, kc, vc, out, H, HKV, D, pos0, pos_dev,
                               scale, softcap, window);
        else
            hipLaunchKernelGGL((attn_full_kernel<2, Q8>), grid, block, 0, s, q, kc, vc, out, H, HKV, D, pos0, pos_dev,
                               scale, softcap, window);
        return;
    }
    const int S = (ld + kCh - 1) / kCh;
    const dim3 grid(unsigned(n_tok * H), unsigned(S));
    const AttnPrep P{};
    if (D <= 128)
        hipLaunchKernelGGL((attn_part_kernel<1, false, Q8>), grid, block, 0, s, q, kc, vc, part, S, H, HKV, D, pos0,
                           pos_dev, scale, softcap, window, P);
    else
        hipLaunchKernelGGL((attn_part_kernel<2, false, Q8>), grid, block, 0, s, q, kc, vc, part, S, H, HKV, D, pos0,
                           pos_dev, scale, softcap, window, P);
    hipLaunchKernelGGL(attn_combine_kernel, dim3(unsigned(n_tok * H)), block, 0, s, part, out, S, H, D, pos0,
                       pos_dev);
}

template <bool Q8>
void attention_prep(const AttnPrep& P, const KvCache& kc, const KvCache& vc, float* out, float* part, int ld, int H,
                    int HKV, int D, int pos0, float scale, hipStream_t s, const int* pos_dev, float softcap,
                    int window) {
    const int S = (ld + kCh - 1) / kCh;
    const dim3 grid{unsigned(H), unsigned(S)}, block{unsigned(kTh)};
    if (D <= 128)
        hipLaunchKernelGGL((attn_part_kernel<1, true, Q8>), grid, block, 0, s, P.q_out, kc, vc, part, S, H, HKV, D,
                           pos0, pos_dev, scale, softcap, window, P);
    else
        hipLaunchKernelGGL((attn_part_kernel<2, true, Q8>), grid, block, 0, s, P.q_out, kc, vc, part, S, H, HKV, D,
                           pos0, pos_dev, scale, softcap, window, P);
    hipLaunchKernelGGL(attn_combine_kernel, dim3(unsigned(H)), block, 0, s, part, out, S, H, D, pos0, pos_dev);
}

}  // namespace

hipError_t launch_qkv_prep(const float* q, const float* k, const float* v, const SpanVecs& vecs, float* q_out,
                           const KvCache& kc, const KvCache& vc, int n_tok, int H, int HKV, int D, int rot_dim,
                           bool neox, float eps, int pos0, const float* cosv, const float* sinv, hipStream_t s,
                           const int* pos_dev) {
    if (n_tok <= 0 || H <= 0 || HKV <= 0 || D <= 0 || D > kTh || rot_dim < 0 || rot_dim > D || rot_dim % 2 ||
        !kv_ok(kc, D) || !kv_ok(vc, D) || !kc.d != !vc.d)
        return hipErrorInvalidValue;
    const dim3 grid(unsigned(n_tok), unsigned(H + HKV));
    if (kc.d)
        hipLaunchKernelGGL(qkv_prep_kernel<true>, grid, dim3(kTh), 0, s, q, k, v, vecs, q_out, kc, vc, H * D, HKV * D,
                           D, rot_dim / 2, neox ? 1 : 0, eps, pos0, pos_dev, cosv, sinv);
    else
        hipLaunchKernelGGL(qkv_prep_kernel<false>, grid, dim3(kTh), 0, s, q, k, v, vecs, q_out, kc, vc, H * D, HKV * D,
                           D, rot_dim / 2, neox ? 1 : 0, eps, pos0, pos_dev, cosv, sinv);
    return hipGetLastError();
}

hipError_t launch_attention(const float* q, const KvCache& kc, const KvCache& vc, float* out, float* part, int ld,
                            int n_tok, int H, int HKV, int D, int pos0, float scale, hipStream_t s,
                            const int* pos_dev, float softcap, int window) {
    if (n_tok <= 0 || D <= 0 || D > kTh || D % 2 || HKV <= 0 || H % HKV || ld < pos0 + n_tok || !kv_ok(kc, D) ||
        !kv_ok(vc, D) || !kc.d != !vc.d)
        return hipErrorInvalidValue;
    if (n_tok > kAttnSplitTok && !pos_dev && (D == 64 || D == 128 || D == 256) && !kc.d) {
        const dim3 grid(unsigned((n_tok + kAttnMfmaTok - 1) / kAttnMfmaTok * H)), block(kTh);
        const _Float16* k16 = static_cast<const _Float16*>(kc.c);
        const _Float16* v16 = static_cast<const _Float16*>(vc.c);
        if (D == 256)
            hipLaunchKernelGGL(attn_mfma16_kernel<256>, grid, block, 0, s, q, k16, v16, out, n_tok, ld, H, HKV, pos0,
                               scale, softcap, window);
        else if (D == 64)
            hipLaunchKernelGGL(attn_mfma16_kernel<64>, grid, block, 0, s, q, k16, v16, out, n_tok, ld, H, HKV, pos0,
                               scale, softcap, window);
        else
            hipLaunchKernelGGL(attn_mfma16_kernel<128>, grid, block, 0, s, q, k16, v16, out, n_tok, ld, H, HKV, pos0,
                               scale, softcap, window);
        return hipGetLastError();
    }
    if (kc.d)
        attention_split<true>(q, kc, vc, out, part, ld, n_tok, H, HKV, D, pos0, scale, s, pos_dev, softcap, window);
    else
        attention_split<false>(q, kc, vc, out, part, ld, n_tok, H, HKV, D, pos0, scale, s, pos_dev, softcap, window);
    return hipGetLastError();
}

hipError_t launch_attention_prep(const float* q, const float* k, const float* v, const SpanVecs& vecs, float* q_out,
                                 const KvCache& kc, const KvCache& vc, float* out, float* part, int ld, int H, int HKV,
                                 int D, int rot_dim, bool neox, float eps, int pos0, const float* cosv,
                                 const float* sinv, float scale, hipStream_t s, const int* pos_dev, float softcap,
                                 int window) {
    if (D <= 0 || D > kTh || D % 2 || HKV <= 0 || H % HKV || ld < pos0 + 1 || rot_dim < 0 || rot_dim > D ||
        rot_dim % 2 || !kv_ok(kc, D) || !kv_ok(vc, D) || !kc.d != !vc.d)
        return hipErrorInvalidValue;
    const AttnPrep P{q, k, v, vecs, q_out, kc, vc, cosv, sinv, rot_dim / 2, neox ? 1 : 0, eps};
    if (kc.d)
        attention_prep<true>(P, kc, vc, out, part, ld, H, HKV, D, pos0, scale, s, pos_dev, softcap, window);
    else
        attention_prep<false>(P, kc, vc, out, part, ld, H, HKV, D, pos0, scale, s, pos_dev, softcap, window);
    return hipGetLastError();
}

size_t attention_scratch_floats(int n_tok, int H, int D, int ld) {
    if (n_tok > kAttnSplitTok) return 0;
    return size_t(n_tok) * H * size_t((ld + kCh - 1) / kCh) * size_t(D + 2);
}

hipError_t launch_silu_mul(float* g, const float* u, size_t n, hipStream_t s, bool gelu) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(act_mul_kernel, dim3(blocks_for(n)), dim3(kTh), 0, s, g, u, n, gelu ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_split_rows(const float* src, int n_tok, float* d0, int w0, float* d1, int w1, float* d2, int w2,
                             hipStream_t s) {
    if (n_tok <= 0 || w0 <= 0 || w1 <= 0 || w2 < 0 || (w2 > 0 && !d2)) return hipErrorInvalidValue;
    const int W = w0 + w1 + w2;
    hipLaunchKernelGGL(split_rows_kernel, dim3(unsigned((W + kTh - 1) / kTh), unsigned(n_tok)), dim3(kTh), 0, s, src,
                       d0, d1, d2, w0, w1, w2);
    return hipGetLastError();
}

hipError_t launch_add(float* x, const float* y, size_t n, hipStream_t s) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(add_kernel, dim3(blocks_for(n)), dim3(kTh), 0, s, x, y, n);
    return hipGetLastError();
}

}  // namespace fishhip
