// The non-matmul steps of a dense transformer layer, for layer spans: a range
// of layers run entirely on the device per forward call (the ComputeBackend
// span contract, backend.h:89-162), with the projections on the matmul kernels.
//
// Each kernel restates FISH's CPU step for one layer (model.cpp:1650-1790):
//   rmsnorm      ops.cpp:18-23   (double sum of squares, f32 scale, x * scale * w)
//   RoPE + KV    ops.cpp:126-152 (table rotation, neox or adjacent pairs) and the
//                KV-cache store of model.cpp:1726-1734
//   attention    ops.cpp:303-357 (causal, GQA head groups, max-subtracted exp,
//                softmax-weighted sum of V; split over position chunks)
//   silu * up    ops.cpp:25-30, model.cpp:1504-1508
//   residual add model.cpp:1772-1776, :1797-1801 (fused into the next rmsnorm)
// The file is compiled without floating-point contraction, so every
// expression rounds as FISH's baseline x86-64 build does; exp is the device's
// expf, within a few ulp of the C library's.
#include "common.h"
#include "kernels.h"

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
// residual add, written back to x), then out = rmsnorm(x)
__global__ __launch_bounds__(kNormTh) void rmsnorm_kernel(float* __restrict__ x, const float* __restrict__ y,
                                                          const float* __restrict__ w, float* __restrict__ out, int n,
                                                          float eps) {
    __shared__ double red[kNormTh];
    float* xr = x + size_t(blockIdx.x) * n;
    const float* yr = y ? y + size_t(blockIdx.x) * n : nullptr;
    float* orow = out + size_t(blockIdx.x) * n;
    double s = 0.0;
#pragma unroll 4
    for (int i = threadIdx.x; i < n; i += kNormTh) {
        float v = xr[i];
        if (yr) {
            v = v + yr[i];
            xr[i] = v;
        }
        s += double(v) * double(v);
    }
    const double sum = block_sum_d(s, red);
    const float scale = 1.0f / sqrtf(float(sum / n) + eps);
    for (int i = threadIdx.x; i < n; i += kNormTh) orow[i] = xr[i] * scale * w[i];
}

// The rotated value of element f of a row of heads of D values (ops.cpp:126-152).
__device__ __forceinline__ float rope_elem(const float* __restrict__ src, int f, int D, int half, int neox,
                                           const float* __restrict__ c, const float* __restrict__ s) {
    const int base = f - f % D, d = f % D;
    if (d >= 2 * half) return src[f];  // past rot_dim: unchanged
    if (neox) {
        const int i = d < half ? d : d - half;
        const float x0 = src[base + i], x1 = src[base + i + half];
        return d < half ? x0 * c[i] - x1 * s[i] : x0 * s[i] + x1 * c[i];
    }
    const int i = d >> 1;
    const float x0 = src[base + 2 * i], x1 = src[base + 2 * i + 1];
    return (d & 1) ? x0 * s[i] + x1 * c[i] : x0 * c[i] - x1 * s[i];
}

// one workgroup per (token t, head): q heads first, then k heads; q_out =
// rope(q), the cache rows of position pos0 + t get rope(k) and v
__global__ __launch_bounds__(kTh) void rope_store_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                         const float* __restrict__ v, float* __restrict__ q_out,
                                                         float* __restrict__ kc, float* __restrict__ vc, int Q,
                                                         int KV, int D, int half, int neox, int pos0,
                                                         const int* __restrict__ pos_dev,
                                                         const float* __restrict__ cosv,
                                                         const float* __restrict__ sinv) {
    if (pos_dev) pos0 = *pos_dev;
    const int t = blockIdx.x, hh = blockIdx.y, pos = pos0 + t, H = Q / D;
    const float* c = cosv + size_t(pos) * half;
    const float* s = sinv + size_t(pos) * half;
    if (hh < H) {
        const float* qr = q + size_t(t) * Q;
        for (int f = hh * D + threadIdx.x; f < (hh + 1) * D; f += kTh)
            q_out[size_t(t) * Q + f] = rope_elem(qr, f, D, half, neox, c, s);
    } else {
        const float* kr = k + size_t(t) * KV;
        const float* vr = v + size_t(t) * KV;
        for (int f = (hh - H) * D + threadIdx.x; f < (hh - H + 1) * D; f += kTh) {
            kc[size_t(pos) * KV + f] = rope_elem(kr, f, D, half, neox, c, s);
            vc[size_t(pos) * KV + f] = vr[f];
        }
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
// Chunks that start past the token's position hold m = -inf, l = 0, o = 0.
// Mathematically FISH's single-pass softmax (ops.cpp:331-350); the rounding
// order differs. Needs D <= 256.
constexpr int kCh = 64;

template <int DL>
__global__ __launch_bounds__(kTh) void attn_part_kernel(const float* __restrict__ q, const float* __restrict__ kc,
                                                        const float* __restrict__ vc, float* __restrict__ part,
                                                        int S, int H, int HKV, int D, int pos0,
                                                        const int* __restrict__ pos_dev, float scale) {
    constexpr int PB = kCh / 4;
    __shared__ float s_e[kCh];
    __shared__ float s_o[4][64 * DL];
    __shared__ float s_ml[2];
    if (pos_dev) pos0 = *pos_dev;
    const int item = blockIdx.x, chunk = blockIdx.y, t = item / H, h = item % H;
    const int pos = pos0 + t, kvh = h / (H / HKV), KV = HKV * D, Q = H * D;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int j0 = chunk * kCh;
    float* pp = part + (size_t(item) * S + chunk) * size_t(D + 2);
    if (j0 > pos) {  // uniform over the workgroup
        for (int d = tid; d < D; d += kTh) pp[d] = 0.0f;
        if (tid == 0) {
            pp[D] = -INFINITY;
            pp[D + 1] = 0.0f;
        }
        return;
    }
    const int jn = min(pos, j0 + kCh - 1);
    float qv[DL];
#pragma unroll
    for (int i = 0; i < DL; ++i) qv[i] = lane + 64 * i < D ? q[size_t(t) * Q + size_t(h) * D + lane + 64 * i] : 0.0f;
    const float* kb = kc + size_t(kvh) * D;
    const float* vb = vc + size_t(kvh) * D;

    // scores of positions j0 + w + 4 b
    float kv[PB][DL];
#pragma unroll
    for (int b = 0; b < PB; ++b) {
        const float* kr = kb + size_t(min(j0 + w + 4 * b, jn)) * KV;
#pragma unroll
        for (int i = 0; i < DL; ++i) kv[b][i] = lane + 64 * i < D ? kr[lane + 64 * i] : 0.0f;
    }
#pragma unroll
    for (int b = 0; b < PB; ++b) {
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < DL; ++i) sum += qv[i] * kv[b][i];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
        if (lane == 0) s_e[w + 4 * b] = j0 + w + 4 * b <= jn ? sum * scale : -INFINITY;
    }
    __syncthreads();
    if (w == 0) {
        float m = s_e[lane];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        const float e = lane <= jn - j0 ? expf(s_e[lane] - m) : 0.0f;
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
    float vv[PB][DL];
#pragma unroll
    for (int b = 0; b < PB; ++b) {
        const float* vr = vb + size_t(min(j0 + w + 4 * b, jn)) * KV;
#pragma unroll
        for (int i = 0; i < DL; ++i) vv[b][i] = lane + 64 * i < D ? vr[lane + 64 * i] : 0.0f;
    }
    float acc[DL];
#pragma unroll
    for (int i = 0; i < DL; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int b = 0; b < PB; ++b) {
        const float e = s_e[w + 4 * b];  // 0 past jn
#pragma unroll
        for (int i = 0; i < DL; ++i) acc[i] += e * vv[b][i];
    }
#pragma unroll
    for (int i = 0; i < DL; ++i) s_o[w][lane + 64 * i] = acc[i];
    __syncthreads();
    for (int d = tid; d < D; d += kTh) pp[d] = (s_o[0][d] + s_o[1][d]) + (s_o[2][d] + s_o[3][d]);
    if (tid == 0) {
        pp[D] = s_ml[0];
        pp[D + 1] = s_ml[1];
    }
}

__global__ __launch_bounds__(kTh) void attn_combine_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                           int S, int H, int D) {
    __shared__ float red[kTh];
    __shared__ float s_w[kTh];
    const int item = blockIdx.x, t = item / H, h = item % H, tid = threadIdx.x;
    const size_t st = size_t(D + 2);
    const float* pp = part + size_t(item) * S * st;
    float m = -INFINITY;
    for (int c = tid; c < S; c += kTh) m = fmaxf(m, pp[size_t(c) * st + D]);
    const float M = block_reduce_f(m, red, true);
    float l = 0.0f, o = 0.0f;
    for (int c0 = 0; c0 < S; c0 += kTh) {
        const int c = c0 + tid;
        float wc = 0.0f;
        if (c < S) {
            const float mc = pp[size_t(c) * st + D];
            wc = mc == -INFINITY ? 0.0f : expf(mc - M);
            l += pp[size_t(c) * st + D + 1] * wc;
        }
        s_w[tid] = wc;
        __syncthreads();
        const int nc = min(kTh, S - c0);
        if (tid < D) {
            const float* pc = pp + size_t(c0) * st + tid;
#pragma unroll 8
            for (int cc = 0; cc < nc; ++cc) o += pc[size_t(cc) * st] * s_w[cc];
        }
        __syncthreads();
    }
    const float L = block_reduce_f(l, red, false);
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    if (tid < D) out[size_t(t) * H * D + size_t(h) * D + tid] = o * inv;
}

// g = silu(g) * u
__global__ __launch_bounds__(kTh) void silu_mul_kernel(float* __restrict__ g, const float* __restrict__ u, size_t n) {
    const size_t i = size_t(blockIdx.x) * kTh + threadIdx.x;
    if (i >= n) return;
    const float v = g[i];
    const float a = v / (1.0f + expf(-v));
    g[i] = a * u[i];
}

// x += y
__global__ __launch_bounds__(kTh) void add_kernel(float* __restrict__ x, const float* __restrict__ y, size_t n) {
    const size_t i = size_t(blockIdx.x) * kTh + threadIdx.x;
    if (i < n) x[i] = x[i] + y[i];
}

unsigned blocks_for(size_t n) { return unsigned((n + kTh - 1) / kTh); }

}  // namespace

hipError_t launch_rmsnorm(float* x, const float* y, const float* w, float* out, int n_tok, int n, float eps,
                          hipStream_t s) {
    if (n_tok <= 0 || n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(unsigned(n_tok)), dim3(kNormTh), 0, s, x, y, w, out, n, eps);
    return hipGetLastError();
}

hipError_t launch_rope_store(const float* q, const float* k, const float* v, float* q_out, float* kc, float* vc,
                             int n_tok, int H, int HKV, int D, int rot_dim, bool neox, int pos0, const float* cosv,
                             const float* sinv, hipStream_t s, const int* pos_dev) {
    if (n_tok <= 0 || H <= 0 || HKV <= 0 || D <= 0 || rot_dim < 0 || rot_dim > D || rot_dim % 2) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_store_kernel, dim3(unsigned(n_tok), unsigned(H + HKV)), dim3(kTh), 0, s, q, k, v, q_out, kc, vc, H * D,
                       HKV * D, D, rot_dim / 2, neox ? 1 : 0, pos0, pos_dev, cosv, sinv);
    return hipGetLastError();
}

hipError_t launch_attention(const float* q, const float* kc, const float* vc, float* out, float* part, int ld,
                            int n_tok, int H, int HKV, int D, int pos0, float scale, hipStream_t s,
                            const int* pos_dev) {
    if (n_tok <= 0 || D <= 0 || D > kTh || HKV <= 0 || H % HKV || ld < pos0 + n_tok) return hipErrorInvalidValue;
    const int S = (ld + kCh - 1) / kCh;
    const dim3 grid(unsigned(n_tok * H), unsigned(S)), block(kTh);
    if (D <= 64)
        hipLaunchKernelGGL(attn_part_kernel<1>, grid, block, 0, s, q, kc, vc, part, S, H, HKV, D, pos0, pos_dev, scale);
    else if (D <= 128)
        hipLaunchKernelGGL(attn_part_kernel<2>, grid, block, 0, s, q, kc, vc, part, S, H, HKV, D, pos0, pos_dev, scale);
    else
        hipLaunchKernelGGL(attn_part_kernel<4>, grid, block, 0, s, q, kc, vc, part, S, H, HKV, D, pos0, pos_dev, scale);
    hipLaunchKernelGGL(attn_combine_kernel, dim3(unsigned(n_tok * H)), block, 0, s, part, out, S, H, D);
    return hipGetLastError();
}

size_t attention_scratch_floats(int n_tok, int H, int D, int ld) {
    return size_t(n_tok) * H * size_t((ld + kCh - 1) / kCh) * size_t(D + 2);
}

hipError_t launch_silu_mul(float* g, const float* u, size_t n, hipStream_t s) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks_for(n)), dim3(kTh), 0, s, g, u, n);
    return hipGetLastError();
}

hipError_t launch_add(float* x, const float* y, size_t n, hipStream_t s) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(add_kernel, dim3(blocks_for(n)), dim3(kTh), 0, s, x, y, n);
    return hipGetLastError();
}

}  // namespace fishhip
