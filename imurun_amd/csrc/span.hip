// The non-matmul steps of a dense transformer layer, for layer spans: a range
// of layers run entirely on the device per forward call (the ComputeBackend
// span contract, backend.h:89-162), with the projections on the matmul kernels.
//
// Each kernel restates FISH's CPU step for one layer (model.cpp:1650-1790):
//   rmsnorm      ops.cpp:18-23   (double sum of squares, f32 scale, x * scale * w)
//   RoPE + KV    ops.cpp:126-152 (table rotation, neox or adjacent pairs) and the
//                KV-cache store of model.cpp:1726-1734
//   attention    ops.cpp:303-357 (causal, GQA head groups, max-subtracted exp,
//                p = e * (1 / sum), o = sum_j p_j v_j)
//   silu * up    ops.cpp:25-30, model.cpp:1504-1508
//   residual add model.cpp:1772-1776, :1797-1801
// The file is compiled without floating-point contraction, so every
// expression rounds as FISH's baseline x86-64 build does; exp is the device's
// expf, within a few ulp of the C library's.
#include "common.h"
#include "kernels.h"

namespace fishhip {

namespace {

constexpr int kTh = 256;

__device__ __forceinline__ double block_sum_d(double v, double* red) {
    const int tid = threadIdx.x;
    red[tid] = v;
    __syncthreads();
    for (int s = kTh / 2; s > 0; s >>= 1) {
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

// one workgroup per token
__global__ __launch_bounds__(kTh) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      float* __restrict__ out, int n, float eps) {
    __shared__ double red[kTh];
    const float* xr = x + size_t(blockIdx.x) * n;
    float* orow = out + size_t(blockIdx.x) * n;
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += kTh) s += double(xr[i]) * double(xr[i]);
    const double sum = block_sum_d(s, red);
    const float scale = 1.0f / sqrtf(float(sum / n) + eps);
    for (int i = threadIdx.x; i < n; i += kTh) orow[i] = xr[i] * scale * w[i];
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

// one workgroup per token t (position pos0 + t): q_out = rope(q), the cache
// rows of the position get rope(k) and v
__global__ __launch_bounds__(kTh) void rope_store_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                         const float* __restrict__ v, float* __restrict__ q_out,
                                                         float* __restrict__ kc, float* __restrict__ vc, int Q,
                                                         int KV, int D, int half, int neox, int pos0,
                                                         const float* __restrict__ cosv,
                                                         const float* __restrict__ sinv) {
    const int t = blockIdx.x, pos = pos0 + t;
    const float* c = cosv + size_t(pos) * half;
    const float* s = sinv + size_t(pos) * half;
    const float* qr = q + size_t(t) * Q;
    const float* kr = k + size_t(t) * KV;
    const float* vr = v + size_t(t) * KV;
    for (int f = threadIdx.x; f < Q; f += kTh) q_out[size_t(t) * Q + f] = rope_elem(qr, f, D, half, neox, c, s);
    for (int f = threadIdx.x; f < KV; f += kTh) {
        kc[size_t(pos) * KV + f] = rope_elem(kr, f, D, half, neox, c, s);
        vc[size_t(pos) * KV + f] = vr[f];
    }
}

// One workgroup (four wavefronts) per (token, head). Lanes run over the
// head's D values (DL = D / 64 per lane, rounded up; lanes past D hold
// zeros), so every K or V row is one coalesced load; wavefront w takes the
// positions j = w, w + 4, ... up to pos.
//   scores: per position a lane-partial dot, summed over the wavefront with
//           xor shuffles, scaled, kept in the workgroup's row of `scores`;
//   softmax: max and sum over the workgroup; p_j = e_j * (1 / sum);
//   o:      each wavefront sums p_j v_j over its positions in registers; the
//           four partial vectors are added in LDS.
// Needs D <= 256.
template <int DL>
__global__ __launch_bounds__(kTh) void attention_kernel(const float* __restrict__ q, const float* __restrict__ kc,
                                                        const float* __restrict__ vc, float* __restrict__ out,
                                                        float* __restrict__ scores, int ld, int H, int HKV, int D,
                                                        int pos0, float scale) {
    __shared__ float red[kTh];
    __shared__ float s_o[4][64 * DL];
    const int item = blockIdx.x, t = item / H, h = item % H;
    const int pos = pos0 + t, kvh = h / (H / HKV), KV = HKV * D, Q = H * D;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    float qv[DL];
#pragma unroll
    for (int i = 0; i < DL; ++i) {
        const int d = lane + 64 * i;
        qv[i] = d < D ? q[size_t(t) * Q + size_t(h) * D + d] : 0.0f;
    }
    float* sc = scores + size_t(item) * ld;
    const float* kb = kc + size_t(kvh) * D;
    const float* vb = vc + size_t(kvh) * D;

    // PB positions per wavefront step, all their row loads issued before the
    // first use (clamped to pos: unconditional loads, extra positions dropped)
    constexpr int PB = 16;
    float m = -INFINITY;
    for (int j0 = w; j0 <= pos; j0 += 4 * PB) {
        float kv[PB][DL];
#pragma unroll
        for (int b = 0; b < PB; ++b) {
            const float* kr = kb + size_t(min(j0 + 4 * b, pos)) * KV;
#pragma unroll
            for (int i = 0; i < DL; ++i) kv[b][i] = lane + 64 * i < D ? kr[lane + 64 * i] : 0.0f;
        }
#pragma unroll
        for (int b = 0; b < PB; ++b) {
            float part = 0.0f;
#pragma unroll
            for (int i = 0; i < DL; ++i) part += qv[i] * kv[b][i];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
            const float sv = part * scale;
            const int j = j0 + 4 * b;
            if (j <= pos) {
                if (lane == 0) sc[j] = sv;
                m = fmaxf(m, sv);
            }
        }
    }
    const float mx = block_reduce_f(m, red, true);  // its barriers also order the sc writes
    float sum = 0.0f;
    for (int j = tid; j <= pos; j += kTh) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        sum += e;
    }
    const float tot = block_reduce_f(sum, red, false);
    const float inv = tot > 0.0f ? 1.0f / tot : 0.0f;

    float acc[DL];
#pragma unroll
    for (int i = 0; i < DL; ++i) acc[i] = 0.0f;
    for (int j0 = w; j0 <= pos; j0 += 4 * PB) {
        float vv[PB][DL], pp[PB];
#pragma unroll
        for (int b = 0; b < PB; ++b) {
            const int j = min(j0 + 4 * b, pos);
            pp[b] = j0 + 4 * b <= pos ? sc[j] * inv : 0.0f;
            const float* vr = vb + size_t(j) * KV;
#pragma unroll
            for (int i = 0; i < DL; ++i) vv[b][i] = lane + 64 * i < D ? vr[lane + 64 * i] : 0.0f;
        }
#pragma unroll
        for (int b = 0; b < PB; ++b)
#pragma unroll
            for (int i = 0; i < DL; ++i) acc[i] += pp[b] * vv[b][i];
    }
#pragma unroll
    for (int i = 0; i < DL; ++i) s_o[w][lane + 64 * i] = acc[i];
    __syncthreads();
    for (int d = tid; d < D; d += kTh)
        out[size_t(t) * Q + size_t(h) * D + d] = (s_o[0][d] + s_o[1][d]) + (s_o[2][d] + s_o[3][d]);
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

hipError_t launch_rmsnorm(const float* x, const float* w, float* out, int n_tok, int n, float eps, hipStream_t s) {
    if (n_tok <= 0 || n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(unsigned(n_tok)), dim3(kTh), 0, s, x, w, out, n, eps);
    return hipGetLastError();
}

hipError_t launch_rope_store(const float* q, const float* k, const float* v, float* q_out, float* kc, float* vc,
                             int n_tok, int H, int HKV, int D, int rot_dim, bool neox, int pos0, const float* cosv,
                             const float* sinv, hipStream_t s) {
    if (n_tok <= 0 || H <= 0 || HKV <= 0 || D <= 0 || rot_dim < 0 || rot_dim > D || rot_dim % 2) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_store_kernel, dim3(unsigned(n_tok)), dim3(kTh), 0, s, q, k, v, q_out, kc, vc, H * D,
                       HKV * D, D, rot_dim / 2, neox ? 1 : 0, pos0, cosv, sinv);
    return hipGetLastError();
}

hipError_t launch_attention(const float* q, const float* kc, const float* vc, float* out, float* scores, int ld,
                            int n_tok, int H, int HKV, int D, int pos0, float scale, hipStream_t s) {
    if (n_tok <= 0 || D <= 0 || D > kTh || HKV <= 0 || H % HKV || ld < pos0 + n_tok) return hipErrorInvalidValue;
    const dim3 grid(unsigned(n_tok * H)), block(kTh);
    if (D <= 64) hipLaunchKernelGGL(attention_kernel<1>, grid, block, 0, s, q, kc, vc, out, scores, ld, H, HKV, D, pos0, scale);
    else if (D <= 128) hipLaunchKernelGGL(attention_kernel<2>, grid, block, 0, s, q, kc, vc, out, scores, ld, H, HKV, D, pos0, scale);
    else hipLaunchKernelGGL(attention_kernel<4>, grid, block, 0, s, q, kc, vc, out, scores, ld, H, HKV, D, pos0, scale);
    return hipGetLastError();
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
