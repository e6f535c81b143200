// Activation quantizer for gfx950: f32 rows -> FISH's two int8 layouts.
//
// Semantics (quantize_acts_scalar / quantize_acts_k_scalar, quant.cpp:400-434,
// built per row by ActBatch::quantize, ops.cpp:158-175):
//   per block of B values (B = 32 or 256): amax = max |x|; d = amax / 127
//   (IEEE f32 division); id = d > 0 ? 1 / d : 0; q = clamp(rint(x * id),
//   -127, 127) with round-half-to-even; 32-layout keeps sum(q), 256-layout
//   keeps the eight per-32 sums.
// The absmax is order independent, so a wavefront reduction is exact; the
// division and reciprocal are the correctly rounded IEEE operations (the
// build keeps -fhip-fp32-correctly-rounded-divide-sqrt and denormals), and
// x * id is a single rounding fed to v_rndne_f32. Inputs are assumed free of
// NaN (FISH's std::max would skip them; the hardware max would not).
//
// One wavefront per (token, run of 256-value chunks); each lane owns 4
// consecutive values of a chunk. Lanes 8j..8j+7 form the 32-block j of the chunk.
#include "common.h"
#include "kernels.h"
#include "qact.h"

namespace fishhip {

namespace {

struct QuantOut {
    int8_t* q32; float* d32; int32_t* s32;
    int8_t* q256; float* d256; int16_t* s16; int8_t* bsm;
    int8_t* m32; int8_t* m256;  // MFMA operand order (rows of whole 256-element units)
    int8_t* gA; float* gX; uint16_t* gJ;  // 32x32x32 MFMA planes (rows padded to 32-token blocks)
    uint8_t* aos32;   // optional FISH Q8Act rows (40 B blocks)
    uint8_t* aos256;  // optional FISH Q8ActK rows (276 B blocks)
};


// Byte offset, inside its 256-element unit, of the dword that holds this
// lane's four codes in MFMA operand order: lane L of the unit holds elements
// 4L..4L+3, i.e. dword L % 8 of group L / 8; dwords 0..3 of a group go to
// quarter q = L % 8 (codes 0..3), dwords 4..7 to quarter L % 8 - 4 (codes 4..7).
__device__ __forceinline__ int mfma_offset(int lane) {
    const int g = lane >> 3, w = lane & 7;
    return (w & 3) * 64 + g * 8 + (w >> 2) * 4;
}

// One (token, 256-value chunk) in registers -> every requested layout.
// GEMM_ONLY: the K-quant GEMM's planes (gA gX gJ) alone, with no run-time checks
// of the other outputs (n_in a multiple of 256).
template <bool GEMM_ONLY>
__device__ __forceinline__ void quantize_chunk(float4 v, int t, int c, int n_tok, int n_in, const QuantOut& o,
                                               int lane) {
    const int k0 = c * 256 + lane * 4;
    const bool real = t < n_tok;
    const bool active = real && k0 < n_in;  // n_in % 32 == 0: whole 8-lane groups switch together
    const float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));

    // ---- 32-value blocks (skipped when no 32-layout plane is requested: a K-quant
    // GEMM's input needs only the 256-value planes)
    if (!GEMM_ONLY && (o.q32 || o.m32 || o.d32 || o.aos32)) {
        const float amax = wave_max8(a);
        const float d = amax / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        const int q0 = code(v.x, id), q1 = code(v.y, id), q2 = code(v.z, id), q3 = code(v.w, id);
        const int sum = wave_sum8(q0 + q1 + q2 + q3);
        if (active) {
            const uint32_t packed = pack4(q0, q1, q2, q3);
            if (o.q32) *reinterpret_cast<uint32_t*>(o.q32 + size_t(t) * n_in + k0) = packed;
            if (o.m32)
                *reinterpret_cast<uint32_t*>(o.m32 + size_t(t) * n_in + size_t(c) * 256 + mfma_offset(lane)) = packed;
            const size_t blk = size_t(t) * (n_in / 32) + k0 / 32;
            if ((lane & 7) == 0) {
                if (o.d32) o.d32[blk] = d;
                if (o.s32) o.s32[blk] = sum;
            }
            if (o.aos32) {
                uint8_t* b = o.aos32 + blk * 40;
                *reinterpret_cast<uint32_t*>(b + 8 + 4 * (lane & 7)) = packed;
                if ((lane & 7) == 0) {
                    *reinterpret_cast<float*>(b) = d;
                    *reinterpret_cast<int32_t*>(b + 4) = sum;
                }
            }
        }
    }

    // ---- 256-value blocks (only when every row is a whole number of them)
    if (GEMM_ONLY || ((o.d256 || o.gA || o.aos256) && (n_in % 256) == 0)) {
        const float amax = wave_max64(a);
        const float d = amax / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        const int q0 = code(v.x, id), q1 = code(v.y, id), q2 = code(v.z, id), q3 = code(v.w, id);
        const int s4 = q0 + q1 + q2 + q3;
        // per-16 sums: lanes 4j..4j+3 hold one 16-value group; 8 lanes one 32-value group
        const int g16 = wave_sum4(s4);
        const int g32 = g16 + dpp_i<kDppHalfMirror>(g16);
        const uint32_t packed = pack4(q0, q1, q2, q3);
        if (GEMM_ONLY || o.gA) {
            // 32x32x32 MFMA planes: token block tb, step k0 / 32, half h, 4-byte slot of the lane
            const int n_sb = n_in / 256, tb = t >> 5, tt = t & 31;
            const size_t step = size_t(k0 >> 5), h = size_t((lane & 7) >> 2);
            *reinterpret_cast<uint32_t*>(o.gA + ((size_t(tb) * (n_in / 32) + step) * 64 + h * 32 + tt) * 16 +
                                         (lane & 3) * 4) = packed;
            const size_t blk = size_t(tb) * n_sb + c;
            if (lane == 0) o.gX[(blk * 2 + ((tt >> 2) & 1)) * 16 + (tt >> 3) * 4 + (tt & 3)] = d;
            if ((lane & 7) == 0) {
                const int g = lane >> 3;
                // 64 (bsum >> 6): a multiple of 64 of magnitude <= 4096, exact in f16
                o.gJ[(blk * 64 + tt) * 8 + g] = __builtin_bit_cast(uint16_t, _Float16(float((g32 >> 6) * 64)));
                o.gJ[(blk * 64 + 32 + tt) * 8 + g] = __builtin_bit_cast(uint16_t, _Float16(float(g32 & 63)));
            }
        }
        if (GEMM_ONLY || !real) return;
        if (o.q256) *reinterpret_cast<uint32_t*>(o.q256 + size_t(t) * n_in + k0) = packed;
        if (o.m256)
            *reinterpret_cast<uint32_t*>(o.m256 + size_t(t) * n_in + size_t(c) * 256 + mfma_offset(lane)) = packed;
        const size_t sb = size_t(t) * (n_in / 256) + c;
        if (lane == 0 && o.d256) o.d256[sb] = d;
        if ((lane & 3) == 0 && o.s16) o.s16[size_t(t) * (n_in / 16) + k0 / 16] = int16_t(g16);
        if ((lane & 7) == 0 && o.bsm) {
            const int g = lane >> 3;
            o.bsm[sb * 16 + g] = int8_t(g32 >> 6);      // arithmetic shift: floor(bsum / 64)
            o.bsm[sb * 16 + 8 + g] = int8_t(g32 & 63);
        }
        if (o.aos256) {
            uint8_t* b = o.aos256 + sb * 276;
            *reinterpret_cast<uint32_t*>(b + 20 + 4 * lane) = packed;
            if (lane == 0) *reinterpret_cast<float*>(b) = d;
            if ((lane & 7) == 0) *reinterpret_cast<int16_t*>(b + 4 + 2 * (lane >> 3)) = int16_t(g32);
        }
    }
}

// One wavefront per (token, run of CPW consecutive chunks): the run's loads are
// all issued before the first chunk is quantized, so each wavefront keeps
// CPW KB (2 CPW KB with u) in flight. With u the values quantized are
// act(x) * u (SiLU, or the tanh GELU when gelu is set), written to h_out when
// given; h_out may be x itself (each value is read and rewritten by one lane).
template <int CPW, bool GEMM_ONLY>
__global__ __launch_bounds__(256) void quantize_kernel(const float* x, int n_tok, int n_in, int ldx, QuantOut o,
                                                       const float* __restrict__ u, float* h_out, int gelu) {
    const int lane = threadIdx.x & 63;
    const int chunks = (n_in + 255) / 256, runs = (chunks + CPW - 1) / CPW;
    const long wave = long(blockIdx.x) * 4 + (threadIdx.x >> 6);
    // rows beyond n_tok (up to the next 32-token block) only zero-fill the gA/gX/gJ planes
    const int rows = o.gA ? (n_tok + 31) / 32 * 32 : n_tok;
    if (wave >= long(rows) * runs) return;
    const int t = int(wave / runs), c0 = int(wave % runs) * CPW;
    float4 v[CPW];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
        const int k0 = (c0 + j) * 256 + lane * 4;
        v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t < n_tok && c0 + j < chunks && k0 < n_in) v[j] = *reinterpret_cast<const float4*>(x + size_t(t) * ldx + k0);
    }
    if (u) {
        // every load of the run before the first store (h_out may be x)
        float4 w[CPW];
#pragma unroll
        for (int j = 0; j < CPW; ++j) {
            const int k0 = (c0 + j) * 256 + lane * 4;
            w[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (t < n_tok && c0 + j < chunks && k0 < n_in) w[j] = *reinterpret_cast<const float4*>(u + size_t(t) * ldx + k0);
        }
        const bool ge = gelu != 0;
#pragma unroll
        for (int j = 0; j < CPW; ++j) {
            const int k0 = (c0 + j) * 256 + lane * 4;
            if (t < n_tok && c0 + j < chunks && k0 < n_in) {
                v[j] = make_float4(act_mul(v[j].x, w[j].x, ge), act_mul(v[j].y, w[j].y, ge),
                                   act_mul(v[j].z, w[j].z, ge), act_mul(v[j].w, w[j].w, ge));
                if (h_out) *reinterpret_cast<float4*>(h_out + size_t(t) * n_in + k0) = v[j];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < CPW; ++j)
        if (c0 + j < chunks) quantize_chunk<GEMM_ONLY>(v[j], t, c0 + j, n_tok, n_in, o, lane);
}

}  // namespace

namespace {

// The outputs of act_layout L in `act` that `planes` asks for.
QuantOut quant_out(const ActLayout& L, void* act, void* aos32, void* aos256, unsigned planes) {
    uint8_t* b = static_cast<uint8_t*>(act);
    const bool gemv = planes & kPlanesGemv, b32 = planes & kPlanesBatch32;
    const bool b256 = L.has256 && (planes & kPlanesBatch256), gemm = L.has256 && (planes & kPlanesGemm);
    QuantOut o;
    o.q32 = gemv ? reinterpret_cast<int8_t*>(b + L.q32) : nullptr;
    o.d32 = (gemv || b32) ? reinterpret_cast<float*>(b + L.d32) : nullptr;
    o.s32 = gemv ? reinterpret_cast<int32_t*>(b + L.s32) : nullptr;
    o.q256 = (gemv && L.has256) ? reinterpret_cast<int8_t*>(b + L.q256) : nullptr;
    o.d256 = ((gemv && L.has256) || b256) ? reinterpret_cast<float*>(b + L.d256) : nullptr;
    o.s16 = (gemv && L.has256) ? reinterpret_cast<int16_t*>(b + L.s16) : nullptr;
    o.bsm = b256 ? reinterpret_cast<int8_t*>(b + L.bsm) : nullptr;
    o.m32 = (b32 && L.has256) ? reinterpret_cast<int8_t*>(b + L.m32) : nullptr;
    o.m256 = b256 ? reinterpret_cast<int8_t*>(b + L.m256) : nullptr;
    o.gA = gemm ? reinterpret_cast<int8_t*>(b + L.gA) : nullptr;
    o.gX = gemm ? reinterpret_cast<float*>(b + L.gX) : nullptr;
    o.gJ = gemm ? reinterpret_cast<uint16_t*>(b + L.gJ) : nullptr;
    o.aos32 = static_cast<uint8_t*>(aos32);
    o.aos256 = L.has256 ? static_cast<uint8_t*>(aos256) : nullptr;
    return o;
}

bool gemm_planes_only(const QuantOut& o) {
    return o.gA && !o.q32 && !o.d32 && !o.d256 && !o.bsm && !o.m32 && !o.m256 && !o.aos32 && !o.aos256;
}

// RMS norm of one token row, then its quantization, in one workgroup of
// kNormQTh threads: x += y (+ b) when y is given (written back), xn = x * scale
// * w with scale = 1 / sqrt(sum x^2 / n + eps), the sum in double over a
// tree of kNormQTh partial sums -- the steps and order of the layer span's
// rmsnorm kernel, each operation rounded on its own (no contraction) -- and
// xn, written out, is read back in 256-value chunks (wavefront w takes chunks
// w, w + 16, ...) and quantized as quantize_kernel does. Rows from n_tok up to
// the next 32-token block (GEMM planes) only zero-fill.
constexpr int kNormQTh = 1024;
template <bool GEMM_ONLY>
__global__ __launch_bounds__(kNormQTh) void rmsnorm_quantize_kernel(float* __restrict__ x, const float* __restrict__ y,
                                                                    const float* __restrict__ b,
                                                                    const float* __restrict__ w, float* xn, int n_tok,
                                                                    int n, float eps, QuantOut o) {
    __shared__ double red[kNormQTh];
    const int t = int(blockIdx.x), tid = int(threadIdx.x), lane = tid & 63, wv = tid >> 6;
    if (t < n_tok) {
        float* xr = x + size_t(t) * n;
        const float* yr = y ? y + size_t(t) * n : nullptr;
        float* orow = xn + size_t(t) * n;
        double sq = 0.0;
#pragma unroll 4
        for (int i = tid; i < n; i += kNormQTh) {
            float v = xr[i];
            if (yr) {
                v = __fadd_rn(v, b ? __fadd_rn(yr[i], b[i]) : yr[i]);
                xr[i] = v;
            } else if (b) {
                v = __fadd_rn(v, b[i]);
                xr[i] = v;
            }
            sq = __dadd_rn(sq, __dmul_rn(double(v), double(v)));
        }
        red[tid] = sq;
        __syncthreads();
        for (int st = kNormQTh / 2; st > 0; st >>= 1) {
            if (tid < st) red[tid] = __dadd_rn(red[tid], red[tid + st]);
            __syncthreads();
        }
        const float scale = 1.0f / sqrtf(__fadd_rn(float(red[0] / n), eps));
        for (int i = tid; i < n; i += kNormQTh) orow[i] = __fmul_rn(__fmul_rn(xr[i], scale), w[i]);
        __syncthreads();  // the row is written before its chunks are read back
    }
    const int chunks = (n + 255) / 256;
    const float* orow = xn + size_t(min(t, n_tok - 1)) * n;
    for (int c = wv; c < chunks; c += kNormQTh / 64) {
        const int k0 = c * 256 + lane * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t < n_tok && k0 < n) v = *reinterpret_cast<const float4*>(orow + k0);
        quantize_chunk<GEMM_ONLY>(v, t, c, n_tok, n, o, lane);
    }
}

}  // namespace

hipError_t launch_quantize(const float* x, int n_tok, int n_in, int ldx, void* act, void* aos32, void* aos256,
                           hipStream_t stream, unsigned planes, const float* u, float* h_out, bool gelu) {
    const ActLayout L = act_layout(n_tok, n_in);
    if (!L.total) return hipErrorInvalidValue;
    const QuantOut o = quant_out(L, act, aos32, aos256, planes);
    const bool gemm = o.gA != nullptr;
    const long rows = gemm ? L.n_tb * 32 : n_tok, chunks = (n_in + 255) / 256;
    // the GEMM's planes alone (a K-quant prefill): the kernel without the other layouts' code
    const bool gemm_only = gemm_planes_only(o);
    // four chunks per wavefront only for the largest launches (measured: 6 % faster at 512 x 14336;
    // at 64 x 4096 or 512 x 4096 one chunk per wavefront is faster, the chain per chunk dominating)
    if (rows * chunks >= 16384) {
        const unsigned blocks = unsigned((rows * ((chunks + 3) / 4) + 3) / 4);
        if (gemm_only)
            hipLaunchKernelGGL((quantize_kernel<4, true>), dim3(blocks), dim3(256), 0, stream, x, n_tok, n_in, ldx, o,
                               u, h_out, gelu ? 1 : 0);
        else
            hipLaunchKernelGGL((quantize_kernel<4, false>), dim3(blocks), dim3(256), 0, stream, x, n_tok, n_in, ldx,
                               o, u, h_out, gelu ? 1 : 0);
    } else {
        const unsigned blocks = unsigned((rows * chunks + 3) / 4);
        if (gemm_only)
            hipLaunchKernelGGL((quantize_kernel<1, true>), dim3(blocks), dim3(256), 0, stream, x, n_tok, n_in, ldx, o,
                               u, h_out, gelu ? 1 : 0);
        else
            hipLaunchKernelGGL((quantize_kernel<1, false>), dim3(blocks), dim3(256), 0, stream, x, n_tok, n_in, ldx,
                               o, u, h_out, gelu ? 1 : 0);
    }
    return hipGetLastError();
}

hipError_t launch_rmsnorm_quantize(float* x, const float* y, const float* b, const float* w, float* xn, int n_tok,
                                   int n, float eps, void* act, unsigned planes, hipStream_t stream) {
    const ActLayout L = act_layout(n_tok, n);
    if (!L.total || n % 4) return hipErrorInvalidValue;
    const QuantOut o = quant_out(L, act, nullptr, nullptr, planes);
    const unsigned rows = unsigned(o.gA ? L.n_tb * 32 : n_tok);
    if (gemm_planes_only(o))
        hipLaunchKernelGGL(rmsnorm_quantize_kernel<true>, dim3(rows), dim3(kNormQTh), 0, stream, x, y, b, w, xn, n_tok,
                           n, eps, o);
    else
        hipLaunchKernelGGL(rmsnorm_quantize_kernel<false>, dim3(rows), dim3(kNormQTh), 0, stream, x, y, b, w, xn, n_tok,
                           n, eps, o);
    return hipGetLastError();
}

}  // namespace fishhip
