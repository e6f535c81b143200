// Many-token matmul (prefill / batched experts) over repacked K-quant weights
// on gfx950 int8 MFMA with i32 accumulation.
//
// Arithmetic (same integers as FISH's dot_q4_K_q8k / dot_q6_K_q8k,
// quant_x86.cpp:346-382, :445-495), per output (token t, row i) and
// super-block sb of 256 values:
//   Q4_K  I = sum_g sc_g sum_l q x       J = sum_g m_g bsum_g
//         y += xd * (d * I - dmin * J)
//   Q6_K  I = sum_j sc_j sum_{16} (q - 32) x            y += d * xd * I
// The per-group integer scale makes w' = sc * q (Q4_K, 0..945) or
// sc * (q - 32) (Q6_K, -4064..4096) too wide for int8, so the dequantised
// weight tile is stored in LDS as two int8 planes, w' = 2^s * hi + lo
// (s = 5 for Q4_K, 6 for Q6_K; lo >= 0), and I = 2^s * (hi . x) + (lo . x)
// comes out of two i8 MFMA accumulators with no per-group VALU work. J is a
// K = 8 product per super-block; bsum = 64 * bh + bl (bh, bl int8, written
// by the quantizer) turns it into two small 32x32x16 i8 MFMAs.
//
// Tiling: a workgroup of 2 wavefronts owns 64 weight rows x 128 tokens; each
// wavefront owns 64 rows x 64 tokens as 2 x 2 blocks of 32 x 32
// (v_mfma_i32_32x32x32_i8). The K loop stages half a super-block (128 values)
// at a time in LDS: activation codes of the 128 tokens and the hi/lo planes
// of the 64 rows.
#include "common.h"
#include "kernels.h"

namespace fishhip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int BN = 64;        // weight rows per workgroup
constexpr int BM = 128;       // tokens per workgroup
constexpr int KS = 128;       // K values staged per step (4 groups of 32)
constexpr int P = KS + 16;    // LDS row pitch (bytes): 16-byte skew between rows

// Bytes 0 and 2 (even) or 1 and 3 (odd) of v as two 16-bit lanes.
__device__ __forceinline__ v2s bytes_even(uint32_t v) {
    return __builtin_bit_cast(v2s, v & 0x00FF00FFu);
}
__device__ __forceinline__ v2s bytes_odd(uint32_t v) {
    return __builtin_bit_cast(v2s, (v >> 8) & 0x00FF00FFu);
}

// Four unsigned codes (bytes of v) -> w' = sc * (code - off) split into
// (hi, lo) bytes with w' = 2^SHIFT * hi + lo, 0 <= lo < 2^SHIFT.
template <int SHIFT>
__device__ __forceinline__ void split4(uint32_t v, short off, short sc, uint32_t& hi, uint32_t& lo) {
    const v2s offv = {off, off}, scv = {sc, sc};
    const v2s we = (bytes_even(v) - offv) * scv;
    const v2s wo = (bytes_odd(v) - offv) * scv;
    const v2s he = we >> SHIFT, ho = wo >> SHIFT;
    const v2s mask = {short((1 << SHIFT) - 1), short((1 << SHIFT) - 1)};
    const v2s le = we & mask, lo2 = wo & mask;
    const uint32_t he32 = __builtin_bit_cast(uint32_t, he) & 0x00FF00FFu;
    const uint32_t ho32 = __builtin_bit_cast(uint32_t, ho) & 0x00FF00FFu;
    hi = he32 | (ho32 << 8);
    lo = __builtin_bit_cast(uint32_t, le) | (__builtin_bit_cast(uint32_t, lo2) << 8);
}

template <uint32_t T>
__global__ __launch_bounds__(128, 2) void gemm_kq_kernel(WeightPtrs W, ActPtrs A, int n_in, int n_out, int n_tok,
                                                         float* __restrict__ y, int ldy) {
    constexpr int SHIFT = (T == kQ4_K) ? 5 : 6;
    __shared__ __attribute__((aligned(16))) uint8_t s_act[BM * P];
    __shared__ __attribute__((aligned(16))) uint8_t s_hi[BN * P];
    __shared__ __attribute__((aligned(16))) uint8_t s_lo[BN * P];
    __shared__ float s_xd[BM];
    __shared__ __attribute__((aligned(16))) int8_t s_bsm[BM * 16];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;
    const int row0 = int(blockIdx.x) * BN, tok0 = int(blockIdx.y) * BM;
    const int wt0 = wave * 64;
    const int groups = n_in / 32, n_sb = n_in / 256;

    float facc[2][2][16];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) facc[a][b][r] = 0.0f;

    for (int s = 0; s < n_sb; ++s) {
        // f32 scales of this super-block for the lane's two rows; Q4_K mins as 8 bytes.
        float dR[2], dminR[2];
        uint64_t minsR[2];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            const int row = row0 + 32 * rb + l32;
            dR[rb] = 0.0f;
            dminR[rb] = 0.0f;
            minsR[rb] = 0;
            if (row < n_out) {
                if constexpr (T == kQ4_K) {
                    const uint4 m = *reinterpret_cast<const uint4*>(W.aux + (size_t(row) * n_sb + s) * 16);
                    dR[rb] = f16_bits_to_f32(uint16_t(m.x & 0xFFFF));
                    dminR[rb] = f16_bits_to_f32(uint16_t(m.x >> 16));
                    uint64_t mm = 0;
#pragma unroll
                    for (int g = 0; g < 8; ++g) {
                        int sc, mn;
                        k4_scale_min(m.y, m.z, m.w, g, sc, mn);
                        mm |= uint64_t(mn) << (8 * g);
                    }
                    minsR[rb] = mm;
                } else {
                    dR[rb] = f16_bits_to_f32(W.d[size_t(row) * n_sb + s]);
                }
            }
        }

        v16i cH[2][2], cL[2][2];
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    cH[a][b][r] = 0;
                    cL[a][b][r] = 0;
                }

        for (int h = 0; h < 2; ++h) {
            __syncthreads();  // the previous step's LDS reads are done
            // ---- activation codes: 128 tokens x 128 bytes
            {
                const int cb = (tid & 7) * 16;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int tl = (tid >> 3) + 16 * j, t = tok0 + tl;
                    uint4 v = make_uint4(0, 0, 0, 0);
                    if (t < n_tok)
                        v = *reinterpret_cast<const uint4*>(A.q256 + size_t(t) * n_in + size_t(s) * 256 + h * KS + cb);
                    *reinterpret_cast<uint4*>(s_act + tl * P + cb) = v;
                }
                if (h == 0) {
                    const int t = tok0 + tid;
                    float xd = 0.0f;
                    uint4 b = make_uint4(0, 0, 0, 0);
                    if (t < n_tok) {
                        xd = A.d256[size_t(t) * n_sb + s];
                        b = *reinterpret_cast<const uint4*>(A.bsm + (size_t(t) * n_sb + s) * 16);
                    }
                    s_xd[tid] = xd;
                    *reinterpret_cast<uint4*>(s_bsm + tid * 16) = b;
                }
            }
            // ---- weight planes: 64 rows x 4 groups, two (row, group) units per thread
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int u = tid + 128 * j, r = u >> 2, gl = u & 3;
                const int row = row0 + r, g = h * 4 + gl, c = s * 8 + g;
                uint4 hiA = make_uint4(0, 0, 0, 0), loA = hiA, hiB = hiA, loB = hiA;
                if (row < n_out) {
                    const uint4 w = *reinterpret_cast<const uint4*>(W.codes + (size_t(row) * groups + c) * 16);
                    uint4 nlo = make_uint4(w.x & 0x0F0F0F0Fu, w.y & 0x0F0F0F0Fu, w.z & 0x0F0F0F0Fu, w.w & 0x0F0F0F0Fu);
                    uint4 nhi = make_uint4((w.x >> 4) & 0x0F0F0F0Fu, (w.y >> 4) & 0x0F0F0F0Fu,
                                           (w.z >> 4) & 0x0F0F0F0Fu, (w.w >> 4) & 0x0F0F0F0Fu);
                    short sca, scb, off;
                    if constexpr (T == kQ4_K) {
                        const uint4 m = *reinterpret_cast<const uint4*>(W.aux + (size_t(row) * n_sb + s) * 16);
                        int sc, mn;
                        k4_scale_min(m.y, m.z, m.w, g, sc, mn);
                        sca = scb = short(sc);
                        off = 0;
                    } else {
                        const uint2 qh = *reinterpret_cast<const uint2*>(W.aux + (size_t(row) * groups + c) * 8);
                        nlo.x |= (qh.x & 0x03030303u) << 4;
                        nlo.y |= ((qh.x >> 2) & 0x03030303u) << 4;
                        nlo.z |= ((qh.x >> 4) & 0x03030303u) << 4;
                        nlo.w |= ((qh.x >> 6) & 0x03030303u) << 4;
                        nhi.x |= (qh.y & 0x03030303u) << 4;
                        nhi.y |= ((qh.y >> 2) & 0x03030303u) << 4;
                        nhi.z |= ((qh.y >> 4) & 0x03030303u) << 4;
                        nhi.w |= ((qh.y >> 6) & 0x03030303u) << 4;
                        const uint16_t s2 = *reinterpret_cast<const uint16_t*>(W.sc + size_t(row) * (n_in / 16) + 2 * c);
                        sca = short(int8_t(s2 & 0xFF));
                        scb = short(int8_t(s2 >> 8));
                        off = 32;
                    }
                    split4<SHIFT>(nlo.x, off, sca, hiA.x, loA.x);
                    split4<SHIFT>(nlo.y, off, sca, hiA.y, loA.y);
                    split4<SHIFT>(nlo.z, off, sca, hiA.z, loA.z);
                    split4<SHIFT>(nlo.w, off, sca, hiA.w, loA.w);
                    split4<SHIFT>(nhi.x, off, scb, hiB.x, loB.x);
                    split4<SHIFT>(nhi.y, off, scb, hiB.y, loB.y);
                    split4<SHIFT>(nhi.z, off, scb, hiB.z, loB.z);
                    split4<SHIFT>(nhi.w, off, scb, hiB.w, loB.w);
                }
                uint8_t* ph = s_hi + r * P + gl * 32;
                uint8_t* pl = s_lo + r * P + gl * 32;
                *reinterpret_cast<uint4*>(ph) = hiA;
                *reinterpret_cast<uint4*>(ph + 16) = hiB;
                *reinterpret_cast<uint4*>(pl) = loA;
                *reinterpret_cast<uint4*>(pl + 16) = loB;
            }
            __syncthreads();
            // ---- MFMA over the 4 staged groups
#pragma unroll
            for (int gl = 0; gl < 4; ++gl) {
                const int ko = gl * 32 + half * 16;
                v4i av[2], bh[2], bl[2];
#pragma unroll
                for (int tb = 0; tb < 2; ++tb)
                    av[tb] = *reinterpret_cast<const v4i*>(s_act + (wt0 + 32 * tb + l32) * P + ko);
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    bh[rb] = *reinterpret_cast<const v4i*>(s_hi + (32 * rb + l32) * P + ko);
                    bl[rb] = *reinterpret_cast<const v4i*>(s_lo + (32 * rb + l32) * P + ko);
                }
#pragma unroll
                for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                    for (int rb = 0; rb < 2; ++rb) {
                        cH[tb][rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[tb], bh[rb], cH[tb][rb], 0, 0, 0);
                        cL[tb][rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[tb], bl[rb], cL[tb][rb], 0, 0, 0);
                    }
            }
        }

        // ---- super-block epilogue. C layout (32x32 i32): lane l, register r
        // -> token 8*(r/4) + 4*(l/32) + r%4 of the block, row l%32.
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            long aj = 0;
            if constexpr (T == kQ4_K)
                aj = *reinterpret_cast<const long*>(s_bsm + (wt0 + 32 * tb + l32) * 16 + 8 * half);
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                v16i I;
#pragma unroll
                for (int r = 0; r < 16; ++r) I[r] = (cH[tb][rb][r] << SHIFT) + cL[tb][rb][r];
                if constexpr (T == kQ4_K) {
                    const long bjh = half ? 0 : long(minsR[rb]);
                    const long bjl = half ? long(minsR[rb]) : 0;
                    v16i J = {};
                    J = __builtin_amdgcn_mfma_i32_32x32x16_i8(aj, bjh, J, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) J[r] <<= 6;
                    J = __builtin_amdgcn_mfma_i32_32x32x16_i8(aj, bjl, J, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int tl = wt0 + 32 * tb + 8 * (r >> 2) + 4 * half + (r & 3);
                        facc[tb][rb][r] += s_xd[tl] * (dR[rb] * float(I[r]) - dminR[rb] * float(J[r]));
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int tl = wt0 + 32 * tb + 8 * (r >> 2) + 4 * half + (r & 3);
                        facc[tb][rb][r] += (dR[rb] * s_xd[tl]) * float(I[r]);
                    }
                }
            }
        }
    }

#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            const int row = row0 + 32 * rb + l32;
            if (row >= n_out) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = tok0 + wt0 + 32 * tb + 8 * (r >> 2) + 4 * half + (r & 3);
                if (t < n_tok) y[size_t(t) * ldy + row] = facc[tb][rb][r];
            }
        }
}

}  // namespace

hipError_t launch_gemm(const void* w, const WeightLayout& WL, const void* act, int n_tok, float* y, int ldy,
                       hipStream_t s) {
    const ActLayout AL = act_layout(n_tok, WL.n_in);
    if (!WL.total || !AL.total || !AL.has256 || n_tok <= 0) return hipErrorInvalidValue;
    const WeightPtrs W = weight_ptrs(w, WL);
    const ActPtrs A = act_ptrs(act, AL);
    const dim3 grid(unsigned((WL.n_out + BN - 1) / BN), unsigned((n_tok + BM - 1) / BM));
    switch (WL.type) {
        case kQ4_K:
            hipLaunchKernelGGL(gemm_kq_kernel<kQ4_K>, grid, dim3(128), 0, s, W, A, WL.n_in, WL.n_out, n_tok, y, ldy);
            break;
        case kQ6_K:
            hipLaunchKernelGGL(gemm_kq_kernel<kQ6_K>, grid, dim3(128), 0, s, W, A, WL.n_in, WL.n_out, n_tok, y, ldy);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace fishhip
