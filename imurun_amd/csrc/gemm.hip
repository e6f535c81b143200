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
// (s = 5 for Q4_K, 6 for Q6_K; 0 <= lo < 2^s), and I = 2^s * (hi . x) +
// (lo . x) comes out of two i8 MFMA accumulators with no per-group VALU
// work. J is a K = 8 product per super-block; bsum = 64 * bh + bl (bh, bl
// int8, written by the quantizer) turns it into two small 32x32x16 MFMAs.
//
// Tiling: a workgroup of 4 wavefronts owns BN weight rows x BM tokens
// (BN * BM = 4 * 64 * 64); each wavefront owns 64 rows x 64 tokens as 2 x 2
// blocks of 32 x 32 (v_mfma_i32_32x32x32_i8). K advances 64 values (two
// groups) per step through double-buffered LDS: while the MFMAs of step k
// run, the global loads of step k+1 are in flight, and the weights of step
// k+1 are dequantised into the hi/lo planes once for all BM tokens.
#include "common.h"
#include "kernels.h"

namespace fishhip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int KS = 64;       // K values per step (two 32-groups)
constexpr int P = KS + 16;   // LDS row pitch in bytes (16-byte skew: conflict-free 128-bit reads)

__device__ __forceinline__ v2s bytes_even(uint32_t v) { return __builtin_bit_cast(v2s, v & 0x00FF00FFu); }
__device__ __forceinline__ v2s bytes_odd(uint32_t v) { return __builtin_bit_cast(v2s, (v >> 8) & 0x00FF00FFu); }

// Four unsigned codes (bytes of v) -> w' = sc * (code - off) split into
// (hi, lo) bytes with w' = 2^SHIFT * hi + lo, 0 <= lo < 2^SHIFT.
template <int SHIFT>
__device__ __forceinline__ void split4(uint32_t v, v2s offv, v2s scv, uint32_t& hi, uint32_t& lo) {
    const v2s we = (bytes_even(v) - offv) * scv;
    const v2s wo = (bytes_odd(v) - offv) * scv;
    const v2s he = we >> SHIFT, ho = wo >> SHIFT;
    const v2s mask = {short((1 << SHIFT) - 1), short((1 << SHIFT) - 1)};
    const uint32_t he32 = __builtin_bit_cast(uint32_t, he) & 0x00FF00FFu;
    const uint32_t ho32 = __builtin_bit_cast(uint32_t, ho) & 0x00FF00FFu;
    hi = he32 | (ho32 << 8);
    lo = __builtin_bit_cast(uint32_t, we & mask) | (__builtin_bit_cast(uint32_t, wo & mask) << 8);
}

// Global data of one step held in registers between its load and its LDS write.
template <int BN, int BM>
struct Stage {
    static constexpr int A_VECS = BM * KS / 16 / 256;   // uint4 of activation codes per thread
    static constexpr int W_HALVES = BN * 4 / 256;       // half-groups (16 values) per thread
    uint4 act[A_VECS];
    uint4 codes[W_HALVES];
    uint32_t qh[W_HALVES];
    int sc[W_HALVES];
    float xd;      // first step of a super-block: this thread's token scale
    uint4 bsm;     // and its bsum split (Q4_K)
};

template <uint32_t T, int BN, int BM>
__global__ __launch_bounds__(256, 1) void gemm_kq_kernel(WeightPtrs W, ActPtrs A, int n_in, int n_out, int n_tok,
                                                         float* __restrict__ y, int ldy) {
    constexpr int SHIFT = (T == kQ4_K) ? 5 : 6;
    constexpr int WN = BN / 64;  // wavefronts along rows
    using S = Stage<BN, BM>;
    __shared__ __attribute__((aligned(16))) uint8_t s_act[2][BM * P];
    __shared__ __attribute__((aligned(16))) uint8_t s_hi[2][BN * P];
    __shared__ __attribute__((aligned(16))) uint8_t s_lo[2][BN * P];
    __shared__ float s_xd[2][BM];
    __shared__ __attribute__((aligned(16))) int8_t s_bsm[2][BM * 16];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;
    const int row0 = int(blockIdx.x) * BN, tok0 = int(blockIdx.y) * BM;
    const int wr0 = (wave % WN) * 64;  // wavefront's rows within the tile
    const int wt0 = (wave / WN) * 64;  // wavefront's tokens within the tile
    const int groups = n_in / 32, n_sb = n_in / 256;
    const int steps = n_in / KS;
    constexpr int SPS = 256 / KS;  // steps per super-block

    // ---- global -> registers for step k
    auto load_stage = [&](int k, S& st) {
        const int sb = k / SPS;
#pragma unroll
        for (int j = 0; j < S::A_VECS; ++j) {
            const int idx = tid + 256 * j;           // 16-byte chunk of the BM x KS tile
            const int tl = idx / (KS / 16), cb = (idx % (KS / 16)) * 16;
            const int t = tok0 + tl;
            st.act[j] = make_uint4(0, 0, 0, 0);
            if (t < n_tok) st.act[j] = *reinterpret_cast<const uint4*>(A.q256 + size_t(t) * n_in + size_t(k) * KS + cb);
        }
#pragma unroll
        for (int j = 0; j < S::W_HALVES; ++j) {
            const int u = tid + 256 * j;              // (row, group-in-step, half)
            const int r = u >> 2, gl = (u >> 1) & 1, h = u & 1;
            const int row = row0 + r, c = k * 2 + gl;
            st.codes[j] = make_uint4(0, 0, 0, 0);
            st.qh[j] = 0;
            st.sc[j] = 0;
            if (row < n_out) {
                st.codes[j] = *reinterpret_cast<const uint4*>(W.codes + (size_t(row) * groups + c) * 16);
                if constexpr (T == kQ4_K) {
                    const uint4 m = *reinterpret_cast<const uint4*>(W.aux + (size_t(row) * n_sb + sb) * 16);
                    int scv, mn;
                    k4_scale_min(m.y, m.z, m.w, c & 7, scv, mn);
                    st.sc[j] = scv;
                } else {
                    st.qh[j] = *reinterpret_cast<const uint32_t*>(W.aux + (size_t(row) * groups + c) * 8 + 4 * h);
                    st.sc[j] = int(W.sc[size_t(row) * (n_in / 16) + 2 * c + h]);
                }
            }
        }
        if (k % SPS == 0 && tid < BM) {
            const int t = tok0 + tid;
            st.xd = 0.0f;
            st.bsm = make_uint4(0, 0, 0, 0);
            if (t < n_tok) {
                st.xd = A.d256[size_t(t) * n_sb + sb];
                if constexpr (T == kQ4_K)
                    st.bsm = *reinterpret_cast<const uint4*>(A.bsm + (size_t(t) * n_sb + sb) * 16);
            }
        }
    };

    // ---- registers -> LDS buffer b (weights dequantised to the hi/lo planes)
    auto store_stage = [&](int k, const S& st, int b) {
#pragma unroll
        for (int j = 0; j < S::A_VECS; ++j) {
            const int idx = tid + 256 * j;
            const int tl = idx / (KS / 16), cb = (idx % (KS / 16)) * 16;
            *reinterpret_cast<uint4*>(&s_act[b][tl * P + cb]) = st.act[j];
        }
#pragma unroll
        for (int j = 0; j < S::W_HALVES; ++j) {
            const int u = tid + 256 * j;
            const int r = u >> 2, gl = (u >> 1) & 1, h = u & 1;
            const uint4 w = st.codes[j];
            uint4 n;  // the 16 codes of this half, element order
            if (h == 0) n = make_uint4(w.x & 0x0F0F0F0Fu, w.y & 0x0F0F0F0Fu, w.z & 0x0F0F0F0Fu, w.w & 0x0F0F0F0Fu);
            else n = make_uint4((w.x >> 4) & 0x0F0F0F0Fu, (w.y >> 4) & 0x0F0F0F0Fu, (w.z >> 4) & 0x0F0F0F0Fu,
                                (w.w >> 4) & 0x0F0F0F0Fu);
            short off = 0;
            if constexpr (T == kQ6_K) {
                const uint32_t q = st.qh[j];
                n.x |= (q & 0x03030303u) << 4;
                n.y |= ((q >> 2) & 0x03030303u) << 4;
                n.z |= ((q >> 4) & 0x03030303u) << 4;
                n.w |= ((q >> 6) & 0x03030303u) << 4;
                off = 32;
            }
            const v2s offv = {off, off}, scv = {short(st.sc[j]), short(st.sc[j])};
            uint4 hi, lo;
            split4<SHIFT>(n.x, offv, scv, hi.x, lo.x);
            split4<SHIFT>(n.y, offv, scv, hi.y, lo.y);
            split4<SHIFT>(n.z, offv, scv, hi.z, lo.z);
            split4<SHIFT>(n.w, offv, scv, hi.w, lo.w);
            *reinterpret_cast<uint4*>(&s_hi[b][r * P + gl * 32 + h * 16]) = hi;
            *reinterpret_cast<uint4*>(&s_lo[b][r * P + gl * 32 + h * 16]) = lo;
        }
        if (k % SPS == 0 && tid < BM) {
            const int p = (k / SPS) & 1;
            s_xd[p][tid] = st.xd;
            *reinterpret_cast<uint4*>(&s_bsm[p][tid * 16]) = st.bsm;
        }
    };

    float facc[2][2][16];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) facc[a][c][r] = 0.0f;
    v16i cH[2][2], cL[2][2];

    S st;
    load_stage(0, st);
    store_stage(0, st, 0);
    __syncthreads();

    for (int k = 0; k < steps; ++k) {
        const int b = k & 1;
        if (k % SPS == 0) {
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    cH[a][c] = v16i{};
                    cL[a][c] = v16i{};
                }
        }
        if (k + 1 < steps) load_stage(k + 1, st);  // in flight during the MFMAs below

#pragma unroll
        for (int gl = 0; gl < 2; ++gl) {
            const int ko = gl * 32 + half * 16;
            v4i av[2], bh[2], bl[2];
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
                av[tb] = *reinterpret_cast<const v4i*>(&s_act[b][(wt0 + 32 * tb + l32) * P + ko]);
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                bh[rb] = *reinterpret_cast<const v4i*>(&s_hi[b][(wr0 + 32 * rb + l32) * P + ko]);
                bl[rb] = *reinterpret_cast<const v4i*>(&s_lo[b][(wr0 + 32 * rb + l32) * P + ko]);
            }
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    cH[tb][rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[tb], bh[rb], cH[tb][rb], 0, 0, 0);
                    cL[tb][rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[tb], bl[rb], cL[tb][rb], 0, 0, 0);
                }
        }

        if (k % SPS == SPS - 1) {
            // super-block epilogue. C layout (32x32 i32): lane l, register r
            // -> token 8*(r/4) + 4*(l/32) + r%4 of the block, row l%32.
            const int sb = k / SPS, p = sb & 1;
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                const int row = row0 + wr0 + 32 * rb + l32;
                float d = 0.0f, dmin = 0.0f;
                uint64_t mins = 0;
                if (row < n_out) {
                    if constexpr (T == kQ4_K) {
                        const uint4 m = *reinterpret_cast<const uint4*>(W.aux + (size_t(row) * n_sb + sb) * 16);
                        d = f16_bits_to_f32(uint16_t(m.x & 0xFFFF));
                        dmin = f16_bits_to_f32(uint16_t(m.x >> 16));
#pragma unroll
                        for (int g = 0; g < 8; ++g) {
                            int scv, mn;
                            k4_scale_min(m.y, m.z, m.w, g, scv, mn);
                            mins |= uint64_t(mn) << (8 * g);
                        }
                    } else {
                        d = f16_bits_to_f32(W.d[size_t(row) * n_sb + sb]);
                    }
                }
#pragma unroll
                for (int tb = 0; tb < 2; ++tb) {
                    v16i I;
#pragma unroll
                    for (int r = 0; r < 16; ++r) I[r] = (cH[tb][rb][r] << SHIFT) + cL[tb][rb][r];
                    if constexpr (T == kQ4_K) {
                        const long aj = *reinterpret_cast<const long*>(&s_bsm[p][(wt0 + 32 * tb + l32) * 16 + 8 * half]);
                        const long bjh = half ? 0 : long(mins);
                        const long bjl = half ? long(mins) : 0;
                        v16i J = __builtin_amdgcn_mfma_i32_32x32x16_i8(aj, bjh, v16i{}, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; ++r) J[r] <<= 6;
                        J = __builtin_amdgcn_mfma_i32_32x32x16_i8(aj, bjl, J, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int tl = wt0 + 32 * tb + 8 * (r >> 2) + 4 * half + (r & 3);
                            facc[tb][rb][r] += s_xd[p][tl] * (d * float(I[r]) - dmin * float(J[r]));
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int tl = wt0 + 32 * tb + 8 * (r >> 2) + 4 * half + (r & 3);
                            facc[tb][rb][r] += (d * s_xd[p][tl]) * float(I[r]);
                        }
                    }
                }
            }
        }

        if (k + 1 < steps) store_stage(k + 1, st, b ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            const int row = row0 + wr0 + 32 * rb + l32;
            if (row >= n_out) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = tok0 + wt0 + 32 * tb + 8 * (r >> 2) + 4 * half + (r & 3);
                if (t < n_tok) y[size_t(t) * ldy + row] = facc[tb][rb][r];
            }
        }
}

template <uint32_t T, int BN, int BM>
hipError_t gemm_launch(const WeightPtrs& W, const ActPtrs& A, int n_in, int n_out, int n_tok, float* y, int ldy,
                       hipStream_t s) {
    const dim3 grid(unsigned((n_out + BN - 1) / BN), unsigned((n_tok + BM - 1) / BM));
    hipLaunchKernelGGL((gemm_kq_kernel<T, BN, BM>), grid, dim3(256), 0, s, W, A, n_in, n_out, n_tok, y, ldy);
    return hipGetLastError();
}

// Tile choice: 64 rows x 256 tokens shares each dequantised weight tile with
// the most tokens; 128 x 128 when that would leave too few workgroups.
template <uint32_t T>
hipError_t gemm_pick(const WeightPtrs& W, const ActPtrs& A, int n_in, int n_out, int n_tok, float* y, int ldy,
                     hipStream_t s) {
    const long wide = long((n_out + 63) / 64) * ((n_tok + 255) / 256);
    if (n_tok > 128 && wide >= 384) return gemm_launch<T, 64, 256>(W, A, n_in, n_out, n_tok, y, ldy, s);
    return gemm_launch<T, 128, 128>(W, A, n_in, n_out, n_tok, y, ldy, s);
}

}  // namespace

hipError_t launch_gemm(const void* w, const WeightLayout& WL, const void* act, int n_tok, float* y, int ldy,
                       hipStream_t s) {
    const ActLayout AL = act_layout(n_tok, WL.n_in);
    if (!WL.total || !AL.total || !AL.has256 || n_tok <= 0) return hipErrorInvalidValue;
    const WeightPtrs W = weight_ptrs(w, WL);
    const ActPtrs A = act_ptrs(act, AL);
    switch (WL.type) {
        case kQ4_K: return gemm_pick<kQ4_K>(W, A, WL.n_in, WL.n_out, n_tok, y, ldy, s);
        case kQ6_K: return gemm_pick<kQ6_K>(W, A, WL.n_in, WL.n_out, n_tok, y, ldy, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace fishhip
