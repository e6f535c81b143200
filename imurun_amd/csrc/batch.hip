// Few-token matmul on int8 MFMA: batches of up to a few dozen tokens and
// expert work-list items (matmul_batch, ops.cpp:177-216; the grouped expert
// products of model.cpp:1563-1572).
//
// One v_mfma_i32_16x16x32_i8 forms the exact integer dot of one 32-element
// group for 16 tokens x 16 weight rows:
//   A (activations): lane l supplies token l % 16, eight codes;
//   B (weights):     lane l supplies row   l % 16, the same eight elements;
//   D:               lane l holds row l % 16 of tokens 4 (l / 16) + r, r < 4.
// Lane quarter q = l / 16 takes elements 4q..4q+3 and 16+4q..16+4q+3 of the
// group, which is dword q of a repacked 16-byte nibble chunk (low nibbles,
// then high nibbles) and dwords q and 4+q of a Q8_0 group. The quantizer
// writes the activation codes in exactly that order (the m32 / m256 planes),
// so a lane's activation operands for a 256-element unit are 64 contiguous
// bytes. The weights keep the layout the GEMV streams; a lane loads 32 (Q8_0:
// 64) contiguous bytes of its row per unit and a 4x4 dword transpose across
// the four lane quarters (v_permlane32_swap + v_permlane16_swap, register
// only) hands every lane its dword of each group. Every load instruction thus
// covers whole 16-byte pieces of 16 rows or tokens.
//
// Because a lane's outputs all belong to one weight row, every per-row group
// scale is a lane scalar: Q4_K's sc_g and Q6_K's two 16-element scales are
// applied in exact int32 (sum_g sc_g * dot_g), Q4_K's mins term
// sum_g m_g * bsum_g is two more MFMAs on the split activation sums
// (bsum = 64 * bh + bl, both int8), and the f32 scales are applied once per
// 32-group (Q8_0, Q4_0) or 256-block (K-quants), as in FISH's AVX2 kernels
// (quant_x86.cpp:280-309, :346-382, :445-495).
//
// Q4_0 nibbles and Q6_K codes are made signed per byte without carries:
// (n + 0x78) ^ 0x80 = n - 8 for n in 0..15, (q + 0x60) ^ 0x80 = q - 32 for
// q in 0..63, so the MFMA sums are exactly FISH's sum (n - 8) x and
// sum (q - 32) x.
//
// Workgroup: four wavefronts, each RB blocks of 16 rows x NB blocks of 16
// tokens. The four either split the 256-element units of K (KS = 4; partial
// sums reduced through LDS in a fixed order) or take four different row
// ranges (KS = 1). Weights and activations of the next unit are in flight
// while the current unit's MFMAs run.
#include "common.h"
#include "kernels.h"

namespace fishhip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma16(long a, long b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) {
    return static_cast<long>((static_cast<unsigned long>(hi) << 32) | lo);
}

__device__ __forceinline__ uint32_t nib_lo(uint32_t w) { return w & 0x0F0F0F0Fu; }
__device__ __forceinline__ uint32_t nib_hi(uint32_t w) { return (w >> 4) & 0x0F0F0F0Fu; }
__device__ __forceinline__ uint32_t minus8(uint32_t n) { return (n + 0x78787878u) ^ 0x80808080u; }
__device__ __forceinline__ uint32_t minus32(uint32_t n) { return (n + 0x60606060u) ^ 0x80808080u; }

__device__ __forceinline__ float half_at(const uint4& v, int i) {
    const uint32_t w = (i < 2) ? v.x : (i < 4) ? v.y : (i < 6) ? v.z : v.w;
    return f16_bits_to_f32(uint16_t((i & 1) ? (w >> 16) : (w & 0xFFFF)));
}

__device__ __forceinline__ uint32_t dword_at(const uint4& v, int i) {
    return (i == 0) ? v.x : (i == 1) ? v.y : (i == 2) ? v.z : v.w;
}

__device__ __forceinline__ int byte_u(uint32_t w, int b) { return int((w >> (8 * b)) & 0xFF); }
__device__ __forceinline__ int byte_s(uint32_t w, int b) { return int(int8_t((w >> (8 * b)) & 0xFF)); }

// In-register 4x4 dword transpose across the lane quarters: on entry, quarter
// q holds row q of the matrix in v.x..v.w; on exit component k of quarter q
// holds element (k, q). permlane32_swap exchanges quarters 2,3 of its first
// operand with quarters 0,1 of its second; permlane16_swap exchanges the odd
// quarters of the first with the even quarters of the second.
__device__ __forceinline__ uint4 transpose4(uint4 v) {
    const auto a = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    return make_uint4(c[0], c[1], d[0], d[1]);
}

// Raw weight data of one 256-element unit for one 16-row block (the lane's row).
struct WUnit {
    uint4 v[4];     // codes: Q4 layouts chunks 2q, 2q+1 (v[0..1]); Q8_0 groups 2q, 2q+1 (v[0..3])
    uint4 m;        // Q8_0/Q4_0: 8 f16 group scales; Q4_K: d, dmin, scales; Q6_K: 16 int8 scales
    uint4 qh[4];    // Q6_K: high bits of the 8 groups (8 bytes each)
    uint32_t d6;    // Q6_K: f16 d
};

// Activation data of one unit for one 16-token block.
struct AUnit {
    uint4 v[4];      // codes in MFMA order: groups 2i, 2i+1 in v[i] (8 bytes each)
    float da[4][8];  // Q8_0/Q4_0: Q8Act d of output token r, group g
    float dk[4];     // K-quants: Q8ActK d of output token r
    uint2 bs;        // Q4_K: quarter 0 bh bytes, quarter 1 bl bytes, else 0
};

template <uint32_t T>
__device__ __forceinline__ void load_w(WUnit& o, const WeightPtrs& W, size_t row, int u, int q, int n_in) {
    const int groups = n_in / 32, units = n_in / 256;
    const int c0 = 8 * u;
    if constexpr (T == kQ8_0) {
        const uint4* p = reinterpret_cast<const uint4*>(W.codes + row * size_t(n_in) + size_t(u) * 256 + 64 * q);
#pragma unroll
        for (int i = 0; i < 4; ++i) o.v[i] = p[i];
        o.m = *reinterpret_cast<const uint4*>(W.d + row * groups + c0);
    } else {
        const uint4* p = reinterpret_cast<const uint4*>(W.codes + (row * groups + c0 + 2 * q) * 16);
        o.v[0] = p[0];
        o.v[1] = p[1];
        if constexpr (T == kQ4_0) {
            o.m = *reinterpret_cast<const uint4*>(W.d + row * groups + c0);
        } else if constexpr (T == kQ4_K) {
            o.m = *reinterpret_cast<const uint4*>(W.aux + (row * units + u) * 16);
        } else {
            const uint4* h = reinterpret_cast<const uint4*>(W.aux + (row * groups + c0) * 8);
#pragma unroll
            for (int i = 0; i < 4; ++i) o.qh[i] = h[i];
            o.m = *reinterpret_cast<const uint4*>(W.sc + row * size_t(n_in / 16) + 16 * u);
            o.d6 = W.d[row * units + u];
        }
    }
}

// arow_a: activation row of the lane's A token; arow_o[r]: rows of its output tokens.
template <uint32_t T>
__device__ __forceinline__ void load_a(AUnit& o, const ActPtrs& A, int arow_a, const int (&arow_o)[4], int u, int q,
                                       int n_in) {
    const int groups = n_in / 32, units = n_in / 256;
    constexpr bool kq = (T == kQ4_K || T == kQ6_K);
    const uint4* p = reinterpret_cast<const uint4*>((kq ? A.m256 : A.m32) + size_t(arow_a) * n_in + size_t(u) * 256 +
                                                    64 * q);
#pragma unroll
    for (int i = 0; i < 4; ++i) o.v[i] = p[i];
    if constexpr (!kq) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float4* d = reinterpret_cast<const float4*>(A.d32 + size_t(arow_o[r]) * groups + 8 * u);
            const float4 a = d[0], b = d[1];
            o.da[r][0] = a.x; o.da[r][1] = a.y; o.da[r][2] = a.z; o.da[r][3] = a.w;
            o.da[r][4] = b.x; o.da[r][5] = b.y; o.da[r][6] = b.z; o.da[r][7] = b.w;
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) o.dk[r] = A.d256[size_t(arow_o[r]) * units + u];
        if constexpr (T == kQ4_K) {
            o.bs = (q < 2) ? *reinterpret_cast<const uint2*>(A.bsm + (size_t(arow_a) * units + u) * 16 + 8 * q)
                           : make_uint2(0u, 0u);
        }
    }
}

__device__ __forceinline__ long a_operand(const AUnit& a, int g) {
    const uint4& v = a.v[g >> 1];
    return (g & 1) ? pack2(v.z, v.w) : pack2(v.x, v.y);
}

// acc[nb][r] += contribution of one unit of one row block for NB token blocks.
template <uint32_t T, int NB>
__device__ __forceinline__ void unit_dot(const WUnit& w, const AUnit (&a)[NB], int q, float (&acc)[NB][4]) {
    // the lane's B operand dwords of the 8 groups (Q8_0: lo = dword q, hi = dword 4+q)
    uint32_t lo[8], hi[8];
    if constexpr (T == kQ8_0) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint4 l = transpose4(w.v[2 * c]), h = transpose4(w.v[2 * c + 1]);
            lo[c] = l.x; lo[2 + c] = l.y; lo[4 + c] = l.z; lo[6 + c] = l.w;
            hi[c] = h.x; hi[2 + c] = h.y; hi[4 + c] = h.z; hi[6 + c] = h.w;
        }
    } else {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint4 t = transpose4(w.v[c]);
            lo[c] = t.x; lo[2 + c] = t.y; lo[4 + c] = t.z; lo[6 + c] = t.w;
        }
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            hi[g] = nib_hi(lo[g]);
            lo[g] = nib_lo(lo[g]);
        }
    }

    if constexpr (T == kQ8_0 || T == kQ4_0) {
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const long b = (T == kQ8_0) ? pack2(lo[g], hi[g]) : pack2(minus8(lo[g]), minus8(hi[g]));
            const float dw = half_at(w.m, g);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const v4i c = mfma16(a_operand(a[nb], g), b);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[nb][r] += float(c[r]) * (dw * a[nb].da[r][g]);
            }
        }
    } else if constexpr (T == kQ4_K) {
        const float d = f16_bits_to_f32(uint16_t(w.m.x & 0xFFFF));
        const float dmin = f16_bits_to_f32(uint16_t(w.m.x >> 16));
        const uint32_t sc_lo = w.m.y & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (w.m.w & 0x0F0F0F0Fu) | ((w.m.y >> 2) & 0x30303030u);
        const uint32_t mn_lo = w.m.z & 0x3F3F3F3Fu;
        const uint32_t mn_hi = ((w.m.w >> 4) & 0x0F0F0F0Fu) | ((w.m.z >> 2) & 0x30303030u);
        int isum[NB][4];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) isum[nb][r] = 0;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const long b = pack2(lo[g], hi[g]);
            const int sc = byte_u(g < 4 ? sc_lo : sc_hi, g & 3);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const v4i c = mfma16(a_operand(a[nb], g), b);
#pragma unroll
                for (int r = 0; r < 4; ++r) isum[nb][r] += sc * c[r];
            }
        }
        const long m8 = pack2(mn_lo, mn_hi);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const long bsv = pack2(a[nb].bs.x, a[nb].bs.y);
            const v4i ch = mfma16(bsv, q == 0 ? m8 : 0L);
            const v4i cl = mfma16(bsv, q == 1 ? m8 : 0L);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int mins = 64 * ch[r] + cl[r];
                acc[nb][r] += a[nb].dk[r] * (d * float(isum[nb][r]) - dmin * float(mins));
            }
        }
    } else {
        const float d = f16_bits_to_f32(uint16_t(w.d6));
        int isum[NB][4];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) isum[nb][r] = 0;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint4& h2 = w.qh[g >> 1];
            const uint32_t qa = (g & 1) ? h2.z : h2.x, qb = (g & 1) ? h2.w : h2.y;
            const uint32_t ca = minus32(lo[g] | (((qa >> (2 * q)) & 0x03030303u) << 4));
            const uint32_t cb = minus32(hi[g] | (((qb >> (2 * q)) & 0x03030303u) << 4));
            const uint32_t s2 = dword_at(w.m, g >> 1);
            const int sa = byte_s(s2, 2 * (g & 1)), sb = byte_s(s2, 2 * (g & 1) + 1);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const long av = a_operand(a[nb], g);
                const v4i xa = mfma16(av, pack2(ca, 0u));
                const v4i xb = mfma16(av, pack2(0u, cb));
#pragma unroll
                for (int r = 0; r < 4; ++r) isum[nb][r] += sa * xa[r] + sb * xb[r];
            }
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[nb][r] += (d * a[nb].dk[r]) * float(isum[nb][r]);
    }
}

template <uint32_t T, int RB, int NB, int KS>
__global__ __launch_bounds__(256) void batch_mfma_kernel(WeightPtrs W, ActPtrs A, int n_in, int n_out, int n_tok,
                                                         TokenMap map, float* __restrict__ y, int ldy) {
    constexpr int RG = 4 / KS;        // row ranges per workgroup
    constexpr int ROWS = 16 * RB;     // rows per wavefront
    constexpr int TOK = 16 * NB;      // tokens per workgroup
    __shared__ float red[KS > 1 ? 256 * RB * NB * 4 : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rg = wave / KS, ks = wave % KS;
    const int j = lane & 15, q = lane >> 4;
    const int units = n_in / 256;

    int s0, cnt;
    size_t wrow0 = 0;
    if (map.items) {
        const int it = int(blockIdx.y);
        if (it >= *map.n_items) return;  // uniform over the workgroup
        wrow0 = size_t(map.items[3 * it]) * size_t(n_out);
        s0 = map.items[3 * it + 1];
        cnt = map.items[3 * it + 2];
    } else {
        s0 = int(blockIdx.y) * TOK;
        cnt = min(TOK, n_tok - s0);
    }
    auto arow_of = [&](int t) {
        const int tt = (t < cnt) ? t : 0;
        return map.act_row ? map.act_row[s0 + tt] : s0 + tt;
    };
    int arow_a[NB], arow_o[NB][4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        arow_a[nb] = arow_of(16 * nb + j);
#pragma unroll
        for (int r = 0; r < 4; ++r) arow_o[nb][r] = arow_of(16 * nb + 4 * q + r);
    }
    const int row0 = (int(blockIdx.x) * RG + rg) * ROWS;
    size_t wrow[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) wrow[rb] = wrow0 + size_t(min(row0 + rb * 16 + j, n_out - 1));

    float acc[RB][NB][4];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[rb][nb][r] = 0.0f;

    const bool busy = row0 < n_out;
    if (busy) {
        WUnit w0[RB], w1[RB];
        AUnit a0[NB], a1[NB];
        auto load = [&](WUnit (&w)[RB], AUnit (&a)[NB], int u) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) load_w<T>(w[rb], W, wrow[rb], u, q, n_in);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) load_a<T>(a[nb], A, arow_a[nb], arow_o[nb], u, q, n_in);
        };
        auto compute = [&](const WUnit (&w)[RB], const AUnit (&a)[NB]) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) unit_dot<T, NB>(w[rb], a, q, acc[rb]);
        };
        int u = ks;
        if (u < units) load(w0, a0, u);
        while (u < units) {
            if (u + KS < units) load(w1, a1, u + KS);
            compute(w0, a0);
            u += KS;
            if (u >= units) break;
            if (u + KS < units) load(w0, a0, u + KS);
            compute(w1, a1);
            u += KS;
        }
    }

    if constexpr (KS > 1) {
        // k-split partial sums: wavefronts ks > 0 park theirs, ks == 0 adds them in order
        constexpr int PER = RB * NB * 4;
        if (ks > 0) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) red[(wave * PER + (rb * NB + nb) * 4 + r) * 64 + lane] = acc[rb][nb][r];
        }
        __syncthreads();
        if (ks > 0) return;
#pragma unroll
        for (int k = 1; k < KS; ++k)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[rb][nb][r] += red[((wave + k) * PER + (rb * NB + nb) * 4 + r) * 64 + lane];
    }
    if (!busy) return;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int row = row0 + rb * 16 + j;
        if (row >= n_out) continue;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * nb + 4 * q + r;
                if (t < cnt) y[size_t(s0 + t) * ldy + row] = acc[rb][nb][r];
            }
    }
}

template <uint32_t T, int RB, int NB, int KS>
hipError_t batch_launch(const WeightPtrs& W, const ActPtrs& A, int n_in, int n_out, int n_tok, const TokenMap& map,
                        int y_blocks, float* y, int ldy, hipStream_t s) {
    constexpr int ROWS_WG = 16 * RB * (4 / KS), TOK = 16 * NB;
    const unsigned gy = map.items ? unsigned(y_blocks) : unsigned((n_tok + TOK - 1) / TOK);
    const dim3 grid(unsigned((n_out + ROWS_WG - 1) / ROWS_WG), gy);
    hipLaunchKernelGGL((batch_mfma_kernel<T, RB, NB, KS>), grid, dim3(256), 0, s, W, A, n_in, n_out, n_tok, map, y,
                       ldy);
    return hipGetLastError();
}

#define BATCH_ARGS W, A, n_in, n_out, n_tok, map, y_blocks, y, ldy, s
#define BATCH_PARAMS                                                                                              \
    const WeightPtrs &W, const ActPtrs &A, int n_in, int n_out, int n_tok, const TokenMap &map, int y_blocks, \
        float *y, int ldy, hipStream_t s

// K split four ways when every wavefront still gets >= 2 units, else four row ranges.
template <uint32_t T, int RB, int NB>
hipError_t batch_pick_ks(BATCH_PARAMS) {
    if (n_in / 256 >= 8) return batch_launch<T, RB, NB, 4>(BATCH_ARGS);
    return batch_launch<T, RB, NB, 1>(BATCH_ARGS);
}

template <uint32_t T>
hipError_t batch_pick(int tok_per_wg, BATCH_PARAMS) {
    if constexpr (T == kQ4_K) {
        // two row blocks per wavefront when that still leaves >= 1024 workgroups
        const long gy = map.items ? y_blocks : 1;
        const bool wide = long((n_out + 31) / 32) * gy >= 1024;
        if (tok_per_wg <= 16) return wide ? batch_pick_ks<T, 2, 1>(BATCH_ARGS) : batch_pick_ks<T, 1, 1>(BATCH_ARGS);
        return wide ? batch_pick_ks<T, 2, 2>(BATCH_ARGS) : batch_pick_ks<T, 1, 2>(BATCH_ARGS);
    } else {
        if (tok_per_wg <= 16) return batch_pick_ks<T, 1, 1>(BATCH_ARGS);
        return batch_pick_ks<T, 1, 2>(BATCH_ARGS);
    }
}

}  // namespace

bool batch_mfma_supported(const WeightLayout& WL) { return WL.total && WL.n_in % 256 == 0; }

hipError_t launch_batch_mfma(const void* w, const WeightLayout& WL, const void* act, int act_rows, int n_tok, float* y,
                             int ldy, hipStream_t s, const TokenMap* group, int item_tokens, int max_items) {
    const ActLayout AL = act_layout(act_rows, WL.n_in);
    if (!batch_mfma_supported(WL) || !AL.total || !AL.has256 || n_tok <= 0) return hipErrorInvalidValue;
    if (group && (item_tokens <= 0 || item_tokens > kBatchItemTokens)) return hipErrorInvalidValue;
    const WeightPtrs W = weight_ptrs(w, WL);
    const ActPtrs A = act_ptrs(act, AL);
    TokenMap map{};
    int tok = n_tok, yb = 0, n_out = WL.n_out;
    if (group) {
        map = *group;
        tok = item_tokens;
        yb = max_items;
        n_out = map.rows_per_expert;
    }
    switch (WL.type) {
        case kQ8_0: return batch_pick<kQ8_0>(tok, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        case kQ4_0: return batch_pick<kQ4_0>(tok, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        case kQ4_K: return batch_pick<kQ4_K>(tok, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        case kQ6_K: return batch_pick<kQ6_K>(tok, W, A, WL.n_in, n_out, n_tok, map, yb, y, ldy, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace fishhip
