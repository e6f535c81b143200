// Many-token matmul (prefill / batched experts) over repacked K-quant weights
// on gfx950 int8 MFMA (v_mfma_i32_32x32x32_i8) with i32 accumulation.
//
// Arithmetic (the integers of FISH's dot_q4_K_q8k / dot_q6_K_q8k,
// quant_x86.cpp:346-382, :445-495), per output (token t, row r) and
// super-block of 256 values:
//   Q4_K  I = sum_g sc_g sum_l q x       J = sum_g m_g bsum_g
//         y += xd * (d * I - dmin * J)       (Q5_K the same with 5-bit q,
//         quant_x86.cpp:384-427)
//   Q6_K  I = sum_j sc_j sum_{16} (q - 32) x            y += xd * (d * I)
// A scaled code (sc * q up to 945, sc * (q - 32) up to 4096 in magnitude) does
// not fit an int8 MFMA operand, so every weight is split into two int8 planes
// that one MFMA each multiplies with the same activation operand:
//   Q4_K  sc = 8 a + b (a, b in 0..7): planes a*q and b*q (<= 105), I = 8 H + L
//         -- one packed 16-bit multiply makes four bytes of a plane;
//   Q6_K  w' = sc * (q - 32) = 64 hi + lo (0 <= lo < 64): I = 64 H + L;
//   Q5_K  w' = sc * q (<= 1953) = 64 hi + lo the same way.
// J is exact on one f16 MFMA per super-block: A = (64 (bsum >> 6), bsum & 63)
// per token (written by the quantizer), B = (m_g, m_g) per row, all small
// integers, so every product and sum is exact in f32.
//
// Tiling: a wavefront owns TPW x RPW 32x32 blocks (tokens x rows), a
// workgroup WT x WR wavefronts; Q4_K / Q5_K use four wavefronts of 32 tokens
// x 64 rows (no activation operand is fetched by two wavefronts of a
// workgroup), Q6_K four of 64 tokens x 32 rows. The weight planes
// of a 128-value stage are dequantised once per workgroup into a three-deep
// LDS ring (one barrier per stage); activations go straight from HBM/L2 into
// the A-operand registers (the quantizer writes them in operand order), one
// stage ahead; two wavefronts per SIMD hide each other's latencies. The lane that owns an output owns its weight row, so row
// scales are lane scalars; token scales come in output-register order.
#include "common.h"
#include "dots.h"
#include "kernels.h"

namespace fishhip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef short v2s __attribute__((ext_vector_type(2)));
typedef unsigned short v2us __attribute__((ext_vector_type(2)));

constexpr int SSTEPS = 4;  // 32-value steps per stage
constexpr int kGemmCUs = 256;  // MI355X compute units
constexpr int RING = 3;    // LDS stages in flight

// Raw weight data of one (row, 32-value step) item, between its global load
// and its dequantisation.
struct Raw {
    uint4 codes;   // 16 bytes: Q4 nibble chunk (Q6_K: the low nibbles)
    uint4 meta;    // Q4_K / Q5_K: d, dmin, scales[12] of the super-block
    uint2 qh;      // Q6_K: high bits
    uint32_t sc2;  // Q6_K: the two 16-value scales of the step (bytes 0, 1)
    uint32_t hb;   // Q5_K: fifth bits of the step's 32 values
};

template <uint32_t T>
__device__ __forceinline__ void load_raw(Raw& r, const WeightPtrs& W, int row, int step, int n_in) {
    const int groups = n_in / 32;
    const size_t gi = size_t(row) * groups + step;
    r.codes = *reinterpret_cast<const uint4*>(W.codes + gi * 16);
    if constexpr (has_mins(T)) {
        r.meta = *reinterpret_cast<const uint4*>(W.aux + (size_t(row) * (n_in / 256) + (step >> 3)) * 16);
        if constexpr (T == kQ5_K) r.hb = W.hb[gi];
    } else {
        r.qh = *reinterpret_cast<const uint2*>(W.aux + gi * 8);
        r.sc2 = *reinterpret_cast<const uint16_t*>(W.sc + size_t(row) * (n_in / 16) + 2 * step);
    }
}

__device__ __forceinline__ uint32_t mul4(uint32_t codes, uint32_t s2) {
    // four byte codes times a small factor; no byte overflows (<= 105)
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2us, codes) * __builtin_bit_cast(v2us, s2));
}

// Q6_K: four 6-bit codes (bytes) -> hi and lo bytes of sc * (q - 32).
__device__ __forceinline__ void split6(uint32_t q, v2s sc, v2s off, uint32_t& hi, uint32_t& lo) {
    const v2s e = __builtin_bit_cast(v2s, q & 0x00FF00FFu);
    const v2s o = __builtin_bit_cast(v2s, (q >> 8) & 0x00FF00FFu);
    const v2s we = e * sc + off, wo = o * sc + off;  // sc * q - 32 sc
    const uint32_t he = __builtin_bit_cast(uint32_t, we >> 6), ho = __builtin_bit_cast(uint32_t, wo >> 6);
    const uint32_t le = __builtin_bit_cast(uint32_t, we) & 0x003F003Fu, lo_ = __builtin_bit_cast(uint32_t, wo) & 0x003F003Fu;
    hi = __builtin_amdgcn_perm(ho, he, 0x06020400u);
    lo = __builtin_amdgcn_perm(lo_, le, 0x06020400u);
}

// Dequantise one item into the two planes x two halves (16 bytes each).
template <uint32_t T>
__device__ __forceinline__ void dequant(const Raw& r, int step, uint4 (&out)[2][2]) {
    const uint4 c = r.codes;
    const uint4 n0 = make_uint4(c.x & 0x0F0F0F0Fu, c.y & 0x0F0F0F0Fu, c.z & 0x0F0F0F0Fu, c.w & 0x0F0F0F0Fu);
    const uint4 n1 = make_uint4((c.x >> 4) & 0x0F0F0F0Fu, (c.y >> 4) & 0x0F0F0F0Fu, (c.z >> 4) & 0x0F0F0F0Fu,
                                (c.w >> 4) & 0x0F0F0F0Fu);
    if constexpr (T == kQ4_K) {
        int sc, mn;
        k4_scale_min(r.meta.y, r.meta.z, r.meta.w, step & 7, sc, mn);
        const uint32_t a = uint32_t(sc >> 3) * 0x00010001u, b = uint32_t(sc & 7) * 0x00010001u;
        out[0][0] = make_uint4(mul4(n0.x, a), mul4(n0.y, a), mul4(n0.z, a), mul4(n0.w, a));
        out[0][1] = make_uint4(mul4(n1.x, a), mul4(n1.y, a), mul4(n1.z, a), mul4(n1.w, a));
        out[1][0] = make_uint4(mul4(n0.x, b), mul4(n0.y, b), mul4(n0.z, b), mul4(n0.w, b));
        out[1][1] = make_uint4(mul4(n1.x, b), mul4(n1.y, b), mul4(n1.z, b), mul4(n1.w, b));
    } else if constexpr (T == kQ5_K) {
        int sc, mn;
        k4_scale_min(r.meta.y, r.meta.z, r.meta.w, step & 7, sc, mn);
        const v2s scv = {short(sc), short(sc)}, off = {0, 0};
        const uint4 q[2] = {q5_codes_lo(n0, r.hb), q5_codes_hi(n1, r.hb)};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            split6(q[h].x, scv, off, out[0][h].x, out[1][h].x);
            split6(q[h].y, scv, off, out[0][h].y, out[1][h].y);
            split6(q[h].z, scv, off, out[0][h].z, out[1][h].z);
            split6(q[h].w, scv, off, out[0][h].w, out[1][h].w);
        }
    } else {
        const uint4 nib[2] = {n0, n1};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t qh = h ? r.qh.y : r.qh.x;
            const uint4 q = make_uint4(nib[h].x | ((qh & 0x03030303u) << 4), nib[h].y | (((qh >> 2) & 0x03030303u) << 4),
                                       nib[h].z | (((qh >> 4) & 0x03030303u) << 4),
                                       nib[h].w | (((qh >> 6) & 0x03030303u) << 4));
            const short s = short(int8_t((r.sc2 >> (8 * h)) & 0xFF));
            const v2s scv = {s, s}, off = {short(-32 * s), short(-32 * s)};
            split6(q.x, scv, off, out[0][h].x, out[1][h].x);
            split6(q.y, scv, off, out[0][h].y, out[1][h].y);
            split6(q.z, scv, off, out[0][h].z, out[1][h].z);
            split6(q.w, scv, off, out[0][h].w, out[1][h].w);
        }
    }
}

// Dequantisation in parts, so that it can be spread over a stage's MFMAs:
// prep once per item, then part j (0..3) writes its 16-byte pieces.
//   Q4_K: part j = plane j >> 1 of half j & 1;  Q5_K, Q6_K: parts 0, 1 = both planes of half j.
struct DqPrep {
    uint32_t f[2];   // Q4_K: packed 16-bit factors a, b of the two planes
    short s6[2];     // Q6_K: the two 16-value scales; Q5_K: the group scale (both)
};

template <uint32_t T>
__device__ __forceinline__ DqPrep dequant_prep(const Raw& r, int step) {
    DqPrep p{};
    if constexpr (T == kQ4_K) {
        int sc, mn;
        k4_scale_min(r.meta.y, r.meta.z, r.meta.w, step & 7, sc, mn);
        p.f[0] = uint32_t(sc >> 3) * 0x00010001u;
        p.f[1] = uint32_t(sc & 7) * 0x00010001u;
    } else if constexpr (T == kQ5_K) {
        int sc, mn;
        k4_scale_min(r.meta.y, r.meta.z, r.meta.w, step & 7, sc, mn);
        p.s6[0] = p.s6[1] = short(sc);
    } else {
        p.s6[0] = short(int8_t(r.sc2 & 0xFF));
        p.s6[1] = short(int8_t((r.sc2 >> 8) & 0xFF));
    }
    return p;
}

// Writes part j of an item to LDS through put(plane, half, piece).
template <uint32_t T, typename Put>
__device__ __forceinline__ void dequant_part(const Raw& r, const DqPrep& p, int j, Put put) {
    const uint4 c = r.codes;
    if constexpr (T == kQ4_K) {
        const int plane = j >> 1, h = j & 1;
        const uint4 n = h ? make_uint4((c.x >> 4) & 0x0F0F0F0Fu, (c.y >> 4) & 0x0F0F0F0Fu, (c.z >> 4) & 0x0F0F0F0Fu,
                                       (c.w >> 4) & 0x0F0F0F0Fu)
                          : make_uint4(c.x & 0x0F0F0F0Fu, c.y & 0x0F0F0F0Fu, c.z & 0x0F0F0F0Fu, c.w & 0x0F0F0F0Fu);
        const uint32_t f = p.f[plane];
        put(plane, h, make_uint4(mul4(n.x, f), mul4(n.y, f), mul4(n.z, f), mul4(n.w, f)));
    } else {
        if (j >= 2) return;
        const int h = j;
        const uint4 n = h ? make_uint4((c.x >> 4) & 0x0F0F0F0Fu, (c.y >> 4) & 0x0F0F0F0Fu, (c.z >> 4) & 0x0F0F0F0Fu,
                                       (c.w >> 4) & 0x0F0F0F0Fu)
                          : make_uint4(c.x & 0x0F0F0F0Fu, c.y & 0x0F0F0F0Fu, c.z & 0x0F0F0F0Fu, c.w & 0x0F0F0F0Fu);
        uint4 q;
        if constexpr (T == kQ5_K) {
            q = h ? q5_codes_hi(n, r.hb) : q5_codes_lo(n, r.hb);
        } else {
            const uint32_t qh = h ? r.qh.y : r.qh.x;
            q = make_uint4(n.x | ((qh & 0x03030303u) << 4), n.y | (((qh >> 2) & 0x03030303u) << 4),
                           n.z | (((qh >> 4) & 0x03030303u) << 4), n.w | (((qh >> 6) & 0x03030303u) << 4));
        }
        const short s = p.s6[h];
        // Q6_K: sc * (q - 32); Q5_K: sc * q
        const short o = (T == kQ5_K) ? short(0) : short(-32 * s);
        const v2s scv = {s, s}, off = {o, o};
        uint4 hi, lo;
        split6(q.x, scv, off, hi.x, lo.x);
        split6(q.y, scv, off, hi.y, lo.y);
        split6(q.z, scv, off, hi.z, lo.z);
        split6(q.w, scv, off, hi.w, lo.w);
        put(0, h, hi);
        put(1, h, lo);
    }
}

// A wavefront owns TPW 32-token blocks x RPW 32-row blocks; a workgroup WT x WR
// wavefronts (32 TPW WT tokens x 32 RPW WR rows) per K part. With KS = 2 the
// workgroup holds two such sets of wavefronts, each over half of the
// super-blocks with its own LDS ring, and the second set's sums are added to
// the first's at the end (through LDS, in that order): twice the wavefronts on
// the same tiles, for grids of one tile per CU or fewer.
template <uint32_t T, int WT, int WR, int TPW, int RPW, int KS>
__global__ __launch_bounds__(64 * WT * WR * KS) __attribute__((amdgpu_waves_per_eu(2))) void gemm_kq_kernel(
    GemmGroup G, ActPtrs A, int n_in, int n_tok, int tok_tiles) {
    constexpr int NW = WT * WR;
    constexpr int RWG = 32 * RPW * WR;                // rows per workgroup
    constexpr int TBW = TPW * WT;                     // 32-token blocks per workgroup
    constexpr int ITEMS = RWG * SSTEPS;               // (row, step) items per stage
    constexpr int IPT = (ITEMS + 64 * NW - 1) / (64 * NW);
    constexpr int SHIFT = (T == kQ4_K) ? 3 : 6;  // I = 8 H + L (Q4_K) or 64 H + L
    // per K part: [stage][plane][step][half][row] of 16-byte pieces
    constexpr int SB = RING * 2 * SSTEPS * 2 * RWG;
    __shared__ uint4 s_b_all[KS * SB];
    // per K part, per super-block epilogue data, loaded during its first stage:
    // row meta (Q4_K / Q5_K d, dmin, scales; Q6_K d in .x), token scales, mins operands
    __shared__ uint4 s_meta_all[KS * RWG];
    __shared__ float4 s_xd_all[KS * TBW * 2 * 4];
    // mins operands: straight from the thread's own load when the thread's wavefront
    // owns one token block (thread tid loads block tid / 64, the wavefront's own)
    constexpr bool J_REG = TPW == 1 && WR == 1;
    constexpr int SJ = has_mins(T) && !J_REG ? TBW * 64 : 0;
    __shared__ uint4 s_j_all[SJ ? KS * SJ : 1];

    // K part of this thread, and its index within the part
    const int ks = int(threadIdx.x) / (64 * NW);
    uint4* s_b = s_b_all + ks * SB;
    uint4* s_meta = s_meta_all + ks * RWG;
    float4* s_xd = s_xd_all + ks * (TBW * 2 * 4);
    uint4* s_j = s_j_all + ks * SJ;
    const int tid = int(threadIdx.x) % (64 * NW), lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;
    const int wt = wave % WT, wr = wave / WT;

    // tile of this workgroup: consecutive tiles of one row range share an XCD
    // (workgroups are dealt to the eight XCDs round-robin)
    const int n_wg = G.tiles_end[G.n - 1] * tok_tiles;
    int lin = int(blockIdx.x);
    if ((n_wg & 7) == 0) lin = (lin & 7) * (n_wg >> 3) + (lin >> 3);
    int row_tile = lin / tok_tiles;
    const int tok_tile = lin % tok_tiles;
    // the group member this row tile belongs to
    int gm = 0;
#pragma unroll
    for (int j = 1; j < kGemmGroupMax; ++j)
        if (j < G.n && row_tile >= G.tiles_end[j - 1]) gm = j;
    if (gm > 0) row_tile -= G.tiles_end[gm - 1];
    const WeightPtrs W = G.w[gm];
    const int n_out = G.n_out[gm], ldy = G.ldy[gm];
    float* __restrict__ y = G.y[gm];
    const int row0 = row_tile * RWG;

    // the part's stages and super-blocks: s0 .. s0 + stages - 1, sb0 .. sb0 + nsb - 1
    const int steps = n_in / 32, n_sb = n_in / 256, stages = steps / SSTEPS / KS, nsb = n_sb / KS;
    const int s0 = ks * stages, sb0 = ks * nsb;
    const int tb0 = tok_tile * TBW + wt * TPW;       // first 32-token block of the wavefront
    int tb[TPW];
#pragma unroll
    for (int b = 0; b < TPW; ++b) tb[b] = min(tb0 + b, A.n_tb - 1);
    const int wrow = wr * 32 * RPW + l32;            // the lane's row in the workgroup (block 0)

    // dequantisation items of this thread: item = tid + 64 NW j -> (row, step)
    int it_row[IPT], it_step[IPT];
    bool it_on[IPT];
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
        const int item = tid + 64 * NW * j;
        it_on[j] = item < ITEMS;
        const int it = it_on[j] ? item : 0;
        it_row[j] = it >> 2;
        it_step[j] = it & 3;
    }
    auto lds_at = [&](int st, int plane, int s, int h, int r) {
        return (((st * 2 + plane) * SSTEPS + s) * 2 + h) * RWG + (r ^ (s << 2));
    };
    auto load_stage = [&](Raw (&raw)[IPT], int stage) {
#pragma unroll
        for (int j = 0; j < IPT; ++j)
            load_raw<T>(raw[j], W, min(row0 + it_row[j], n_out - 1), (s0 + stage) * SSTEPS + it_step[j], n_in);
    };
    auto store_stage = [&](const Raw (&raw)[IPT], int stage, int slot) {
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            if constexpr (ITEMS % (64 * NW) != 0) {
                if (!it_on[j]) continue;
            }
            uint4 o[2][2];
            dequant<T>(raw[j], (s0 + stage) * SSTEPS + it_step[j], o);
#pragma unroll
            for (int p = 0; p < 2; ++p)
#pragma unroll
                for (int h = 0; h < 2; ++h) s_b[lds_at(slot, p, it_step[j], h, it_row[j])] = o[p][h];
        }
    };
    // A operand of (block b, step s of a stage): 1 KB pieces, lane-contiguous;
    // a uniform stage base plus a per-lane offset and an immediate
    const uint4* gA = reinterpret_cast<const uint4*>(A.gA);
    int a_off[TPW];
#pragma unroll
    for (int b = 0; b < TPW; ++b) a_off[b] = tb[b] * steps * 64 + lane;
    auto load_a = [&](v4i (&a)[TPW][SSTEPS], int stage) {
        const uint4* base = gA + size_t(s0 + stage) * (SSTEPS * 64);
#pragma unroll
        for (int b = 0; b < TPW; ++b)
#pragma unroll
            for (int s = 0; s < SSTEPS; ++s) a[b][s] = __builtin_bit_cast(v4i, base[a_off[b] + s * 64]);
    };

    v16i accH[TPW][RPW], accL[TPW][RPW];
    v16f accY[TPW][RPW];
#pragma unroll
    for (int b = 0; b < TPW; ++b)
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            accH[b][r] = v16i{};
            accL[b][r] = v16i{};
            accY[b][r] = v16f{};
        }

    // MFMAs of one stage from LDS slot `slot`; each step's A registers are
    // refilled with the same step of stage `next` as soon as its MFMAs are
    // issued (one A buffer), the next step's weight operands are read from LDS
    // before the current step's MFMAs, and the dequantisation of `raw` (stage
    // dq_stage) into slot dq_slot is spread over the steps so the wavefront has
    // VALU work between its MFMAs.
    auto compute_stage = [&](v4i (&a)[TPW][SSTEPS], int slot, int next, const Raw (&raw)[IPT], int dq_stage,
                             int dq_slot) {
        const uint4* base = gA + size_t(s0 + next) * (SSTEPS * 64);
        DqPrep prep[IPT];
#pragma unroll
        for (int j = 0; j < IPT; ++j) prep[j] = dequant_prep<T>(raw[j], (s0 + dq_stage) * SSTEPS + it_step[j]);
        v4i bh[RPW], bl[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            bh[r] = __builtin_bit_cast(v4i, s_b[lds_at(slot, 0, 0, half, wrow + 32 * r)]);
            bl[r] = __builtin_bit_cast(v4i, s_b[lds_at(slot, 1, 0, half, wrow + 32 * r)]);
        }
#pragma unroll
        for (int s = 0; s < SSTEPS; ++s) {
            v4i nbh[RPW], nbl[RPW];
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                nbh[r] = bh[r];
                nbl[r] = bl[r];
                if (s + 1 < SSTEPS) {
                    nbh[r] = __builtin_bit_cast(v4i, s_b[lds_at(slot, 0, s + 1, half, wrow + 32 * r)]);
                    nbl[r] = __builtin_bit_cast(v4i, s_b[lds_at(slot, 1, s + 1, half, wrow + 32 * r)]);
                }
            }
#pragma unroll
            for (int b = 0; b < TPW; ++b) {
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    accH[b][r] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[b][s], bh[r], accH[b][r], 0, 0, 0);
                    accL[b][r] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[b][s], bl[r], accL[b][r], 0, 0, 0);
                }
                a[b][s] = __builtin_bit_cast(v4i, base[a_off[b] + s * 64]);
            }
#pragma unroll
            for (int j = 0; j < IPT; ++j) {
                if constexpr (ITEMS % (64 * NW) != 0) {
                    if (!it_on[j]) continue;
                }
                dequant_part<T>(raw[j], prep[j], s, [&](int plane, int h, uint4 v) {
                    s_b[lds_at(dq_slot, plane, it_step[j], h, it_row[j])] = v;
                });
            }
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                bh[r] = nbh[r];
                bl[r] = nbl[r];
            }
        }
    };

    // epilogue data of super-block sb: global -> registers (issued with its
    // first stage) -> LDS (after that stage's MFMAs)
    constexpr int EJ = has_mins(T) ? TBW * 64 : 0;  // mins-operand pieces
    constexpr int EX = TBW * 2 * 4;                 // token-scale pieces
    uint4 e_meta = make_uint4(0, 0, 0, 0), e_j = make_uint4(0, 0, 0, 0);
    float4 e_x = make_float4(0.f, 0.f, 0.f, 0.f);
    const int e_tb = min(tok_tile * TBW + (tid >> 6) % TBW, A.n_tb - 1);
    // every thread loads and stores (duplicate copies of the same values):
    // no divergent branch, so no wait for all outstanding loads
    auto load_epi = [&](int sb) {
        sb += sb0;  // the part's super-block
        const size_t r = size_t(min(row0 + tid % RWG, n_out - 1));
        if constexpr (has_mins(T)) e_meta = *reinterpret_cast<const uint4*>(W.aux + (r * n_sb + sb) * 16);
        else e_meta.x = W.d[r * n_sb + sb];
        if constexpr (has_mins(T))
            e_j = *reinterpret_cast<const uint4*>(A.gJ + ((size_t(e_tb) * n_sb + sb) * 64 + lane) * 8);
        const int xi = tid % EX, b = xi >> 3, q = xi & 7;  // block of the workgroup, 16-byte piece of its 128 bytes
        const int tbb = min(tok_tile * TBW + b, A.n_tb - 1);
        e_x = reinterpret_cast<const float4*>(A.gX + (size_t(tbb) * n_sb + sb) * 32)[q];
    };
    uint4 cur_j = make_uint4(0, 0, 0, 0);  // the mins operand of the super-block in flight (J_REG)
    auto store_epi = [&]() {
        s_meta[tid % RWG] = e_meta;
        if constexpr (has_mins(T) && !J_REG) s_j[tid % EJ] = e_j;
        if constexpr (has_mins(T) && J_REG) cur_j = e_j;
        s_xd[tid % EX] = e_x;
    };

    // super-block epilogue: y += xd * (d * I - dmin * J)   (Q6_K: y += xd * (d * I))
    auto epilogue = [&]() {
        float d[RPW], dmin[RPW];
        v8h bj[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const uint4 m = s_meta[wrow + 32 * r];
            dmin[r] = 0.0f;
            if constexpr (has_mins(T)) {
                d[r] = f16_bits_to_f32(uint16_t(m.x & 0xFFFF));
                dmin[r] = f16_bits_to_f32(uint16_t(m.x >> 16));
                // the eight 6-bit mins, four per dword (quant.cpp:136-144 packing)
                const uint32_t mn_lo = m.z & 0x3F3F3F3Fu;
                const uint32_t mn_hi = ((m.w >> 4) & 0x0F0F0F0Fu) | ((m.z >> 2) & 0x30303030u);
                v8h v;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    v[g] = _Float16(float((mn_lo >> (8 * g)) & 0xFF));
                    v[4 + g] = _Float16(float((mn_hi >> (8 * g)) & 0xFF));
                }
                bj[r] = v;
            } else {
                d[r] = f16_bits_to_f32(uint16_t(m.x));
            }
        }
#pragma unroll
        for (int b = 0; b < TPW; ++b) {
            const int wb = wt * TPW + b;  // block index within the workgroup
            float xd[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = s_xd[wb * 8 + half * 4 + q];
                xd[4 * q] = v.x; xd[4 * q + 1] = v.y; xd[4 * q + 2] = v.z; xd[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                v16f J = v16f{};
                if constexpr (has_mins(T)) {
                    const v8h aj = __builtin_bit_cast(v8h, J_REG ? cur_j : s_j[wb * 64 + lane]);
                    J = __builtin_amdgcn_mfma_f32_32x32x16_f16(aj, bj[r], v16f{}, 0, 0, 0);
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float fi = float((accH[b][r][i] << SHIFT) + accL[b][r][i]);
                    float t = d[r] * fi;
                    if constexpr (has_mins(T)) t = fmaf(-dmin[r], J[i], t);
                    accY[b][r][i] = fmaf(xd[i], t, accY[b][r][i]);
                }
                accH[b][r] = v16i{};
                accL[b][r] = v16i{};
            }
        }
    };

    // ---- prologue: stages 0 and 1 into the ring, stage 2 raw in registers,
    // super-block 0's epilogue data in registers
    Raw raw0[IPT], raw1[IPT];
    load_epi(0);
    load_stage(raw0, 0);
    load_stage(raw1, min(1, stages - 1));
    store_stage(raw0, 0, 0);
    store_stage(raw1, 1, 1);
    load_stage(raw0, min(2, stages - 1));
    v4i a0[TPW][SSTEPS];
    load_a(a0, 0);

    // ---- main loop, one super-block (two stages) per iteration; stage i
    // computes from slot i % 3, prefetches raw(i + 3) and A(i + 1), and
    // dequantises raw(i + 2) into slot (i + 2) % 3. Every global load is
    // consumed one stage after it is issued: the epilogue data of super-block
    // sb + 1 is loaded during the second stage of sb, ahead of that stage's
    // weight loads (the scheduling barriers keep the issue order, so waiting
    // for it never waits for weights still on their way from HBM).
    int slot = 0;
    for (int i = 0; i < stages; i += 2) {
        // even stage i: raw0 holds stage i + 2
        __syncthreads();
        store_epi();
        __builtin_amdgcn_sched_barrier(0);
        load_stage(raw1, min(i + 3, stages - 1));
        __builtin_amdgcn_sched_barrier(0);
        compute_stage(a0, slot, i + 1, raw0, i + 2, slot + 2 >= RING ? slot + 2 - RING : slot + 2);
        slot = slot + 1 == RING ? 0 : slot + 1;
        // odd stage i + 1: raw1 holds stage i + 3
        __syncthreads();
        load_epi(min((i >> 1) + 1, nsb - 1));
        __builtin_amdgcn_sched_barrier(0);
        load_stage(raw0, min(i + 4, stages - 1));
        __builtin_amdgcn_sched_barrier(0);
        compute_stage(a0, slot, min(i + 2, stages - 1), raw1, i + 3, slot + 2 >= RING ? slot + 2 - RING : slot + 2);
        slot = slot + 1 == RING ? 0 : slot + 1;
        epilogue();
    }

    if constexpr (KS == 2) {
        // the second part's sums go through LDS to the same lane of the first part's
        // same wavefront, which adds them to its own (first part + second part)
        constexpr int NV = TPW * RPW * 16;
        static_assert(size_t(NV) * 64 * NW * 4 <= sizeof(s_b_all), "exchange fits the LDS rings");
        float* xch = reinterpret_cast<float*>(s_b_all) + size_t(tid) * NV;
        __syncthreads();  // every wavefront is done with the rings
        if (ks == 1) {
#pragma unroll
            for (int b = 0; b < TPW; ++b)
#pragma unroll
                for (int r = 0; r < RPW; ++r)
#pragma unroll
                    for (int i = 0; i < 16; ++i) xch[(b * RPW + r) * 16 + i] = accY[b][r][i];
        }
        __syncthreads();
        if (ks == 1) return;
#pragma unroll
        for (int b = 0; b < TPW; ++b)
#pragma unroll
            for (int r = 0; r < RPW; ++r)
#pragma unroll
                for (int i = 0; i < 16; ++i) accY[b][r][i] = accY[b][r][i] + xch[(b * RPW + r) * 16 + i];
    }

    // ---- store: lane owns row block r's row, register i of token block b is token 8 (i / 4) + 4 half + i % 4
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int my_row = row0 + wrow + 32 * r;
        if (my_row >= n_out) continue;
#pragma unroll
        for (int b = 0; b < TPW; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int t = (tb0 + b) * 32 + 8 * (i >> 2) + 4 * half + (i & 3);
                if (t < n_tok) y[size_t(t) * ldy + my_row] = accY[b][r][i];
            }
    }
}

// KS = 2 (two K parts per workgroup) for grids of at most one workgroup per CU whose
// super-blocks split evenly: measured at M = 512, down (Q6_K 4096x14336, 256 workgroups)
// 106 -> 94 us and o (4096x4096, 256) 32.6 -> 29.1 us, while the larger grids lost (gate+up,
// 1792 workgroups: 171 -> 187 us). The split changes the order of the f32 additions, so a
// tensor's outputs can differ in the last bits between a launch that splits and one that
// does not (a large group and the same tensor alone).
template <uint32_t T, int WT, int WR, int TPW, int RPW>
hipError_t gemm_launch(GemmGroup G, const int* n_outs, const ActPtrs& A, int n_in, int n_tok, hipStream_t s) {
    int tiles = 0;
    for (int j = 0; j < G.n; ++j) {
        tiles += (n_outs[j] + 32 * RPW * WR - 1) / (32 * RPW * WR);
        G.tiles_end[j] = tiles;
    }
    const int tok_tiles = (n_tok + 32 * TPW * WT - 1) / (32 * TPW * WT);
    const dim3 grid(unsigned(tiles * tok_tiles));
    if ((n_in / 256) % 2 == 0 && tiles * tok_tiles <= kGemmCUs)
        hipLaunchKernelGGL((gemm_kq_kernel<T, WT, WR, TPW, RPW, 2>), grid, dim3(2 * 64 * WT * WR), 0, s, G, A, n_in,
                           n_tok, tok_tiles);
    else
        hipLaunchKernelGGL((gemm_kq_kernel<T, WT, WR, TPW, RPW, 1>), grid, dim3(64 * WT * WR), 0, s, G, A, n_in,
                           n_tok, tok_tiles);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_group(int n, const void* const* ws, const WeightLayout* WLs, const void* act, int n_tok,
                             float* const* ys, const int* ldys, hipStream_t s) {
    if (n <= 0 || n > kGemmGroupMax || n_tok <= 0) return hipErrorInvalidValue;
    const uint32_t type = WLs[0].type;
    const int n_in = WLs[0].n_in;
    const ActLayout AL = act_layout(n_tok, n_in);
    if (!AL.total || !AL.has256) return hipErrorInvalidValue;
    GemmGroup G{};
    G.n = n;
    int n_outs[kGemmGroupMax];
    for (int j = 0; j < n; ++j) {
        if (!WLs[j].total || WLs[j].type != type || WLs[j].n_in != n_in) return hipErrorInvalidValue;
        G.w[j] = weight_ptrs(ws[j], WLs[j]);
        G.n_out[j] = n_outs[j] = WLs[j].n_out;
        G.y[j] = ys[j];
        G.ldy[j] = ldys[j];
    }
    const ActPtrs A = act_ptrs(act, AL);
    // a grid of the default tiles that leaves half the CUs without a workgroup (a
    // 4096-row projection of a 256-token chunk: 128 workgroups) takes tiles of half the
    // rows (Q4_K / Q5_K) or half the tokens (Q6_K) instead: 256 workgroups, measured
    // 20 % (o, 4096x4096) and 14 % (down, 4096x14336) faster at M = 256; at 192 and more
    // workgroups the default tiles were as fast or faster
    int rows64 = 0, rows32 = 0;
    for (int j = 0; j < n; ++j) {
        rows64 += (n_outs[j] + 63) / 64;
        rows32 += (n_outs[j] + 31) / 32;
    }
    const bool small = type == kQ6_K ? rows32 * ((n_tok + 255) / 256) <= kGemmCUs / 2
                                     : rows64 * ((n_tok + 127) / 128) <= kGemmCUs / 2;
    // still a quarter of the CUs or fewer with those tiles (a lone 1024-row projection of a
    // 256-token chunk: 64 workgroups): two token wavefronts per workgroup, twice the workgroups
    const bool tiny = small && rows32 * ((n_tok + 127) / 128) <= kGemmCUs / 4;
    switch (type) {
        case kQ4_K:
            if (tiny) return gemm_launch<kQ4_K, 2, 1, 1, 1>(G, n_outs, A, n_in, n_tok, s);
            return small ? gemm_launch<kQ4_K, 4, 1, 1, 1>(G, n_outs, A, n_in, n_tok, s)
                         : gemm_launch<kQ4_K, 4, 1, 1, 2>(G, n_outs, A, n_in, n_tok, s);
        case kQ5_K:
            if (tiny) return gemm_launch<kQ5_K, 2, 1, 1, 1>(G, n_outs, A, n_in, n_tok, s);
            return small ? gemm_launch<kQ5_K, 4, 1, 1, 1>(G, n_outs, A, n_in, n_tok, s)
                         : gemm_launch<kQ5_K, 4, 1, 1, 2>(G, n_outs, A, n_in, n_tok, s);
        // Q6_K (no mins MFMA, heavier dequantization): four token wavefronts share each
        // dequantized stage (measured 8-11 % faster on the 4096 x 14336 down projection)
        case kQ6_K:
            if (tiny) return gemm_launch<kQ6_K, 2, 1, 1, 1>(G, n_outs, A, n_in, n_tok, s);
            return small ? gemm_launch<kQ6_K, 4, 1, 1, 1>(G, n_outs, A, n_in, n_tok, s)
                         : gemm_launch<kQ6_K, 4, 1, 2, 1>(G, n_outs, A, n_in, n_tok, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm(const void* w, const WeightLayout& WL, const void* act, int n_tok, float* y, int ldy,
                       hipStream_t s) {
    return launch_gemm_group(1, &w, &WL, act, n_tok, &y, &ldy, s);
}

}  // namespace fishhip
