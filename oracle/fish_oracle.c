/*
 * CPU restatement of FISH's quantized-matmul path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file is the checker for the HIP path, not part of the product. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * It is written from the GGUF block specification and from what FISH's CPU
 * path computes (citations are files of the reference repository, under
 * model/fish/); none of the reference's code is reused.
 *
 * Pinning (what fixes each function besides this file's own formulas):
 *   or_fp16_to_fp32 / or_fp32_to_fp16  exhaustive / dense comparison against
 *       numpy's IEEE binary16 conversion (tests/test_oracle.py).
 *   or_quantize_acts(_k)  golden bytes from the reference's own quantizers
 *       (tests/golden/), the tie / zero-block / outlier cases of
 *       test/test_kernels.cpp:135-152, and brute force of the closed form.
 *   or_dequant_row        the Q4_K known-answer block of test/test_m1.cpp:35-71
 *       plus golden dequantised rows for every type.
 *   or_block_dots         brute force from dequantised integer codes.
 *   or_quantize_row       golden packed blocks from the reference's quantize_row.
 *   or_vec_dot_q8 / or_matmul_batch  golden per-row dots and matmul outputs.
 *   or_silu_mul           a float64 restatement within 4 ulps (tests/test_oracle.py).
 *   or_moe_ffn            golden output of a tiny MoE layer composed from the
 *       reference's own primitives in the order of model.cpp:1523-1580.
 *   or_dequant_row / or_matmul_f32path (Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL,
 *       MXFP4, F32, F16, BF16)  golden dequant_row values bit for bit, golden
 *       one-token matmul_batch outputs bit for bit, more tokens within f32
 *       rounding, and a float64 dot of the dequantised values.
 *   or_router_logits      golden matmul_batch outputs on f32 / f16 router
 *       rows (to f32 rounding: the reference's installed dot sums in another
 *       order) and a float64 dot of the same operands.
 * Nothing here is "parity unpinned".
 */
#define _GNU_SOURCE
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_F32 0u
#define OR_F16 1u
#define OR_Q4_0 2u
#define OR_Q4_1 3u
#define OR_Q5_0 6u
#define OR_Q5_1 7u
#define OR_Q8_0 8u
#define OR_Q2_K 10u
#define OR_Q3_K 11u
#define OR_Q4_K 12u
#define OR_Q5_K 13u
#define OR_Q6_K 14u
#define OR_IQ4_NL 20u
#define OR_IQ4_XS 23u
#define OR_BF16 30u
#define OR_MXFP4 39u

/* Byte layouts (model/fish/include/fish/quant.h:28-37, :58-70). */
#define SZ_Q4_0 18
#define SZ_Q8_0 34
#define SZ_Q4_K 144
#define SZ_Q5_K 176
#define SZ_Q6_K 210
#define SZ_Q4_1 20
#define SZ_Q5_0 22
#define SZ_Q5_1 24
#define SZ_Q2_K 84
#define SZ_Q3_K 110
#define SZ_IQ4_NL 18
#define SZ_IQ4_XS 136
#define SZ_MXFP4 17
#define SZ_ACT32 40   /* f32 d; i32 sum; i8 qs[32] */
#define SZ_ACT256 276 /* f32 d; i16 bsums[8]; i8 qs[256] */

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static void wr16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static float rdf(const uint8_t* p) { float f; memcpy(&f, p, 4); return f; }

/* ------------------------------------------------------------------ fp16 */

/* IEEE binary16 -> binary32, exact for every input (quant.cpp:22-44). */
float or_fp16_to_fp32(uint16_t h) {
    const int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);                    /* zero / subnormal */
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(1024 + m), e - 25);
    if (e == 31 && m) {                                        /* keep payload like a bit copy */
        uint32_t bits = ((uint32_t)s << 31) | 0x7F800000u | ((uint32_t)m << 13);
        memcpy(&v, &bits, 4);
        return v;
    }
    return s ? -v : v;
}

/* binary32 -> binary16, round to nearest even, subnormals kept, overflow to
 * infinity, NaN to a quiet NaN (quantize.cpp:32-55). Written as the textbook
 * "round the 24-bit significand at the target position" method. */
uint16_t or_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    const int e = (int)(ax >> 23) - 127;                       /* unbiased exponent */
    if (e > 15) return (uint16_t)(sign | 0x7C00u);
    if (e < -25) return sign;                                  /* below half the smallest subnormal */
    uint32_t sig = (ax & 0x7FFFFFu) | (ax >> 23 ? 0x800000u : 0u);
    /* number of low significand bits dropped: normal half keeps 10 fraction bits */
    int drop = (e >= -14) ? 13 : 13 + (-14 - e);
    uint32_t keep = sig >> drop;
    const uint32_t rem = sig & ((1u << drop) - 1u), halfway = 1u << (drop - 1);
    if (rem > halfway || (rem == halfway && (keep & 1u))) keep += 1u;
    uint32_t out;
    if (e >= -14) out = ((uint32_t)(e + 15) << 10) + (keep - 0x400u); /* carry may bump the exponent */
    else out = keep;                                           /* subnormal; may round up to min normal */
    if (out >= 0x7C00u) out = 0x7C00u;
    return (uint16_t)(sign | out);
}

/* ------------------------------------------------------------------ activations */

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* One scale for `len` values: d = amax / 127 (IEEE f32 division), id = 1/d,
 * codes = clamp(round-half-even(x * id), -127, 127) (quant.cpp:400-434). */
static float act_scale(const float* x, int len, float* id_out) {
    float amax = 0.0f;
    for (int k = 0; k < len; ++k) {
        const float a = fabsf(x[k]);
        if (a > amax) amax = a;
    }
    const float d = amax / 127.0f;
    *id_out = d > 0.0f ? 1.0f / d : 0.0f;
    return d;
}

static int8_t act_code(float x, float id) {
    volatile float p = x * id;                                  /* no contraction into anything */
    return (int8_t)clampi((int)lrintf(p), -127, 127);
}

void or_quantize_acts(const float* x, uint64_t n, void* out_v) {
    uint8_t* out = (uint8_t*)out_v;
    for (uint64_t i = 0; i < n; i += 32, out += SZ_ACT32) {
        float id;
        const float d = act_scale(x + i, 32, &id);
        int32_t sum = 0;
        for (int k = 0; k < 32; ++k) {
            const int8_t q = act_code(x[i + k], id);
            out[8 + k] = (uint8_t)q;
            sum += q;
        }
        memcpy(out, &d, 4);
        memcpy(out + 4, &sum, 4);
    }
}

void or_quantize_acts_k(const float* x, uint64_t n, void* out_v) {
    uint8_t* out = (uint8_t*)out_v;
    for (uint64_t i = 0; i < n; i += 256, out += SZ_ACT256) {
        float id;
        const float d = act_scale(x + i, 256, &id);
        memcpy(out, &d, 4);
        for (int b = 0; b < 8; ++b) {
            int32_t sum = 0;
            for (int k = 0; k < 32; ++k) {
                const int8_t q = act_code(x[i + 32 * b + k], id);
                out[20 + 32 * b + k] = (uint8_t)q;
                sum += q;
            }
            const int16_t s16 = (int16_t)sum;
            memcpy(out + 4 + 2 * b, &s16, 2);
        }
    }
}

/* ------------------------------------------------------------------ integer codes
 * Each decoder writes, for one block, the integer code q of every element and
 * the integer (sub-)block scale it multiplies, so that
 *   w = d * scale * q - dmin * min   (K-quants)    or   w = d * q   (32-blocks).
 * Layouts: quant.cpp:83-90 (Q4_0), :129-133 (Q8_0), :136-163 (Q4_K),
 * :165-192 (Q5_K), :194-216 (Q6_K). */

/* 6-bit scale and min of sub-block j from the 12-byte K-quant table. */
static void k4_scale_min(const uint8_t* s12, int j, int* sc, int* mn) {
    if (j < 4) {
        *sc = s12[j] & 63;
        *mn = s12[j + 4] & 63;
    } else {
        *sc = (s12[j + 4] & 15) | ((s12[j - 4] >> 6) << 4);
        *mn = (s12[j + 4] >> 4) | ((s12[j] >> 6) << 4);
    }
}

/* Q4_K / Q5_K element e of a super-block: sub-block g = e / 32, lane l = e % 32. */
static int q4k_code(const uint8_t* blk, int e) {
    const int g = e >> 5, l = e & 31;
    const uint8_t byte = blk[16 + 32 * (g >> 1) + l];
    return (g & 1) ? (byte >> 4) : (byte & 15);
}

static int q5k_code(const uint8_t* blk, int e) {
    const int g = e >> 5, l = e & 31;
    const uint8_t byte = blk[48 + 32 * (g >> 1) + l];
    const int lo = (g & 1) ? (byte >> 4) : (byte & 15);
    return lo | (((blk[16 + l] >> g) & 1) << 4);
}

/* Q6_K element e = 128n + 32r + l: 6-bit code (0..63) and its scale slot. */
static int q6k_code(const uint8_t* blk, int e, int* slot) {
    const int n = e >> 7, r = (e >> 5) & 3, l = e & 31;
    const uint8_t lq = blk[64 * n + l + 32 * (r & 1)];
    const int lo = (r >= 2) ? (lq >> 4) : (lq & 15);
    const int hi = (blk[128 + 32 * n + l] >> (2 * r)) & 3;
    *slot = 8 * n + (l >> 4) + 2 * r;
    return lo | (hi << 4);
}

static int block_elems(uint32_t t) {
    switch (t) {
        case OR_F32: case OR_F16: case OR_BF16: return 1;
        case OR_Q4_0: case OR_Q8_0: case OR_Q4_1: case OR_Q5_0: case OR_Q5_1: case OR_IQ4_NL: case OR_MXFP4:
            return 32;
        default: return 256;
    }
}
static int block_bytes(uint32_t t) {
    switch (t) {
        case OR_F32: return 4;
        case OR_F16: case OR_BF16: return 2;
        case OR_Q4_0: return SZ_Q4_0;
        case OR_Q8_0: return SZ_Q8_0;
        case OR_Q4_K: return SZ_Q4_K;
        case OR_Q5_K: return SZ_Q5_K;
        case OR_Q6_K: return SZ_Q6_K;
        case OR_Q4_1: return SZ_Q4_1;
        case OR_Q5_0: return SZ_Q5_0;
        case OR_Q5_1: return SZ_Q5_1;
        case OR_Q2_K: return SZ_Q2_K;
        case OR_Q3_K: return SZ_Q3_K;
        case OR_IQ4_NL: return SZ_IQ4_NL;
        case OR_IQ4_XS: return SZ_IQ4_XS;
        case OR_MXFP4: return SZ_MXFP4;
        default: return 0;
    }
}
/* types with an int8 kernel in FISH (quant.cpp:475-481): the rest take the f32 path */
static int int8_type(uint32_t t) {
    return t == OR_Q4_0 || t == OR_Q8_0 || t == OR_Q4_K || t == OR_Q5_K || t == OR_Q6_K;
}

uint64_t or_row_bytes(uint32_t type, uint64_t n) {
    const int be = block_elems(type), bb = block_bytes(type);
    return bb ? (n / (uint64_t)be) * (uint64_t)bb : 0;
}

/* Dequantise one block into 32 or 256 floats, with FISH's float order:
 * Q4_K/Q5_K  (d*sc)*q - (dmin*m);  Q6_K  (d*sc)*q;  Q4_0/Q8_0  d*q. */
static void deq_block(uint32_t t, const uint8_t* b, float* y) {
    switch (t) {
        case OR_Q8_0: {
            const float d = or_fp16_to_fp32(rd16(b));
            for (int k = 0; k < 32; ++k) y[k] = d * (float)(int8_t)b[2 + k];
            break;
        }
        case OR_Q4_0: {
            const float d = or_fp16_to_fp32(rd16(b));
            for (int k = 0; k < 16; ++k) {
                y[k] = d * (float)((b[2 + k] & 15) - 8);
                y[k + 16] = d * (float)((b[2 + k] >> 4) - 8);
            }
            break;
        }
        case OR_Q4_K:
        case OR_Q5_K: {
            const float d = or_fp16_to_fp32(rd16(b)), dmin = or_fp16_to_fp32(rd16(b + 2));
            for (int g = 0; g < 8; ++g) {
                int sc, mn;
                k4_scale_min(b + 4, g, &sc, &mn);
                const float ds = d * (float)sc, dm = dmin * (float)mn;
                for (int l = 0; l < 32; ++l) {
                    const int e = 32 * g + l;
                    const int q = (t == OR_Q4_K) ? q4k_code(b, e) : q5k_code(b, e);
                    y[e] = ds * (float)q - dm;
                }
            }
            break;
        }
        case OR_Q6_K: {
            const float d = or_fp16_to_fp32(rd16(b + 208));
            for (int e = 0; e < 256; ++e) {
                int slot;
                const int q = q6k_code(b, e, &slot);
                /* (d * sc) * (q - 32): the float order of quant.cpp:206-209 */
                y[e] = d * (float)(int8_t)b[192 + slot] * (float)(q - 32);
            }
            break;
        }
        case OR_F32: memcpy(y, b, 4); break;
        case OR_F16: y[0] = or_fp16_to_fp32(rd16(b)); break;
        case OR_BF16: { const uint32_t u = (uint32_t)rd16(b) << 16; memcpy(y, &u, 4); break; }
        case OR_Q4_1:
        case OR_Q5_1: {
            /* d * q + m (quant.cpp:92-100, :115-126); Q5_1's fifth bits after d, m */
            const float d = or_fp16_to_fp32(rd16(b)), m = or_fp16_to_fp32(rd16(b + 2));
            const int q5 = t == OR_Q5_1;
            const uint32_t qh = q5 ? (uint32_t)b[4] | ((uint32_t)b[5] << 8) | ((uint32_t)b[6] << 16) | ((uint32_t)b[7] << 24) : 0;
            const uint8_t* qs = b + (q5 ? 8 : 4);
            for (int k = 0; k < 16; ++k) {
                const int lo = (qs[k] & 15) | (int)(((qh >> k) & 1) << 4), hi = (qs[k] >> 4) | (int)(((qh >> (k + 16)) & 1) << 4);
                y[k] = d * (float)lo + m;
                y[k + 16] = d * (float)hi + m;
            }
            break;
        }
        case OR_Q5_0: {
            /* d * (q - 16), q = nibble | fifth bit << 4 (quant.cpp:102-113) */
            const float d = or_fp16_to_fp32(rd16(b));
            const uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
            for (int k = 0; k < 16; ++k) {
                const int lo = (b[6 + k] & 15) | (int)(((qh >> k) & 1) << 4), hi = (b[6 + k] >> 4) | (int)(((qh >> (k + 16)) & 1) << 4);
                y[k] = d * (float)(lo - 16);
                y[k + 16] = d * (float)(hi - 16);
            }
            break;
        }
        case OR_Q2_K: {
            /* scales[16] qs[64] d dmin: element 128 n + 32 j + 16 h + l uses scale byte
             * 8 n + 2 j + h and bits 2 j of qs[32 n + 16 h + l]; (d * sc) * q - dmin * m
             * (quant.cpp:218-240) */
            const float d = or_fp16_to_fp32(rd16(b + 80)), dmin = or_fp16_to_fp32(rd16(b + 82));
            for (int e = 0; e < 256; ++e) {
                const int n = e >> 7, j = (e >> 5) & 3, h = (e >> 4) & 1, l = e & 15;
                const int sc = b[8 * n + 2 * j + h];
                const int q = (b[16 + 32 * n + 16 * h + l] >> (2 * j)) & 3;
                y[e] = (d * (float)(sc & 15)) * (float)q - dmin * (float)(sc >> 4);
            }
            break;
        }
        case OR_Q3_K: {
            /* hmask[32] qs[64] scales[12] d: 6-bit signed scales (low 4 bits from bytes
             * 0..7, high 2 bits from bytes 8..11), 2-bit codes minus 4 where the hmask bit
             * is clear (quant.cpp:242-280) */
            const float dall = or_fp16_to_fp32(rd16(b + 108));
            int sc[16];
            for (int i = 0; i < 16; ++i) {
                const int lo = (i < 8) ? (b[96 + i] & 15) : (b[96 + i - 8] >> 4);
                const int hi = (b[104 + (i & 3)] >> (2 * (i >> 2))) & 3;
                sc[i] = (lo | (hi << 4)) - 32;
            }
            for (int e = 0; e < 256; ++e) {
                const int n = e >> 7, j = (e >> 5) & 3, h = (e >> 4) & 1, l = e & 15;
                const int idx = 16 * h + l;  /* byte within the 32-byte rows */
                const int q2 = (b[32 + 32 * n + idx] >> (2 * j)) & 3;
                const int hm = (b[idx] >> (4 * n + j)) & 1;
                y[e] = (dall * (float)sc[8 * n + 2 * j + h]) * (float)(q2 - (hm ? 0 : 4));
            }
            break;
        }
        case OR_IQ4_NL:
        case OR_IQ4_XS: {
            /* the non-linear 4-bit codebook (quant.cpp:286-316); IQ4_XS adds 6-bit
             * per-32 scales minus 32 under d */
            static const int8_t cb[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
            const float d = or_fp16_to_fp32(rd16(b));
            if (t == OR_IQ4_NL) {
                for (int k = 0; k < 16; ++k) {
                    y[k] = d * (float)cb[b[2 + k] & 15];
                    y[k + 16] = d * (float)cb[b[2 + k] >> 4];
                }
            } else {
                const uint16_t sh = rd16(b + 2);
                for (int g = 0; g < 8; ++g) {
                    const int ls = ((b[4 + g / 2] >> (4 * (g % 2))) & 15) | (((sh >> (2 * g)) & 3) << 4);
                    const float dl = d * (float)(ls - 32);
                    const uint8_t* qs = b + 8 + 16 * g;
                    for (int k = 0; k < 16; ++k) {
                        y[32 * g + k] = dl * (float)cb[qs[k] & 15];
                        y[32 * g + 16 + k] = dl * (float)cb[qs[k] >> 4];
                    }
                }
            }
            break;
        }
        case OR_MXFP4: {
            /* e8m0 scale 2^(e - 127) times signed e2m1 codes (quant.cpp:318-331) */
            static const float e2m1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
            const float d = ldexpf(1.0f, (int)b[0] - 127);
            for (int k = 0; k < 16; ++k) {
                const int lo = b[1 + k] & 15, hi = b[1 + k] >> 4;
                y[k] = d * ((lo & 8) ? -e2m1[lo & 7] : e2m1[lo & 7]);
                y[k + 16] = d * ((hi & 8) ? -e2m1[hi & 7] : e2m1[hi & 7]);
            }
            break;
        }
        default: break;
    }
}

int or_dequant_row(uint32_t type, const void* src, float* dst, uint64_t n) {
    const int be = block_elems(type), bb = block_bytes(type);
    if (!bb || n % (uint64_t)be) return 0;
    const uint8_t* p = (const uint8_t*)src;
    for (uint64_t i = 0; i < n; i += (uint64_t)be, p += bb) deq_block(type, p, dst + i);
    return 1;
}

/* ------------------------------------------------------------------ exact integer dots
 * Per block, the integers FISH's AVX2 kernels form before any float
 * (quant_x86.cpp:280-297, :299-309, :346-382, :445-495):
 *   Q8_0: isum = sum_k w_k x_k                              (1 int per 32-block)
 *   Q4_0: isum = sum_k (nib_k - 8) x_k                      (1 int per 32-block)
 *   Q4_K: sumi = sum_g sc_g sum_l q x ;  mins = sum_g m_g bsum_g   (2 ints per 256)
 *   Q5_K: same as Q4_K with 5-bit codes                      (2 ints per 256)
 *   Q6_K: sumi = sum_j sc_j sum_{16} (q - 32) x              (1 int per 256)
 * `out` receives them in block order. Returns the number of ints written. */
int64_t or_block_dots(uint32_t type, const void* row, const void* acts, uint64_t n, int32_t* out) {
    const uint8_t* w = (const uint8_t*)row;
    const uint8_t* a = (const uint8_t*)acts;
    int64_t nw = 0;
    if (type == OR_Q8_0 || type == OR_Q4_0) {
        for (uint64_t i = 0; i < n; i += 32) {
            const uint8_t* b = w + (i / 32) * block_bytes(type);
            const int8_t* xq = (const int8_t*)(a + (i / 32) * SZ_ACT32 + 8);
            int32_t s = 0;
            for (int k = 0; k < 32; ++k) {
                const int q = (type == OR_Q8_0) ? (int8_t)b[2 + k]
                                                : ((k < 16 ? (b[2 + k] & 15) : (b[2 + k - 16] >> 4)) - 8);
                s += q * xq[k];
            }
            out[nw++] = s;
        }
        return nw;
    }
    for (uint64_t i = 0; i < n; i += 256) {
        const uint8_t* b = w + (i / 256) * block_bytes(type);
        const uint8_t* ab = a + (i / 256) * SZ_ACT256;
        const int8_t* xq = (const int8_t*)(ab + 20);
        if (type == OR_Q6_K) {
            int32_t sumi = 0;
            for (int j = 0; j < 16; ++j) {
                int32_t dj = 0, slot = 0;
                for (int e = 0; e < 256; ++e) {
                    int s;
                    const int q = q6k_code(b, e, &s);
                    if (s == j) { dj += (q - 32) * xq[e]; slot = s; }
                }
                sumi += (int8_t)b[192 + slot] * dj;
            }
            out[nw++] = sumi;
        } else {
            int32_t sumi = 0, mins = 0;
            for (int g = 0; g < 8; ++g) {
                int sc, mn;
                k4_scale_min(b + 4, g, &sc, &mn);
                int32_t dg = 0;
                for (int l = 0; l < 32; ++l) {
                    const int e = 32 * g + l;
                    const int q = (type == OR_Q4_K) ? q4k_code(b, e) : q5k_code(b, e);
                    dg += q * xq[e];
                }
                int16_t bs;
                memcpy(&bs, ab + 4 + 2 * g, 2);
                sumi += sc * dg;
                mins += mn * bs;
            }
            out[nw++] = sumi;
            out[nw++] = mins;
        }
    }
    return nw;
}

/* ------------------------------------------------------------------ float dots
 * FISH's scalar int8 reference (quant.cpp:353-398): dequantise the weight
 * block, expand the activations to d*q, dot in f32 with four interleaved
 * partial sums, add the block's dot to a running f32 sum. */
static float dot4(const float* a, const float* b, int n) {
    float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    for (int i = 0; i < n; i += 4) {
        s0 += a[i] * b[i];
        s1 += a[i + 1] * b[i + 1];
        s2 += a[i + 2] * b[i + 2];
        s3 += a[i + 3] * b[i + 3];
    }
    return (s0 + s1) + (s2 + s3);
}

float or_vec_dot_q8(uint32_t type, const void* row, const void* acts, uint64_t n) {
    const int be = block_elems(type), bb = block_bytes(type);
    const uint8_t* w = (const uint8_t*)row;
    const uint8_t* a = (const uint8_t*)acts;
    float buf[256], xs[256], sum = 0.0f;
    for (uint64_t i = 0; i < n; i += (uint64_t)be, w += bb) {
        deq_block(type, w, buf);
        if (be == 32) {
            const uint8_t* ab = a + (i / 32) * SZ_ACT32;
            const float d = rdf(ab);
            for (int k = 0; k < 32; ++k) xs[k] = d * (float)(int8_t)ab[8 + k];
        } else {
            const uint8_t* ab = a + (i / 256) * SZ_ACT256;
            const float d = rdf(ab);
            for (int k = 0; k < 256; ++k) xs[k] = d * (float)(int8_t)ab[20 + k];
        }
        sum += dot4(buf, xs, be);
    }
    return sum;
}

/* ------------------------------------------------------------------ matmul
 * y[t * n_out + i] = dot(W_i, x_t) (ops.h:78-84, ops.cpp:177-216); the int8
 * layout is chosen by weight type (quant.cpp:475-481). Rows are split over
 * n_threads POSIX threads; each (row, token) value is independent of the
 * split. */
typedef struct {
    uint32_t type;
    const uint8_t* w;
    const uint8_t* acts;
    int n_tok, n_in, n_out, r0, r1;
    float* y;
} MmJob;

static void* mm_worker(void* p) {
    const MmJob* j = (const MmJob*)p;
    const uint64_t rb = or_row_bytes(j->type, (uint64_t)j->n_in);
    const int be = block_elems(j->type);
    const uint64_t ab = (be == 32) ? (uint64_t)(j->n_in / 32) * SZ_ACT32 : (uint64_t)(j->n_in / 256) * SZ_ACT256;
    for (int t = 0; t < j->n_tok; ++t)
        for (int i = j->r0; i < j->r1; ++i)
            j->y[(size_t)t * j->n_out + i] =
                or_vec_dot_q8(j->type, j->w + (size_t)i * rb, j->acts + (size_t)t * ab, (uint64_t)j->n_in);
    return NULL;
}

/* acts32: n_tok rows of n_in/32 Q8Act blocks; acts256: n_tok rows of n_in/256
 * Q8ActK blocks. The one matching `type` is used. Returns 0 on bad input. */
int or_matmul_batch(uint32_t type, const void* w, const void* acts32, const void* acts256,
                    int n_tok, int n_in, int n_out, float* y, int n_threads) {
    const int be = block_elems(type);
    if (!int8_type(type) || n_in % be || n_tok < 0 || n_out < 0) return 0;
    const void* acts = (be == 32) ? acts32 : acts256;
    if (!acts) return 0;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    if (n_threads > n_out) n_threads = n_out > 0 ? n_out : 1;
    pthread_t th[64];
    MmJob jobs[64];
    for (int k = 0; k < n_threads; ++k) {
        jobs[k] = (MmJob){type, (const uint8_t*)w, (const uint8_t*)acts, n_tok, n_in, n_out,
                          (int)((int64_t)n_out * k / n_threads), (int)((int64_t)n_out * (k + 1) / n_threads), y};
    }
    for (int k = 1; k < n_threads; ++k) pthread_create(&th[k], NULL, mm_worker, &jobs[k]);
    mm_worker(&jobs[0]);
    for (int k = 1; k < n_threads; ++k) pthread_join(th[k], NULL);
    return 1;
}

/* ------------------------------------------------------------------ router (f32 / f16 weights)
 * matmul_batch on a weight type without an int8 kernel (ops.cpp:219-250),
 * as the router of model.cpp:1529 runs it for f32 / f16 gate_inp tensors:
 *   n_tok == 1: vec_dot (quant.cpp:530-546): f32 rows dot the whole row; f16
 *       rows are widened 64 values at a time and each chunk's dot is added
 *       to a running f32 sum;
 *   n_tok > 1: the row is widened once and dotted with every token.
 * Every dot is FISH's scalar dot_f32 (quant.cpp:67-78): four interleaved f32
 * partial sums, a scalar tail into the first, then (s0 + s1) + (s2 + s3). The
 * reference installs an AVX2 dot in its place on x86, which sums in another
 * order, so this agrees with it to f32 rounding only. */
static float dot_f32_scalar(const float* a, const float* b, int n) {
    float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    int i = 0;
    for (; i + 4 <= n; i += 4) {
        s0 += a[i] * b[i];
        s1 += a[i + 1] * b[i + 1];
        s2 += a[i + 2] * b[i + 2];
        s3 += a[i + 3] * b[i + 3];
    }
    for (; i < n; ++i) s0 += a[i] * b[i];
    return (s0 + s1) + (s2 + s3);
}

/* logits [n_tok][n_expert]; w holds n_expert rows of n_embd f32 or f16 bits. */
int or_router_logits(uint32_t type, const void* w, const float* x, int n_tok, int n_embd, int n_expert,
                     float* logits) {
    if ((type != OR_F32 && type != OR_F16) || n_tok < 1 || n_embd < 1 || n_expert < 1) return 0;
    float* row = (float*)malloc(sizeof(float) * (size_t)n_embd);
    if (!row) return 0;
    for (int e = 0; e < n_expert; ++e) {
        const size_t off = (size_t)e * n_embd;
        if (type == OR_F32) memcpy(row, (const float*)w + off, sizeof(float) * (size_t)n_embd);
        else
            for (int k = 0; k < n_embd; ++k) row[k] = or_fp16_to_fp32(((const uint16_t*)w)[off + k]);
        for (int t = 0; t < n_tok; ++t) {
            const float* xt = x + (size_t)t * n_embd;
            float v;
            if (n_tok == 1 && type == OR_F16) {
                v = 0.0f;
                for (int i = 0; i < n_embd; i += 64) v += dot_f32_scalar(row + i, xt + i, n_embd - i < 64 ? n_embd - i : 64);
            } else {
                v = dot_f32_scalar(row, xt, n_embd);
            }
            logits[(size_t)t * n_expert + e] = v;
        }
    }
    free(row);
    return 1;
}

/* matmul_batch for a weight type without an int8 kernel (ops.cpp:219-250;
 * Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, IQ4_XS, MXFP4, F32, F16, BF16):
 *   n_tok == 1: vec_dot (quant.cpp:530-572): quantized types dequantise one
 *       block at a time and add its scalar dot_f32 to a running sum
 *       (dot_blockwise, quant.cpp:341-353); F16 / BF16 the same over 64-value
 *       chunks; F32 one dot over the row;
 *   n_tok > 1: the whole row dequantised once, one dot per token.
 * Every dot is the scalar dot_f32 of quant.cpp:67-78 (FISH installs an AVX2
 * dot for the whole-row case, so that agrees to f32 rounding only). */
int or_matmul_f32path(uint32_t type, const void* w, const float* x, int n_tok, int n_in, int n_out, float* y) {
    const int be = block_elems(type), bb = block_bytes(type);
    if (!bb || int8_type(type) || n_in % be || n_tok < 1 || n_out < 0) return 0;
    const uint64_t rb = (uint64_t)(n_in / be) * (uint64_t)bb;
    float* row = (float*)malloc(sizeof(float) * (size_t)n_in);
    if (!row) return 0;
    const int chunk = (type == OR_F16 || type == OR_BF16) ? 64 : (type == OR_F32 ? n_in : be);
    for (int i = 0; i < n_out; ++i) {
        const uint8_t* src = (const uint8_t*)w + (size_t)i * rb;
        for (int k = 0; k < n_in; k += be) deq_block(type, src + (size_t)(k / be) * bb, row + k);
        for (int t = 0; t < n_tok; ++t) {
            const float* xt = x + (size_t)t * n_in;
            float v;
            if (n_tok == 1) {
                v = 0.0f;
                for (int k = 0; k < n_in; k += chunk) v += dot_f32_scalar(row + k, xt + k, n_in - k < chunk ? n_in - k : chunk);
            } else {
                v = dot_f32_scalar(row, xt, n_in);
            }
            y[(size_t)t * n_out + i] = v;
        }
    }
    free(row);
    return 1;
}

/* ActBatch::quantize (ops.cpp:158-175): both layouts per token row; the
 * 256 layout only when n_in % 256 == 0 (acts256 may then be NULL). */
void or_act_batch(const float* x, int n_tok, int n_in, void* acts32, void* acts256) {
    for (int t = 0; t < n_tok; ++t) {
        const float* xr = x + (size_t)t * n_in;
        if (acts32) or_quantize_acts(xr, (uint64_t)n_in, (uint8_t*)acts32 + (size_t)t * (n_in / 32) * SZ_ACT32);
        if (acts256 && n_in % 256 == 0)
            or_quantize_acts_k(xr, (uint64_t)n_in, (uint8_t*)acts256 + (size_t)t * (n_in / 256) * SZ_ACT256);
    }
}

/* ------------------------------------------------------------------ block writers
 * FISH's own packers (quantize.cpp:108-416): Q8_0 absmax/127; Q4_0 signed
 * max-magnitude value to -8; Q4_K/Q5_K per-group min/max start plus four
 * least-squares refinements, 6-bit scales under f16 super-scales; Q6_K signed
 * max to -32 with one least-squares refinement per 16-group, int8 scales. */

static int nearest_away(float v) { return (int)lroundf(v); }

static void refit_q8_0(const float* x, uint8_t* b) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = (amax < fabsf(x[i])) ? fabsf(x[i]) : amax;
    wr16(b, or_fp32_to_fp16(amax / 127.0f));
    const float d = or_fp16_to_fp32(rd16(b));
    for (int i = 0; i < 32; ++i) b[2 + i] = (uint8_t)(int8_t)(d > 0 ? clampi(nearest_away(x[i] / d), -128, 127) : 0);
}

static void refit_q4_0(const float* x, uint8_t* b) {
    float amax = 0.0f, mx = 0.0f;
    for (int i = 0; i < 32; ++i)
        if (fabsf(x[i]) > amax) { amax = fabsf(x[i]); mx = x[i]; }
    wr16(b, or_fp32_to_fp16(mx / -8.0f));
    const float d = or_fp16_to_fp32(rd16(b));
    int q[32];
    for (int i = 0; i < 32; ++i) q[i] = d != 0.0f ? clampi(nearest_away(x[i] / d) + 8, 0, 15) : 8;
    for (int j = 0; j < 16; ++j) b[2 + j] = (uint8_t)(q[j] | (q[j + 16] << 4));
}

/* x ~ scale * q - m over 32 values, q in [0, nmax], m >= 0. */
static void fit_group(const float* x, int nmax, float* scale, float* mout) {
    float lo = 0.0f, hi = x[0];
    /* std::min / std::max semantics: keep the running value unless strictly beaten */
    for (int i = 0; i < 32; ++i) { lo = (x[i] < lo) ? x[i] : lo; hi = (hi < x[i]) ? x[i] : hi; }
    if (hi <= lo) { *scale = 0.0f; *mout = -lo; return; }
    float sc = (hi - lo) / (float)nmax, off = lo;
    for (int it = 0; it < 4; ++it) {
        double n1 = 0, n2 = 0, sx = 0, sqx = 0;
        const float inv = 1.0f / sc;
        for (int i = 0; i < 32; ++i) {
            const int q = clampi(nearest_away((x[i] - off) * inv), 0, nmax);
            n1 += q;
            n2 += (double)q * q;
            sx += x[i];
            sqx += (double)q * x[i];
        }
        const double det = 32.0 * n2 - n1 * n1;
        if (det <= 0) break;
        double nsc = (32.0 * sqx - n1 * sx) / det;
        double noff = (sx - nsc * n1) / 32.0;
        if (noff > 0) { noff = 0; nsc = n2 > 0 ? sqx / n2 : 0; }
        if (!(nsc > 0)) break;
        sc = (float)nsc;
        off = (float)noff;
    }
    *scale = sc;
    *mout = -off;
}

static void pack_k4_scales(const int* ls, const int* lm, uint8_t* s12) {
    memset(s12, 0, 12);
    for (int j = 0; j < 4; ++j) {
        s12[j] |= (uint8_t)(ls[j] & 63);
        s12[j + 4] |= (uint8_t)(lm[j] & 63);
    }
    for (int j = 4; j < 8; ++j) {
        s12[j + 4] = (uint8_t)((ls[j] & 15) | ((lm[j] & 15) << 4));
        s12[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
        s12[j] |= (uint8_t)((lm[j] >> 4) << 6);
    }
}

static void refit_k45(const float* x, int nmax, uint8_t* b, int* q) {
    float sc[8], mn[8], maxsc = 0.0f, maxm = 0.0f;
    for (int g = 0; g < 8; ++g) {
        fit_group(x + 32 * g, nmax, &sc[g], &mn[g]);
        maxsc = (maxsc < sc[g]) ? sc[g] : maxsc;
        maxm = (maxm < mn[g]) ? mn[g] : maxm;
    }
    wr16(b, or_fp32_to_fp16(maxsc / 63.0f));
    wr16(b + 2, or_fp32_to_fp16(maxm / 63.0f));
    const float dd = or_fp16_to_fp32(rd16(b)), dm = or_fp16_to_fp32(rd16(b + 2));
    int ls[8], lm[8];
    for (int g = 0; g < 8; ++g) {
        ls[g] = dd > 0 ? clampi(nearest_away(sc[g] / dd), 0, 63) : 0;
        lm[g] = dm > 0 ? clampi(nearest_away(mn[g] / dm), 0, 63) : 0;
        const float s = dd * (float)ls[g], m = dm * (float)lm[g];
        for (int i = 0; i < 32; ++i) q[32 * g + i] = s > 0 ? clampi(nearest_away((x[32 * g + i] + m) / s), 0, nmax) : 0;
    }
    pack_k4_scales(ls, lm, b + 4);
}

static void refit_q4_K(const float* x, uint8_t* b) {
    int q[256];
    refit_k45(x, 15, b, q);
    for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 32; ++l) b[16 + 32 * j + l] = (uint8_t)(q[64 * j + l] | (q[64 * j + 32 + l] << 4));
}

static void refit_q5_K(const float* x, uint8_t* b) {
    int q[256];
    refit_k45(x, 31, b, q);
    memset(b + 16, 0, 32);
    for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 32; ++l) {
            const int lo = q[64 * j + l], hi = q[64 * j + 32 + l];
            b[48 + 32 * j + l] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
            if (lo & 16) b[16 + l] |= (uint8_t)(1u << (2 * j));
            if (hi & 16) b[16 + l] |= (uint8_t)(2u << (2 * j));
        }
}

static void refit_q6_K(const float* x, uint8_t* b) {
    /* group j of the scale table holds the 16 elements with q6k slot j */
    int members[16][16], count[16] = {0};
    for (int e = 0; e < 256; ++e) {
        int slot;
        (void)q6k_code(b, e, &slot); /* slot depends only on e */
        members[slot][count[slot]++] = e;
    }
    float gs[16], maxs = 0.0f, maxs_signed = 0.0f;
    for (int g = 0; g < 16; ++g) {
        float amax = 0.0f, mx = 0.0f;
        for (int k = 0; k < 16; ++k) {
            const float v = x[members[g][k]];
            if (fabsf(v) > amax) { amax = fabsf(v); mx = v; }
        }
        float s = mx / -32.0f;
        if (s != 0.0f) {
            double sqx = 0, sqq = 0;
            for (int k = 0; k < 16; ++k) {
                const int q = clampi(nearest_away(x[members[g][k]] / s), -32, 31);
                sqx += (double)q * x[members[g][k]];
                sqq += (double)q * q;
            }
            if (sqq > 0) {
                const float ls = (float)(sqx / sqq);
                if (ls != 0.0f) s = ls;
            }
        }
        gs[g] = s;
        if (fabsf(s) > maxs) { maxs = fabsf(s); maxs_signed = s; }
    }
    const float iscale = maxs_signed != 0.0f ? -128.0f / maxs_signed : 0.0f;
    wr16(b + 208, or_fp32_to_fp16(iscale != 0.0f ? 1.0f / iscale : 0.0f));
    const float d = or_fp16_to_fp32(rd16(b + 208));
    for (int g = 0; g < 16; ++g) b[192 + g] = (uint8_t)(int8_t)clampi(nearest_away(iscale * gs[g]), -128, 127);
    memset(b, 0, 192);
    for (int e = 0; e < 256; ++e) {
        int slot;
        (void)q6k_code(b, e, &slot);
        const float s = d * (float)(int8_t)b[192 + slot];
        const int q = (s != 0.0f ? clampi(nearest_away(x[e] / s), -32, 31) : 0) + 32;
        const int n = e >> 7, r = (e >> 5) & 3, l = e & 31;
        uint8_t* lq = b + 64 * n + l + 32 * (r & 1);
        *lq = (uint8_t)(*lq | ((r < 2) ? (q & 15) : ((q & 15) << 4)));
        b[128 + 32 * n + l] = (uint8_t)(b[128 + 32 * n + l] | (((q >> 4) & 3) << (2 * r)));
    }
}

int or_quantize_row(uint32_t type, const float* x, void* dst, uint64_t n) {
    const int be = block_elems(type), bb = block_bytes(type);
    if (!bb || n % (uint64_t)be) return 0;
    uint8_t* out = (uint8_t*)dst;
    for (uint64_t i = 0; i < n; i += (uint64_t)be, out += bb) {
        switch (type) {
            case OR_Q8_0: refit_q8_0(x + i, out); break;
            case OR_Q4_0: refit_q4_0(x + i, out); break;
            case OR_Q4_K: refit_q4_K(x + i, out); break;
            case OR_Q5_K: refit_q5_K(x + i, out); break;
            case OR_Q6_K: refit_q6_K(x + i, out); break;
            default: return 0;
        }
    }
    return 1;
}

/* Packs many rows on n_threads threads (input preparation for large shapes). */
typedef struct { uint32_t type; const float* x; uint8_t* dst; uint64_t n_in; int64_t r0, r1; } PackJob;
static void* pack_worker(void* p) {
    const PackJob* j = (const PackJob*)p;
    const uint64_t rb = or_row_bytes(j->type, j->n_in);
    for (int64_t r = j->r0; r < j->r1; ++r) or_quantize_row(j->type, j->x + (size_t)r * j->n_in, j->dst + (size_t)r * rb, j->n_in);
    return NULL;
}
int or_quantize_rows(uint32_t type, const float* x, void* dst, int64_t n_rows, uint64_t n_in, int n_threads) {
    if (!block_bytes(type) || n_in % (uint64_t)block_elems(type)) return 0;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    pthread_t th[64];
    PackJob jobs[64];
    for (int k = 0; k < n_threads; ++k)
        jobs[k] = (PackJob){type, x, (uint8_t*)dst, n_in, n_rows * k / n_threads, n_rows * (k + 1) / n_threads};
    for (int k = 1; k < n_threads; ++k) pthread_create(&th[k], NULL, pack_worker, &jobs[k]);
    pack_worker(&jobs[0]);
    for (int k = 1; k < n_threads; ++k) pthread_join(th[k], NULL);
    return 1;
}

/* ------------------------------------------------------------------ MoE
 * softmax (ops.cpp:40-55), SiLU (ops.cpp:25-30) and the expert-grouped FFN
 * of model.cpp:1523-1580 with the router logits given:
 *   p = softmax(logits_t); top-k by probability, descending; if `norm`,
 *   w_k /= sum of the k probabilities; for e = 0..NE-1 ascending, the tokens
 *   that chose e (ascending t) form a batch: gate, up = W_e . x; h =
 *   silu(gate) * up; down = W_e . quantize(h); out[t] += w * down.
 * Weights: gate/up [NE][F][row E], down [NE][E][row F], expert slices
 * contiguous (model.cpp:66-69). out must hold n_tok * E floats. */
void or_softmax(float* x, int n) {
    if (n <= 0) return;
    float m = x[0];
    for (int i = 1; i < n; ++i) if (x[i] > m) m = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) { x[i] = expf(x[i] - m); sum += x[i]; }
    if (sum <= 0.0f) { for (int i = 0; i < n; ++i) x[i] = 1.0f / (float)n; return; }
    const float inv = 1.0f / sum;
    for (int i = 0; i < n; ++i) x[i] *= inv;
}

float or_silu(float v) { return v / (1.0f + expf(-v)); }

/* h = silu(g) * u element by element, as ffn_block does it: silu_inplace
 * (ops.cpp:25-30), then g[i] *= u[i] (model.cpp:1504-1508), each step one f32
 * rounding. Pinned by tests/test_oracle.py against a float64 restatement. */
void or_silu_mul(const float* g, const float* u, uint64_t n, float* h) {
    for (uint64_t i = 0; i < n; ++i) {
        const float s = or_silu(g[i]);
        h[i] = s * u[i];
    }
}

/* Top-k of p[0..ne) by value, descending (ties: lower index first). */
void or_route(const float* logits, int n_tok, int ne, int k, int norm, int* sel, float* wsel) {
    float* p = (float*)malloc(sizeof(float) * (size_t)ne);
    unsigned char* used = (unsigned char*)malloc((size_t)ne);
    for (int t = 0; t < n_tok; ++t) {
        memcpy(p, logits + (size_t)t * ne, sizeof(float) * (size_t)ne);
        or_softmax(p, ne);
        memset(used, 0, (size_t)ne);
        float sum = 0.0f;
        for (int j = 0; j < k; ++j) {
            int best = -1;
            for (int e = 0; e < ne; ++e)
                if (!used[e] && (best < 0 || p[e] > p[best])) best = e;
            used[best] = 1;
            sel[t * k + j] = best;
            wsel[t * k + j] = p[best];
            sum += p[best];
        }
        if (norm && sum > 0.0f)
            for (int j = 0; j < k; ++j) wsel[t * k + j] /= sum;
    }
    free(p);
    free(used);
}

static uint64_t act_row_bytes(uint32_t type, int n_in) {
    return block_elems(type) == 32 ? (uint64_t)(n_in / 32) * SZ_ACT32 : (uint64_t)(n_in / 256) * SZ_ACT256;
}

int or_moe_ffn(const float* x, const float* logits, int n_tok, int E, int F, int NE, int K, int norm,
               uint32_t t_gate, const void* w_gate, uint32_t t_up, const void* w_up,
               uint32_t t_down, const void* w_down, float* out, int n_threads) {
    int* sel = (int*)malloc(sizeof(int) * (size_t)n_tok * K);
    float* wsel = (float*)malloc(sizeof(float) * (size_t)n_tok * K);
    or_route(logits, n_tok, NE, K, norm, sel, wsel);
    memset(out, 0, sizeof(float) * (size_t)n_tok * E);
    const uint64_t gsz = or_row_bytes(t_gate, (uint64_t)E) * (uint64_t)F;
    const uint64_t usz = or_row_bytes(t_up, (uint64_t)E) * (uint64_t)F;
    const uint64_t dsz = or_row_bytes(t_down, (uint64_t)F) * (uint64_t)E;
    int* toks = (int*)malloc(sizeof(int) * (size_t)n_tok);
    float* wts = (float*)malloc(sizeof(float) * (size_t)n_tok);
    float* xin = (float*)malloc(sizeof(float) * (size_t)n_tok * E);
    float* g = (float*)malloc(sizeof(float) * (size_t)n_tok * F);
    float* u = (float*)malloc(sizeof(float) * (size_t)n_tok * F);
    float* dn = (float*)malloc(sizeof(float) * (size_t)n_tok * E);
    uint8_t* a32 = (uint8_t*)malloc((size_t)n_tok * (E / 32) * SZ_ACT32 + (size_t)n_tok * (F / 32) * SZ_ACT32 + 64);
    uint8_t* a256 = (uint8_t*)malloc((size_t)n_tok * (E / 256 + F / 256 + 1) * SZ_ACT256 + 64);
    for (int e = 0; e < NE; ++e) {
        int cnt = 0;
        for (int t = 0; t < n_tok; ++t)
            for (int j = 0; j < K; ++j)
                if (sel[t * K + j] == e) { toks[cnt] = t; wts[cnt] = wsel[t * K + j]; ++cnt; }
        if (!cnt) continue;
        for (int j = 0; j < cnt; ++j) memcpy(xin + (size_t)j * E, x + (size_t)toks[j] * E, sizeof(float) * (size_t)E);
        or_act_batch(xin, cnt, E, a32, (E % 256 == 0) ? a256 : NULL);
        or_matmul_batch(t_gate, (const uint8_t*)w_gate + gsz * e, a32, a256, cnt, E, F, g, n_threads);
        or_matmul_batch(t_up, (const uint8_t*)w_up + usz * e, a32, a256, cnt, E, F, u, n_threads);
        for (size_t i = 0; i < (size_t)cnt * F; ++i) g[i] = or_silu(g[i]) * u[i];
        or_act_batch(g, cnt, F, a32, (F % 256 == 0) ? a256 : NULL);
        or_matmul_batch(t_down, (const uint8_t*)w_down + dsz * e, a32, a256, cnt, F, E, dn, n_threads);
        for (int j = 0; j < cnt; ++j) {
            float* o = out + (size_t)toks[j] * E;
            const float* d = dn + (size_t)j * E;
            for (int i = 0; i < E; ++i) o[i] += wts[j] * d[i];
        }
    }
    free(sel); free(wsel); free(toks); free(wts); free(xin); free(g); free(u); free(dn); free(a32); free(a256);
    (void)act_row_bytes;
    return 1;
}
