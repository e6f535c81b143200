// Host-side block writer: FISH's quantize_row (quantize.cpp:400-416) for the
// five weight types of this path, used to prepare weights (benchmark inputs,
// conversion of f32 tensors) before upload. Byte-identical to FISH's packer:
//   Q8_0  d = f16(amax / 127), q = clamp(round(x / d), -128, 127)     (:118-125)
//   Q4_0  d = f16(max-magnitude value / -8), q = clamp(round(x/d)+8, 0, 15)  (:141-151)
//   Q4_K  per 32-group a min/max start and four least-squares refinements of
//   Q5_K  (scale, offset) for codes 0..15 (Q4_K) or 0..31 (Q5_K); 6-bit
//         scales/mins under f16 super-scales (:189-262)
//   Q6_K  per 16-group the max-magnitude value to -32 and one least-squares
//         scale refinement; int8 scales under an f16 super-scale (:301-347)
// round() is round-half-away-from-zero (std::lround); the f16 encoder rounds
// to nearest even. Compiled without floating-point contraction so every
// intermediate rounds like FISH's baseline x86-64 build.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/fish_hip.h"
#include "common.h"

namespace {

using fishhip::kQ4_0;
using fishhip::kQ4_K;
using fishhip::kQ5_K;
using fishhip::kQ6_K;
using fishhip::kQ8_0;

uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
    const uint32_t mag = x & 0x7FFFFFFFu;
    if (mag >= 0x7F800000u) return uint16_t(sign | 0x7C00u | (mag > 0x7F800000u ? 0x200u : 0u));
    if (mag >= 0x477FF000u) return uint16_t(sign | 0x7C00u);  // rounds to >= 65520: infinity
    if (mag < 0x33000001u) return sign;                      // <= 2^-25: rounds to zero
    const int exp = int(mag >> 23);
    uint32_t mant = (mag & 0x7FFFFFu) | 0x800000u;
    // the half's unit in the last place is 2^-24 for subnormals, 2^(e-10) otherwise
    const int shift = exp >= 113 ? 13 : 13 + (113 - exp);
    const uint32_t rest = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    mant >>= shift;
    if (rest > half || (rest == half && (mant & 1u))) ++mant;
    const uint32_t biased = exp >= 113 ? uint32_t(exp - 112) : 0u;
    // mant carries the implicit bit for normals; adding the exponent field
    // lets a mantissa carry roll into the exponent, as rounding requires
    return uint16_t(sign | ((biased << 10) + (exp >= 113 ? mant - 0x400u : mant)));
}

float f16_to_f32(uint16_t h) {
    const int e = (h >> 10) & 31, m = h & 1023;
    float v = e == 0 ? std::ldexp(float(m), -24) : std::ldexp(float(1024 + m), e - 25);
    return (h & 0x8000) ? -v : v;
}

int iround(float v) { return int(std::lround(v)); }
int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
void put16(uint8_t* p, uint16_t v) { std::memcpy(p, &v, 2); }

void pack_q8_0(const float* x, uint8_t* b) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = std::fabs(x[i]) > amax ? std::fabs(x[i]) : amax;
    const uint16_t h = f32_to_f16(amax / 127.0f);
    put16(b, h);
    const float d = f16_to_f32(h);
    for (int i = 0; i < 32; ++i) b[2 + i] = uint8_t(int8_t(d > 0 ? clampi(iround(x[i] / d), -128, 127) : 0));
}

void pack_q4_0(const float* x, uint8_t* b) {
    float amax = 0.0f, vmax = 0.0f;
    for (int i = 0; i < 32; ++i)
        if (std::fabs(x[i]) > amax) {
            amax = std::fabs(x[i]);
            vmax = x[i];
        }
    const uint16_t h = f32_to_f16(vmax / -8.0f);
    put16(b, h);
    const float d = f16_to_f32(h);
    int q[32];
    for (int i = 0; i < 32; ++i) q[i] = d != 0.0f ? clampi(iround(x[i] / d) + 8, 0, 15) : 8;
    for (int j = 0; j < 16; ++j) b[2 + j] = uint8_t(q[j] | (q[j + 16] << 4));
}

// Least-squares fit of x ~ scale * q - m over one 32-group (q in [0, 15]).
void fit32(const float* x, int nmax, float& scale, float& m) {
    float lo = 0.0f, hi = x[0];
    for (int i = 0; i < 32; ++i) {
        if (x[i] < lo) lo = x[i];
        if (hi < x[i]) hi = x[i];
    }
    if (hi <= lo) {
        scale = 0.0f;
        m = -lo;
        return;
    }
    float s = (hi - lo) / float(nmax), b = lo;
    for (int it = 0; it < 4; ++it) {
        double cq = 0, cqq = 0, cx = 0, cqx = 0;
        const float inv = 1.0f / s;
        for (int i = 0; i < 32; ++i) {
            const int q = clampi(iround((x[i] - b) * inv), 0, nmax);
            cq += q;
            cqq += double(q) * q;
            cx += x[i];
            cqx += double(q) * x[i];
        }
        const double det = 32.0 * cqq - cq * cq;
        if (det <= 0) break;
        double ns = (32.0 * cqx - cq * cx) / det;
        double nb = (cx - ns * cq) / 32.0;
        if (nb > 0) {
            nb = 0;
            ns = cqq > 0 ? cqx / cqq : 0;
        }
        if (!(ns > 0)) break;
        s = float(ns);
        b = float(nb);
    }
    scale = s;
    m = -b;
}

// d, dmin and the 12 scale bytes of a Q4_K / Q5_K super-block (bytes 0..15,
// the same in both) and its codes q[256] in 0..nmax
void pack_k45(const float* x, int nmax, uint8_t* b, int* q) {
    float sc[8], mn[8], top_s = 0.0f, top_m = 0.0f;
    for (int g = 0; g < 8; ++g) {
        fit32(x + 32 * g, nmax, sc[g], mn[g]);
        if (top_s < sc[g]) top_s = sc[g];
        if (top_m < mn[g]) top_m = mn[g];
    }
    const uint16_t hd = f32_to_f16(top_s / 63.0f), hm = f32_to_f16(top_m / 63.0f);
    put16(b, hd);
    put16(b + 2, hm);
    const float dd = f16_to_f32(hd), dm = f16_to_f32(hm);
    int ls[8], lm[8];
    for (int g = 0; g < 8; ++g) {
        ls[g] = dd > 0 ? clampi(iround(sc[g] / dd), 0, 63) : 0;
        lm[g] = dm > 0 ? clampi(iround(mn[g] / dm), 0, 63) : 0;
        const float s = dd * float(ls[g]), m = dm * float(lm[g]);
        for (int i = 0; i < 32; ++i) q[32 * g + i] = s > 0 ? clampi(iround((x[32 * g + i] + m) / s), 0, nmax) : 0;
    }
    uint8_t* s12 = b + 4;
    std::memset(s12, 0, 12);
    for (int j = 0; j < 8; ++j) {
        if (j < 4) {
            s12[j] |= uint8_t(ls[j] & 63);
            s12[j + 4] |= uint8_t(lm[j] & 63);
        } else {
            s12[j + 4] = uint8_t((ls[j] & 15) | ((lm[j] & 15) << 4));
            s12[j - 4] |= uint8_t((ls[j] >> 4) << 6);
            s12[j] |= uint8_t((lm[j] >> 4) << 6);
        }
    }
}

void pack_q4_K(const float* x, uint8_t* b) {
    int q[256];
    pack_k45(x, 15, b, q);
    for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 32; ++l) b[16 + 32 * j + l] = uint8_t(q[64 * j + l] | (q[64 * j + 32 + l] << 4));
}

// Q5_K: qh[32] at byte 16 (bit g of qh[l]: the fifth bit of element 32 g + l),
// then Q4_K's nibble layout at byte 48
void pack_q5_K(const float* x, uint8_t* b) {
    int q[256];
    pack_k45(x, 31, b, q);
    uint8_t* qh = b + 16;
    std::memset(qh, 0, 32);
    for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 32; ++l) {
            const int lo = q[64 * j + l], hi = q[64 * j + 32 + l];
            b[48 + 32 * j + l] = uint8_t((lo & 15) | ((hi & 15) << 4));
            qh[l] = uint8_t(qh[l] | ((lo >> 4) << (2 * j)) | ((hi >> 4) << (2 * j + 1)));
        }
}

// Q6_K element e = 128n + 32r + l sits in scale group 8n + l/16 + 2r.
int q6_group(int e) { return 8 * (e >> 7) + ((e & 31) >> 4) + 2 * ((e >> 5) & 3); }

void pack_q6_K(const float* x, uint8_t* b) {
    float gs[16];
    float top = 0.0f, top_signed = 0.0f;
    for (int g = 0; g < 16; ++g) {
        int idx[16], k = 0;
        for (int e = 0; e < 256 && k < 16; ++e)
            if (q6_group(e) == g) idx[k++] = e;
        float amax = 0.0f, vmax = 0.0f;
        for (int i = 0; i < 16; ++i)
            if (std::fabs(x[idx[i]]) > amax) {
                amax = std::fabs(x[idx[i]]);
                vmax = x[idx[i]];
            }
        float s = vmax / -32.0f;
        if (s != 0.0f) {
            double cqx = 0, cqq = 0;
            for (int i = 0; i < 16; ++i) {
                const int q = clampi(iround(x[idx[i]] / s), -32, 31);
                cqx += double(q) * x[idx[i]];
                cqq += double(q) * q;
            }
            if (cqq > 0) {
                const float ls = float(cqx / cqq);
                if (ls != 0.0f) s = ls;
            }
        }
        gs[g] = s;
        if (std::fabs(s) > top) {
            top = std::fabs(s);
            top_signed = s;
        }
    }
    const float iscale = top_signed != 0.0f ? -128.0f / top_signed : 0.0f;
    const uint16_t hd = f32_to_f16(iscale != 0.0f ? 1.0f / iscale : 0.0f);
    put16(b + 208, hd);
    const float d = f16_to_f32(hd);
    int8_t sc[16];
    for (int g = 0; g < 16; ++g) sc[g] = int8_t(clampi(iround(iscale * gs[g]), -128, 127));
    std::memcpy(b + 192, sc, 16);
    std::memset(b, 0, 192);
    for (int e = 0; e < 256; ++e) {
        const float s = d * float(sc[q6_group(e)]);
        const int q = (s != 0.0f ? clampi(iround(x[e] / s), -32, 31) : 0) + 32;
        const int n = e >> 7, r = (e >> 5) & 3, l = e & 31;
        b[64 * n + l + 32 * (r & 1)] |= uint8_t(r < 2 ? (q & 15) : ((q & 15) << 4));
        b[128 + 32 * n + l] |= uint8_t(((q >> 4) & 3) << (2 * r));
    }
}

bool pack_row(uint32_t type, const float* x, uint8_t* dst, int n) {
    switch (type) {
        case kQ8_0: for (int i = 0; i < n; i += 32, dst += 34) pack_q8_0(x + i, dst); return true;
        case kQ4_0: for (int i = 0; i < n; i += 32, dst += 18) pack_q4_0(x + i, dst); return true;
        case kQ4_K: for (int i = 0; i < n; i += 256, dst += 144) pack_q4_K(x + i, dst); return true;
        case kQ5_K: for (int i = 0; i < n; i += 256, dst += 176) pack_q5_K(x + i, dst); return true;
        case kQ6_K: for (int i = 0; i < n; i += 256, dst += 210) pack_q6_K(x + i, dst); return true;
        default: return false;
    }
}

}  // namespace

extern "C" int fish_hip_quantize_rows(uint32_t type, const float* x, void* dst, int n_rows, int n_in, int n_threads) {
    const size_t rb = fishhip::gguf_row_bytes(type, n_in);
    const int blk = fishhip::is_kquant(type) ? 256 : 32;
    if (!x || !dst || n_rows < 0 || n_in <= 0 || n_in % blk || !rb) return FISH_HIP_ERR_ARG;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    uint8_t* out = static_cast<uint8_t*>(dst);
    if (!pack_row(type, x, out, 0)) return FISH_HIP_ERR_ARG;  // a type without a block writer
    auto work = [&](int r0, int r1) {
        for (int r = r0; r < r1; ++r) pack_row(type, x + size_t(r) * n_in, out + size_t(r) * rb, n_in);
    };
    std::vector<std::thread> th;
    for (int k = 1; k < n_threads; ++k)
        th.emplace_back(work, int(int64_t(n_rows) * k / n_threads), int(int64_t(n_rows) * (k + 1) / n_threads));
    work(0, int(int64_t(n_rows) / n_threads));
    for (auto& t : th) t.join();
    return 0;
}
