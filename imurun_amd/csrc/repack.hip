// Upload-time repack of GGUF blocks (already in device memory) into the
// device layout described in common.h. Runs once per tensor; byte loads are
// fine here because GGUF blocks are only 2-byte aligned.
//
// Source layouts: quant.h:28-37 (block structs), quant.cpp:83-90 (Q4_0),
// :129-133 (Q8_0), :136-163 (Q4_K), :165-192 (Q5_K), :194-216 (Q6_K).
#include "common.h"
#include "kernels.h"

namespace fishhip {

namespace {

__device__ __forceinline__ int q4k_code(const uint8_t* sb, int e) {
    const int g = e >> 5, l = e & 31;
    const uint8_t byte = sb[16 + 32 * (g >> 1) + l];
    return (g & 1) ? (byte >> 4) : (byte & 15);
}

// Q5_K: the low nibble as Q4_K's (after the 32 qh bytes), fifth bit l of qh[g]
__device__ __forceinline__ int q5k_code(const uint8_t* sb, int e) {
    const int g = e >> 5, l = e & 31;
    const uint8_t byte = sb[48 + 32 * (g >> 1) + l];
    const int lo = (g & 1) ? (byte >> 4) : (byte & 15);
    return lo | (((sb[16 + l] >> g) & 1) << 4);
}

__device__ __forceinline__ int q6k_code(const uint8_t* sb, int e) {
    const int n = e >> 7, r = (e >> 5) & 3, l = e & 31;
    const uint8_t lq = sb[64 * n + l + 32 * (r & 1)];
    const int lo = (r >= 2) ? (lq >> 4) : (lq & 15);
    const int hi = (sb[128 + 32 * n + l] >> (2 * r)) & 3;
    return lo | (hi << 4);
}

// One thread per (row, 32-element group) of rows row0 .. row0 + n_rows - 1 of
// the tensor whose layout is L; src holds those rows' GGUF bytes.
__global__ void repack_kernel(uint32_t type, const uint8_t* __restrict__ src, int n_in, int row0, int n_rows,
                              size_t src_row, uint8_t* __restrict__ dst, WeightLayout L) {
    const long gid = long(blockIdx.x) * blockDim.x + threadIdx.x;
    const int groups = n_in / 32;
    if (gid >= long(n_rows) * groups) return;
    const int rr = int(gid / groups), c = int(gid % groups), r = row0 + rr;
    const uint8_t* row = src + size_t(rr) * src_row;
    uint8_t* codes = dst + L.codes + (size_t(r) * groups + c) * 16;
    uint8_t q[32];
    switch (type) {
        case kQ8_0: {
            const uint8_t* b = row + size_t(c) * 34;
            uint8_t* out = dst + L.codes + size_t(r) * n_in + size_t(c) * 32;
            for (int k = 0; k < 32; ++k) out[k] = b[2 + k];
            uint8_t* d = dst + L.d + (size_t(r) * groups + c) * 2;
            d[0] = b[0];
            d[1] = b[1];
            return;
        }
        case kQ4_0: {
            const uint8_t* b = row + size_t(c) * 18;
            for (int k = 0; k < 16; ++k) codes[k] = b[2 + k];
            uint8_t* d = dst + L.d + (size_t(r) * groups + c) * 2;
            d[0] = b[0];
            d[1] = b[1];
            return;
        }
        case kQ4_K: {
            const int s = c >> 3, g = c & 7;
            const uint8_t* sb = row + size_t(s) * 144;
            for (int l = 0; l < 32; ++l) q[l] = uint8_t(q4k_code(sb, 32 * g + l));
            for (int j = 0; j < 16; ++j) codes[j] = uint8_t(q[j] | (q[j + 16] << 4));
            if (g == 0) {
                uint8_t* meta = dst + L.aux + (size_t(r) * (n_in / 256) + s) * 16;
                for (int k = 0; k < 16; ++k) meta[k] = sb[k];
            }
            return;
        }
        case kQ5_K: {
            const int s = c >> 3, g = c & 7;
            const uint8_t* sb = row + size_t(s) * 176;
            for (int l = 0; l < 32; ++l) q[l] = uint8_t(q5k_code(sb, 32 * g + l));
            for (int j = 0; j < 16; ++j) codes[j] = uint8_t((q[j] & 15) | ((q[j + 16] & 15) << 4));
            uint32_t h = 0;  // bit 8b + k: element 4k + b; bit 8b + 4 + k: element 16 + 4k + b
            for (int k = 0; k < 4; ++k)
                for (int b = 0; b < 4; ++b) {
                    h |= uint32_t(q[4 * k + b] >> 4) << (8 * b + k);
                    h |= uint32_t(q[16 + 4 * k + b] >> 4) << (8 * b + 4 + k);
                }
            *reinterpret_cast<uint32_t*>(dst + L.hb + (size_t(r) * groups + c) * 4) = h;
            if (g == 0) {
                uint8_t* meta = dst + L.aux + (size_t(r) * (n_in / 256) + s) * 16;
                for (int k = 0; k < 16; ++k) meta[k] = sb[k];
            }
            return;
        }
        case kQ6_K: {
            const int s = c >> 3, g = c & 7;
            const uint8_t* sb = row + size_t(s) * 210;
            for (int l = 0; l < 32; ++l) q[l] = uint8_t(q6k_code(sb, 32 * g + l));
            for (int j = 0; j < 16; ++j) codes[j] = uint8_t((q[j] & 15) | ((q[j + 16] & 15) << 4));
            uint8_t* qh = dst + L.aux + (size_t(r) * groups + c) * 8;
            for (int half = 0; half < 2; ++half)
                for (int b = 0; b < 4; ++b) {
                    uint8_t v = 0;
                    for (int k = 0; k < 4; ++k) v = uint8_t(v | (((q[16 * half + 4 * k + b] >> 4) & 3) << (2 * k)));
                    qh[4 * half + b] = v;
                }
            if (g == 0) {
                uint8_t* sc = dst + L.sc + size_t(r) * (n_in / 16) + size_t(s) * 16;
                for (int k = 0; k < 16; ++k) sc[k] = sb[192 + k];
                uint8_t* d = dst + L.d + (size_t(r) * (n_in / 256) + s) * 2;
                d[0] = sb[208];
                d[1] = sb[209];
            }
            return;
        }
        default:
            return;
    }
}

}  // namespace

hipError_t launch_repack_rows(uint32_t type, const void* gguf, int n_in, int n_out, int row0, int n_rows, void* dst,
                              hipStream_t stream) {
    const WeightLayout L = weight_layout(type, n_in, n_out);
    if (!L.total || row0 < 0 || n_rows <= 0 || row0 + n_rows > n_out) return hipErrorInvalidValue;
    const long threads = long(n_rows) * (n_in / 32);
    const unsigned blocks = unsigned((threads + 255) / 256);
    hipLaunchKernelGGL(repack_kernel, dim3(blocks), dim3(256), 0, stream, type, static_cast<const uint8_t*>(gguf),
                       n_in, row0, n_rows, gguf_row_bytes(type, n_in), static_cast<uint8_t*>(dst), L);
    return hipGetLastError();
}

hipError_t launch_repack(uint32_t type, const void* gguf, int n_in, int n_out, void* dst, hipStream_t stream) {
    return launch_repack_rows(type, gguf, n_in, n_out, 0, n_out, dst, stream);
}

}  // namespace fishhip
