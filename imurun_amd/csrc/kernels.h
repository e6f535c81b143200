// Host-side launchers of the gfx950 kernels (internal to libfish_hip.so).
// Every launcher is asynchronous on `stream` and returns the launch status.
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace fishhip {

// f32 x[n_tok][ldx] -> device activation buffer `act` (act_layout(n_tok, n_in)).
// aos32 / aos256 (nullable) receive FISH's Q8Act / Q8ActK bytes as well.
hipError_t launch_quantize(const float* x, int n_tok, int n_in, int ldx, void* act, void* aos32, void* aos256,
                           hipStream_t stream);

// GGUF rows (device bytes) -> repacked device layout (weight_layout()).
hipError_t launch_repack(uint32_t type, const void* gguf, int n_in, int n_out, void* dst, hipStream_t stream);

// Few-token matmul: y[t * ldy + i] for t < n_tok, i < n_out.
hipError_t launch_gemv(const void* w, const WeightLayout& L, const void* act, int n_tok, float* y, int ldy,
                       hipStream_t stream);

// Many-token matmul on int8 MFMA (K-quants).
hipError_t launch_gemm(const void* w, const WeightLayout& L, const void* act, int n_tok, float* y, int ldy,
                       hipStream_t stream);

// Per-block integer dots of every row with token 0 of `act`.
hipError_t launch_block_ints(const void* w, const WeightLayout& L, const void* act, int32_t* out, hipStream_t stream);

}  // namespace fishhip
