// fish_hip_matmul_tensors_noalloc: matmul_tensors on f32 input for callers
// that cannot allocate device memory (code under HIP graph capture, serving
// loops, hosts that forbid hipMalloc). It is fish_hip_matmul_tensors with the
// activation workspace taken from a fixed device array of this library
// instead of the caller.
//
// The array, `scratch`, is a file-scope __device__ variable: every GPU the
// library runs on holds its own kScratchBytes copy until the process ends.
// Host code never uses the array's name as a device address (it is only a
// host-side handle of the symbol); the address of the current device's copy
// comes from hipGetSymbolAddress, taken once per device on the first call
// made with that device current, and is what the kernels receive.
//
// Calls share the array of their GPU and it keeps the last call's contents.
// Nothing needs to start at zero: the quantizer writes every byte of every
// plane the following matmul reads (including the zero rows that pad the
// last 32-token block). Two calls that overlap on one GPU (different streams,
// or different threads without ordering) race on the array.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "../../include/fish_hip.h"
#include "common.h"
#include "kernels.h"

namespace {

constexpr size_t kScratchBytes = size_t(FISH_HIP_NOALLOC_SCRATCH_MB) << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

// The current device's copy of `scratch` (nullptr and an error message on failure).
void* scratch_for_current_device(std::string& err) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        err = std::string("no current device: ") + hipGetErrorString(e);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
            return nullptr;
        }
        g_ptr[dev] = p;
    }
    return g_ptr[dev];
}

}  // namespace

extern "C" {

uint64_t fish_hip_noalloc_scratch_bytes(void) { return kScratchBytes; }

int fish_hip_matmul_tensors_noalloc(uint32_t type, int n, const void* const* ws, const float* x, int n_tok, int n_in,
                                    const int* n_outs, float* const* ys, void* stream) {
    // one token and the f32-path types need no workspace: the plain entry point as it is
    const uint64_t need = fish_hip_act_bytes(n_tok, n_in);
    if (n_tok > 0 && n_in > 0 && n_in % 32 == 0 && need > kScratchBytes) {
        fishhip::set_last_error("matmul_tensors_noalloc: " + std::to_string(n_tok) + " x " + std::to_string(n_in) +
                                " activations need " + std::to_string(need) + " bytes of scratch, more than the " +
                                std::to_string(kScratchBytes) + " this library holds per device");
        return FISH_HIP_ERR_ARG;
    }
    std::string err;
    void* p = scratch_for_current_device(err);
    if (!p) {
        fishhip::set_last_error("matmul_tensors_noalloc: " + err);
        return FISH_HIP_ERR_DEVICE;
    }
    return fish_hip_matmul_tensors(type, n, ws, x, n_tok, n_in, n_outs, ys, p, kScratchBytes, stream);
}

}  // extern "C"
