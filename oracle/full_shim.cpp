// Whole-model harness over the reference's own runtime -- TEST INFRASTRUCTURE ONLY.
//
// Linked by oracle/Makefile into _ref/libfish_full_hip.so with FISH's runtime
// sources where they lie (c_api, model, tokenizer, sampler, gguf, ops, quant,
// ...) and the HIP backend binding of imurun_amd/fish_side/hip_backend.cpp,
// which registers itself with FISH at load when a gfx950 device is usable.
// The library then exports FISH's own fish_* C ABI (include/fish/c_api.h), so a
// test loads a GGUF file and generates through FISH's loader, placement and
// forward pass, with every weight matmul routed by matmul_tensor(s)
// (ops.cpp:283-299) to the backend. The one extra entry point switches the
// registered backend off and on, so the same process can also produce FISH's
// CPU-only result for comparison.
#include <fish/backend.h>

using namespace fish;

extern "C" {

// on = 0: FISH sees no GPU backend (the next fish_load places nothing on the
// device); on = 1: the backend registered at load is back. Returns the
// backend's name, or "" when none was registered.
const char* full_set_gpu(int on) {
    static ComputeBackend* registered = gpu_backend();
    set_gpu_backend(on ? registered : nullptr);
    return registered ? registered->name() : "";
}

}  // extern "C"
