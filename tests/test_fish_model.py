"""A whole GGUF model generating through FISH's own runtime and the HIP path.

oracle/_ref/libfish_full_hip.so is FISH's runtime compiled from its sources
where they lie -- the fish_* C ABI (c_api.cpp), the GGUF loader (gguf.cpp),
placement and forward pass (model.cpp), tokenizer and sampler -- plus the
FISH-side backend binding (imurun_amd/fish_side/hip_backend.cpp), which
registers itself at load. The tests bind that C ABI by name with ctypes, as
FISH's Python client does (model/fish_native.py:271-345), write a small random
llama model with tests/gguf_model.py, and generate greedily:
- on the CPU (the backend switched off), FISH's own result;
- with the backend on: FISH's loader uploads every layer's projections and the
  output matrix (model.cpp:1290-1390, spans off), and every weight matmul of
  prefill (one call over the whole prompt) and decode (one token) goes through
  matmul_tensor(s) (ops.cpp:283-299) to the device.
The generated token ids and text must be identical. Greedy decoding flips only
at a near-tie of the two largest logits; the device and CPU logits differ at
f32 rounding, far below the margins of these seeded models. Without the
library (no reference sources at build time) the tests skip.
"""
import ctypes
import os

import pytest

import imurun_amd as fh

from gguf_model import F32, U32, tiny_llama, tiny_model

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FULL_SO = os.path.join(ROOT, "oracle", "_ref", "libfish_full_hip.so")

pytestmark = pytest.mark.skipif(not os.path.exists(FULL_SO), reason="oracle/_ref/libfish_full_hip.so not built")

PROMPT = b"the quick brown fox jumps over the lazy dog and then some more words follow " * 2
N_GEN = 24

# weight types per model: a Q4_K_M-style mix, the 32-block int8 types, and types
# FISH multiplies in f32 (dequantised on the device)
MODELS = {
    "q4_k_m": dict(q=fh.Q4_K, k=fh.Q4_K, v=fh.Q6_K, o=fh.Q4_K, gate=fh.Q4_K, up=fh.Q4_K, down=fh.Q6_K,
                   output=fh.Q6_K, embd=fh.Q4_K),
    "q5_k": dict(q=fh.Q5_K, k=fh.Q5_K, v=fh.Q6_K, o=fh.Q5_K, gate=fh.Q5_K, up=fh.Q5_K, down=fh.Q6_K,
                 output=fh.Q6_K, embd=fh.Q5_K),
    "q8_0_q4_0": dict(q=fh.Q8_0, k=fh.Q8_0, v=fh.Q8_0, o=fh.Q4_0, gate=fh.Q4_0, up=fh.Q4_0, down=fh.Q8_0,
                      output=fh.Q8_0, embd=fh.Q8_0),
    "f32_path": dict(q=fh.Q4_1, k=fh.Q5_0, v=fh.Q5_1, o=fh.IQ4_NL, gate=fh.Q3_K, up=fh.Q2_K, down=fh.MXFP4,
                     output=fh.F16, embd=fh.Q8_0),
}


class FishStats(ctypes.Structure):
    """fish_stats, ABI 4 (include/fish/c_api.h:34-77)."""
    _fields_ = [
        ("load_seconds", ctypes.c_double), ("prefill_seconds", ctypes.c_double),
        ("decode_seconds", ctypes.c_double), ("tokens_per_second", ctypes.c_double),
        ("prompt_tokens", ctypes.c_int), ("generated_tokens", ctypes.c_int),
        ("context_used", ctypes.c_int), ("context_size", ctypes.c_int),
        ("weights_bytes", ctypes.c_ulonglong), ("kv_bytes", ctypes.c_ulonglong),
        ("peak_rss_mb", ctypes.c_double),
        ("truncated", ctypes.c_int), ("cached_tokens", ctypes.c_int), ("n_threads", ctypes.c_int),
        ("streaming", ctypes.c_int), ("prefill_tokens_per_second", ctypes.c_double),
        ("gpu_layers", ctypes.c_int), ("ram_layers", ctypes.c_int), ("disk_layers", ctypes.c_int),
        ("gpu_bytes", ctypes.c_ulonglong), ("gpu_name", ctypes.c_char * 64),
        ("draft_proposed", ctypes.c_int), ("draft_accepted", ctypes.c_int), ("draft_active", ctypes.c_int),
        ("gpu_mix", ctypes.c_char * 160), ("placement", ctypes.c_char * 320), ("load_profile", ctypes.c_char * 400),
        ("vram_total", ctypes.c_ulonglong), ("vram_free", ctypes.c_ulonglong), ("vram_headroom", ctypes.c_ulonglong),
    ]


class FishModelInfo(ctypes.Structure):
    """fish_model_info, ABI 4 (include/fish/c_api.h:79-90)."""
    _fields_ = [
        ("arch", ctypes.c_char * 32), ("n_layers", ctypes.c_int), ("n_embd", ctypes.c_int), ("n_ff", ctypes.c_int),
        ("n_head", ctypes.c_int), ("n_head_kv", ctypes.c_int), ("head_dim", ctypes.c_int), ("n_ctx", ctypes.c_int),
        ("vocab", ctypes.c_int), ("tied_output", ctypes.c_int), ("quant", ctypes.c_char * 64),
        ("n_experts", ctypes.c_int), ("n_experts_per_tok", ctypes.c_int), ("n_ctx_train", ctypes.c_int),
        ("chat_format", ctypes.c_char * 16), ("tokenizer", ctypes.c_char * 8),
    ]


CB = ctypes.CFUNCTYPE(None, ctypes.c_char_p, ctypes.c_int, ctypes.c_void_p)


@pytest.fixture(scope="module")
def fish():
    return open_fish()


def open_fish():
    """FISH's C ABI from the harness library, with the prototypes it is called with."""
    # torch's HIP runtime first: the harness library pulls in libfish_hip.so, and
    # whichever runtime library loads first is the one the whole process shares
    import torch
    torch.cuda.is_available()
    os.environ.setdefault("FISH_THREADS", "8")
    os.environ["FISH_GPU_SPAN"] = "0"  # per-matmul routing (this backend offers no spans)
    lib = ctypes.CDLL(FULL_SO)
    lib.fish_abi_version.restype = ctypes.c_int
    lib.fish_kernel_name.restype = ctypes.c_char_p
    lib.fish_create.restype = ctypes.c_void_p
    lib.fish_destroy.argtypes = [ctypes.c_void_p]
    lib.fish_load.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int]
    lib.fish_last_error.argtypes = [ctypes.c_void_p]
    lib.fish_last_error.restype = ctypes.c_char_p
    lib.fish_model_info_of.argtypes = [ctypes.c_void_p, ctypes.POINTER(FishModelInfo)]
    lib.fish_get_stats.argtypes = [ctypes.c_void_p, ctypes.POINTER(FishStats)]
    lib.fish_generate.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                  ctypes.c_int, ctypes.c_float, ctypes.c_float, CB, ctypes.c_void_p]
    lib.full_set_gpu.argtypes = [ctypes.c_int]
    lib.full_set_gpu.restype = ctypes.c_char_p
    assert lib.fish_abi_version() == 4
    return lib


def run(lib, path, gpu: bool, n_ctx=512):
    """Loads `path` in a fresh context with the backend on or off and generates
    N_GEN tokens greedily. Returns (streamed (text, id) pairs, stats, info)."""
    lib.full_set_gpu(1 if gpu else 0)
    ctx = lib.fish_create()
    try:
        assert lib.fish_load(ctx, path.encode(), n_ctx) == 0, lib.fish_last_error(ctx)
        info = FishModelInfo()
        assert lib.fish_model_info_of(ctx, ctypes.byref(info)) == 0
        out = []
        cb = CB(lambda text, tid, user: out.append((bytes(text), tid)))
        n = lib.fish_generate(ctx, PROMPT, 1, N_GEN, 0.0, 0, 1.0, 1.0, cb, None)
        assert n > 0, lib.fish_last_error(ctx)
        st = FishStats()
        lib.fish_get_stats(ctx, ctypes.byref(st))
        return out, st, info
    finally:
        lib.fish_destroy(ctx)
        lib.full_set_gpu(1)


def test_cpu_generation_of_a_written_model(fish, tmp_path):
    # the GGUF writer's file is what FISH's loader and tokenizer accept; greedy decoding is reproducible
    path = str(tmp_path / "tiny.gguf")
    cfg = tiny_llama(path, MODELS["q4_k_m"], seed=14)
    a, st, info = run(fish, path, gpu=False)
    b, _, _ = run(fish, path, gpu=False)
    assert a == b and len(a) > 0
    assert info.arch == b"llama" and info.n_layers == cfg["n_layers"] and info.n_embd == cfg["n_embd"]
    assert info.n_ff == cfg["n_ff"] and info.vocab == cfg["vocab"] and info.tokenizer == b"spm"
    assert st.generated_tokens == N_GEN and st.prompt_tokens > 64 and st.gpu_layers == 0


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(MODELS))
def test_model_generates_through_the_hip_backend(fish, tmp_path, name):
    from test_gpu_f32path import rows_of
    path = str(tmp_path / f"{name}.gguf")
    cfg = tiny_llama(path, MODELS[name], seed=14, raw=rows_of)
    assert fish.full_set_gpu(1) == b"hip", "the HIP backend did not register (no usable gfx950 device?)"
    cpu, st_cpu, _ = run(fish, path, gpu=False)
    served0 = fh.load().fish_hip_backend_served()
    dev, st, _ = run(fish, path, gpu=True)
    served = fh.load().fish_hip_backend_served() - served0
    assert st_cpu.gpu_layers == 0
    assert st.gpu_layers == cfg["n_layers"], st.placement
    assert st.gpu_bytes > 0 and st.gpu_name
    # prefill: per layer q/k/v, o, gate/up, down (4 calls) + output; then the same per decoded token
    assert served >= (4 * cfg["n_layers"] + 1) * N_GEN
    assert dev == cpu


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["q4_k_m", "q8_0_q4_0"])
def test_model_generates_through_a_layer_span(fish, tmp_path, name):
    # FISH offers its GPU layers as one span (model.cpp:780-850); the backend runs norms,
    # projections, RoPE, the KV cache, attention, SiLU and residuals of both layers on the
    # device, one call per forward (plus the output matmul), token-identical to the CPU
    path = str(tmp_path / f"{name}.gguf")
    tiny_llama(path, MODELS[name], seed=14)
    cpu, _, _ = run(fish, path, gpu=False)
    os.environ["FISH_GPU_SPAN"] = "1"
    os.environ["FISH_GPU_NO_IMPORTANCE"] = "1"
    try:
        served0 = fh.load().fish_hip_backend_served()
        dev, st, _ = run(fish, path, gpu=True)
        served = fh.load().fish_hip_backend_served() - served0
    finally:
        os.environ["FISH_GPU_SPAN"] = "0"
        os.environ.pop("FISH_GPU_NO_IMPORTANCE", None)
    assert st.gpu_layers == 2, st.placement
    # one span call and one output matmul per forward, not per-matmul routing (9 per forward)
    assert st.generated_tokens <= served <= 3 * st.generated_tokens, (served, st.placement, st.gpu_mix)
    assert dev == cpu


@pytest.mark.gpu
def test_model_generates_through_a_span_with_int8_kv(fish, tmp_path):
    # FISH_GPU_KV=q8 makes FISH's planner ask for the int8 KV cache (model.cpp:1019-1036); the
    # span keeps it (one f32 scale per 32 values) and runs both layers through it, one call per
    # forward. The int8 K and V move the logits by a fraction of a percent; on this model greedy
    # decoding still picks the CPU's tokens.
    path = str(tmp_path / "kvq8.gguf")
    tiny_llama(path, MODELS["q4_k_m"], seed=14)
    cpu, _, _ = run(fish, path, gpu=False)
    os.environ["FISH_GPU_SPAN"] = "1"
    os.environ["FISH_GPU_NO_IMPORTANCE"] = "1"
    os.environ["FISH_GPU_KV"] = "q8"
    try:
        served0 = fh.load().fish_hip_backend_served()
        dev, st, _ = run(fish, path, gpu=True)
        served = fh.load().fish_hip_backend_served() - served0
    finally:
        os.environ["FISH_GPU_SPAN"] = "0"
        os.environ.pop("FISH_GPU_NO_IMPORTANCE", None)
        os.environ.pop("FISH_GPU_KV", None)
    assert st.gpu_layers == 2 and b"KV int8" in st.placement, st.placement
    assert st.generated_tokens <= served <= 3 * st.generated_tokens, (served, st.placement)
    assert dev == cpu


# Qwen-family layers: Qwen-3 (per-head q / k RMSNorm, n_head * head_dim != n_embd) and
# Qwen-2 (q / k / v biases), both with FISH's NeoX RoPE; Phi-3 (fused q|k|v and fused
# gate|up); Gemma-2 (post norms, GELU, attention soft cap 5 and a 32-position sliding
# window on even layers -- the prompt is longer -- plus FISH's embedding scale and final soft
# cap outside the span)
QWEN = {
    "qwen3": dict(arch="qwen3", head_dim=128, qk_norm=True),
    "qwen2": dict(arch="qwen2", biases=True),
    "phi3": dict(arch="phi3", fused_qkv=True, fused_gate_up=True),
    "gemma2": dict(arch="gemma2", post_norms=True,
                   extra_meta=(("attn_logit_softcapping", F32, 5.0), ("final_logit_softcapping", F32, 30.0),
                               ("attention.sliding_window", U32, 32))),
}


def test_cpu_generation_of_qwen_models(fish, tmp_path):
    # the written Qwen-family files load in FISH and generate reproducibly on the CPU
    for name, kw in QWEN.items():
        path = str(tmp_path / f"{name}.gguf")
        cfg = tiny_model(path, MODELS["q4_k_m"], seed=15, **kw)
        a, st, info = run(fish, path, gpu=False)
        b, _, _ = run(fish, path, gpu=False)
        assert a == b and st.generated_tokens == N_GEN
        assert info.arch == kw["arch"].encode() and info.n_layers == cfg["n_layers"]


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(QWEN))
def test_qwen_model_generates_through_the_hip_backend(fish, tmp_path, name):
    # per-matmul routing: the projections' shapes follow head_dim (q 512 x 256, o 256 x 512 for qwen3)
    path = str(tmp_path / f"{name}.gguf")
    cfg = tiny_model(path, MODELS["q4_k_m"], seed=15, **QWEN[name])
    cpu, _, _ = run(fish, path, gpu=False)
    dev, st, _ = run(fish, path, gpu=True)
    assert st.gpu_layers == cfg["n_layers"], st.placement
    assert dev == cpu


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(QWEN))
def test_qwen_model_generates_through_a_layer_span(fish, tmp_path, name):
    # the span runs the Qwen-family steps on the device (q / k norms after the projections,
    # biases, NeoX RoPE), one call per forward, token-identical to FISH's CPU forward
    path = str(tmp_path / f"{name}.gguf")
    tiny_model(path, MODELS["q4_k_m"], seed=15, **QWEN[name])
    cpu, _, _ = run(fish, path, gpu=False)
    os.environ["FISH_GPU_SPAN"] = "1"
    os.environ["FISH_GPU_NO_IMPORTANCE"] = "1"
    try:
        served0 = fh.load().fish_hip_backend_served()
        dev, st, _ = run(fish, path, gpu=True)
        served = fh.load().fish_hip_backend_served() - served0
    finally:
        os.environ["FISH_GPU_SPAN"] = "0"
        os.environ.pop("FISH_GPU_NO_IMPORTANCE", None)
    assert st.gpu_layers == 2, st.placement
    assert st.generated_tokens <= served <= 3 * st.generated_tokens, (served, st.placement, st.gpu_mix)
    assert dev == cpu
