"""The C-ABI library loads and exports what include/fish_hip.h declares (no GPU needed)."""
import os
import re
import subprocess

import numpy as np
import pytest

import imurun_amd as fh

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fish_hip.h")


def declared_symbols():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"FISH_HIP_API\s+[\w\s\*]+?\b(fish_hip_\w+)\s*\(", src)))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "fish_hip_matmul" in names and "fish_hip_quantize" in names and len(names) >= 20


def test_library_exports_every_declared_symbol():
    L = fh.load()
    out = subprocess.run(["nm", "-D", "--defined-only", fh.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\sT\s+(\w+)", out))
    for name in declared_symbols():
        assert name in exported, name
        assert getattr(L, name) is not None


def test_identity():
    L = fh.load()
    assert L.fish_hip_abi_version() == 3
    assert L.fish_hip_kernel_name() == b"hip-gfx950"


@pytest.mark.parametrize("t", [fh.Q8_0, fh.Q4_0, fh.Q4_K, fh.Q5_K, fh.Q6_K])
@pytest.mark.parametrize("n_in,n_out", [(4096, 4096), (4096, 14336), (14336, 4096), (768, 2048), (2048, 768)])
def test_weight_layout_size_matches_gguf(t, n_in, n_out):
    # the repacked copy holds exactly the GGUF bytes plus at most 4 alignment pads
    got = fh.weight_bytes(t, n_in, n_out)
    gguf = fh.gguf_row_bytes(t, n_in) * n_out
    assert gguf <= got <= gguf + 4 * 256


def test_layout_refusals():
    assert fh.weight_bytes(fh.Q4_K, 4000, 16) == 0     # K-quant rows need n_in % 256 == 0
    assert fh.weight_bytes(fh.Q8_0, 48, 16) == 0       # 32-blocks need n_in % 32 == 0
    assert fh.weight_bytes(99, 4096, 16) == 0
    assert fh.act_bytes(4, 48) == 0
    assert fh.act_bytes(1, 4096) >= 4096 * 2 + 4096 // 32 * 8


def test_bad_arguments_return_errors_without_device_work():
    L = fh.load()
    assert L.fish_hip_quantize(None, 1, 4096, None, None, None, None) == -1
    assert "bad arguments" in fh.last_error()
    assert L.fish_hip_matmul(fh.Q4_K, None, None, 1, 4000, 16, None, None) == -1
    assert L.fish_hip_supports(fh.Q4_K) == 1 and L.fish_hip_supports(fh.Q5_K) == 1
    assert all(L.fish_hip_supports(t) == 1 for t in fh.F32_PATH_TYPES)
    assert L.fish_hip_supports(9) == 0 and L.fish_hip_supports(23) == 0  # Q8_1, IQ4_XS
    # quantize_for: only int8-path types, refused before any device work
    assert L.fish_hip_quantize_for(fh.Q4_1, 1 << 20, 1, 256, 1 << 20, None) == -1
    assert L.fish_hip_quantize_for(fh.Q4_K, 1 << 20, 1, 4000, 1 << 20, None) == -1  # 32-blocks only
    assert L.fish_hip_quantize_for(fh.Q4_K, 1 << 20, 1, 4064, 1 << 20, None) == -1  # not whole 256s
    # a type without a block writer is refused
    assert L.fish_hip_quantize_rows(fh.Q4_1, 1 << 20, 1 << 20, 1, 256, 1) == -1
    # f32-path types: only fish_hip_matmul_tensors and the backend take them
    assert L.fish_hip_matmul(fh.Q4_1, 1 << 20, 1 << 20, 1, 256, 16, 1 << 20, None) == -1
    assert L.fish_hip_weight_bytes(fh.Q4_1, 256, 16) == 16 * 8 * 20
    assert L.fish_hip_weight_bytes(fh.Q3_K, 128, 16) == 0  # whole 256-value blocks only
    # moe_ffn: a workspace that is not 256-byte aligned is refused before any device work
    # (the pointers are never dereferenced on this path)
    n_tok, E, F, NE, K = 4, 256, 256, 8, 2
    nb = fh.moe_workspace_bytes(n_tok, E, F, NE, K)
    assert nb > 0
    fake = 1 << 20
    assert L.fish_hip_moe_ffn(fake, fake, n_tok, E, F, NE, K, 1, fh.Q4_K, fake, fh.Q4_K, fake, fh.Q4_K, fake,
                              fake + 16, nb, fake, None) == -1
    assert "aligned" in fh.last_error()
    assert L.fish_hip_moe_ffn(fake, fake, n_tok, E, F, NE, K, 1, fh.Q4_K, fake, fh.Q4_K, fake, fh.Q4_K, fake,
                              fake, nb - 1, fake, None) == -1
    assert "too small" in fh.last_error()
    # router_logits: weight type, row length and alignment are checked before any device work
    assert L.fish_hip_router_logits(fake, 4, 4096, fh.Q8_0, fake, 8, fake, None) == -1
    assert "f32 or f16" in fh.last_error()
    assert L.fish_hip_router_logits(fake, 4, 4094, 0, fake, 8, fake, None) == -1
    assert "multiple of 4" in fh.last_error()
    assert L.fish_hip_router_logits(fake + 8, 4, 4096, 0, fake, 8, fake, None) == -1
    assert "misaligned" in fh.last_error()
    assert L.fish_hip_router_logits(fake, 4, 4096, 0, fake + 8, 8, fake, None) == -1
    assert "misaligned" in fh.last_error()
    assert L.fish_hip_router_logits(fake, 0, 4096, 1, fake, 8, fake, None) == -1
    assert "bad arguments" in fh.last_error()


@pytest.mark.parametrize("t", [fh.Q8_0, fh.Q4_0, fh.Q4_K, fh.Q5_K, fh.Q6_K])
def test_block_writer_matches_golden_and_oracle(golden, oracle, t):
    """The library's host packer (input preparation) writes FISH's bytes."""
    g = golden("pack")
    w = g[f"w_{t}"]
    assert np.array_equal(fh.quantize_rows(t, w.reshape(1, -1)), g[f"packed_{t}"])
    from imurun_amd.synth import normal
    x = normal(31 + t, (64, 1024), 0.02)
    x[3, :256] = 0.0
    x[5, 7] = 9.0
    assert np.array_equal(fh.quantize_rows(t, x, n_threads=3), oracle.quantize_rows(t, x))
