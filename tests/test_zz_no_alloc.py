"""fish_hip_matmul_tensors_noalloc through the C ABI against fish_hip_matmul_tensors.

The allocation-free entry point quantizes into the library's fixed per-GPU
array instead of a caller workspace and then runs the same kernels, so its
outputs must equal the workspace entry point's bit for bit; both are held
to the oracle at 1e-4 of max|y|. Two calls in a row, the second smaller
(fewer tokens and a shorter row), show that the array's leftover contents
from the first call do not leak into the second.
"""
import numpy as np
import pytest

import imurun_amd as fh
from imurun_amd.synth import normal

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    fh.load()
    return torch, torch.device("cuda:0")


def dev(torch_dev, a):
    torch, d = torch_dev
    return torch.from_numpy(np.ascontiguousarray(a)).to(d)


def one_call(torch_dev, oracle, t, n_tok, n_in, n_outs, seed):
    torch, d = torch_dev
    rows = [oracle.quantize_rows(t, normal(seed + i, (n, n_in), 0.02)) for i, n in enumerate(n_outs)]
    x = normal(seed + 10, (n_tok, n_in))
    xd = dev(torch_dev, x)
    ws = [fh.repack(t, dev(torch_dev, r), n_in, n) for r, n in zip(rows, n_outs)]
    want_dev = fh.matmul_tensors(t, ws, xd, n_outs)                       # caller's workspace
    ys = [torch.full((n_tok, n), float("nan"), dtype=torch.float32, device=d) for n in n_outs]
    got_dev = fh.matmul_tensors_noalloc(t, ws, xd, n_outs, ys)            # the library's array
    for r, n, g, w in zip(rows, n_outs, got_dev, want_dev):
        got, want = g.cpu().numpy(), w.cpu().numpy()
        assert np.array_equal(got, want), f"{fh.TYPE_NAMES[t]} M={n_tok} n_out={n}: differs from the workspace call"
        ref = oracle.matmul_f32(t, r, x, n)
        err = float(np.max(np.abs(got - ref)))
        assert err <= TOL * float(np.max(np.abs(ref))), f"{fh.TYPE_NAMES[t]} M={n_tok}: err {err:.3e}"


# (first call, second smaller call): batch kernel, GEMM, GEMV-sized and one token
@pytest.mark.parametrize("t", [fh.Q4_0, fh.Q8_0, fh.Q4_K, fh.Q5_K, fh.Q6_K])
@pytest.mark.parametrize("first,second", [((130, 2048), (20, 1024)), ((64, 1024), (3, 512)),
                                          ((300, 4096), (65, 768)), ((9, 1024), (1, 1024))])
def test_noalloc_matches_workspace_entry_point(torch_dev, oracle, t, first, second):
    if fh.BLOCK_ELEMS[t] == 256 and (first[1] % 256 or second[1] % 256):
        pytest.skip("K-quant rows are whole 256-value super-blocks")
    one_call(torch_dev, oracle, t, *first, [160, 48], 4000 + t)
    one_call(torch_dev, oracle, t, *second, [96], 4100 + t)


def test_noalloc_refuses_sizes_beyond_its_array(torch_dev):
    torch, d = torch_dev
    cap = fh.noalloc_scratch_bytes()
    assert cap == 32 << 20
    n_tok, n_in = 1024, 14336
    assert fh.act_bytes(n_tok, n_in) > cap
    w = torch.zeros(fh.weight_bytes(fh.Q4_K, n_in, 32), dtype=torch.uint8, device=d)
    x = torch.zeros((n_tok, n_in), dtype=torch.float32, device=d)
    y = torch.zeros((n_tok, 32), dtype=torch.float32, device=d)
    with pytest.raises(fh.FishHipError, match="scratch"):
        fh.matmul_tensors_noalloc(fh.Q4_K, [w], x, [32], [y])
    torch.cuda.synchronize()
    assert float(y.abs().max()) == 0.0  # refused before any device work
