"""Weight types FISH multiplies in f32 (ops.cpp:219-250): Q4_1, Q5_0, Q5_1,
Q2_K, Q3_K, IQ4_NL, MXFP4, F32, F16, BF16, through the C ABI's
fish_hip_matmul_tensors, against the oracle (oracle/fish_oracle.c
or_matmul_f32path, pinned on FISH's golden dequant_row / matmul_batch) and
the golden outputs themselves. Bar: max error <= 1e-4 of the output's L-inf
norm (both sides sum in f32, in different orders)."""
import numpy as np
import pytest

import imurun_amd as fh
from imurun_amd.synth import normal, uniform

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    fh.load()
    return torch, torch.device("cuda:0")


def rows_of(t, n_out, n_in, seed):
    """Random code bytes with sane f16 scale fields (MXFP4: exponents near 2^0; plain
    float types: N(0, 0.05) values)."""
    if t in (fh.F32, fh.F16, fh.BF16):
        v = normal(seed, (n_out * n_in,), 0.05)
        if t == fh.F32:
            return v.view(np.uint8).copy()
        if t == fh.F16:
            return v.astype(np.float16).view(np.uint8).copy()
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).copy()
    be, bb = fh.BLOCK_ELEMS[t], fh.BLOCK_BYTES[t]
    nb = n_out * n_in // be
    blocks = (uniform(seed, nb * bb) * 256).astype(np.uint8).reshape(nb, bb)

    def f16(s, lo, hi):
        return (lo + uniform(s, nb) * (hi - lo)).astype(np.float32).astype(np.float16).view(np.uint8).reshape(nb, 2)
    if t == fh.MXFP4:
        blocks[:, 0] = (118 + uniform(seed + 1, nb) * 12).astype(np.uint8)
    else:
        off = {fh.Q2_K: 80, fh.Q3_K: 108}.get(t, 0)
        blocks[:, off:off + 2] = f16(seed + 1, 0.001, 0.05)
        if t in (fh.Q4_1, fh.Q5_1):
            blocks[:, 2:4] = f16(seed + 2, -0.5, 0.5)
        if t == fh.Q2_K:
            blocks[:, 82:84] = f16(seed + 2, 0.001, 0.05)
    return blocks.reshape(-1)


def gpu(torch_dev, t, rows, x, n_out):
    torch, d = torch_dev
    n_in = x.shape[1]
    w = fh.repack(t, torch.from_numpy(rows).to(d), n_in, n_out)
    y = fh.matmul_tensors(t, [w], torch.from_numpy(np.ascontiguousarray(x)).to(d), [n_out])[0]
    return y.cpu().numpy()


def check(got, want, what):
    err = float(np.max(np.abs(got - want)))
    scale = float(np.max(np.abs(want)))
    assert err <= TOL * scale, f"{what}: max err {err:.3e} vs {TOL} * {scale:.3e}"


@pytest.mark.parametrize("t", fh.F32_PATH_TYPES)
def test_golden(torch_dev, golden, t):
    g = golden("f32path")
    for m in (1, 3):
        want = g[f"y_{t}_{m}"]
        check(gpu(torch_dev, t, g[f"w_{t}"], g[f"x_{t}_{m}"], want.shape[1]), want, f"{fh.TYPE_NAMES[t]} M={m}")


@pytest.mark.parametrize("t", fh.F32_PATH_TYPES)
@pytest.mark.parametrize("n_out,n_in,n_tok", [(300, 4096, 1), (96, 1024, 5), (40, 2048, 17), (7, 256, 9)])
def test_matches_oracle(torch_dev, oracle, t, n_out, n_in, n_tok):
    rows = rows_of(t, n_out, n_in, 500 + t + n_in)
    x = normal(600 + n_tok + t, (n_tok, n_in), 1.0)
    check(gpu(torch_dev, t, rows, x, n_out), oracle.matmul_f32path(t, rows, x, n_out),
          f"{fh.TYPE_NAMES[t]} {n_out}x{n_in} M={n_tok}")


@pytest.mark.parametrize("t", [fh.Q4_1, fh.Q3_K, fh.MXFP4, fh.F16])
def test_backend_upload_and_group(torch_dev, oracle, t):
    """The backend surface (host buffers, FISH's ComputeBackend contract) takes these types too:
    upload keeps the GGUF bytes, matmul_group on two of them runs the f32 path."""
    b = fh.HipBackend()
    n_in, outs = 1024, [64, 48]
    rows = [rows_of(t, n, n_in, 700 + i + t) for i, n in enumerate(outs)]
    keys = [f"w{t}_{i}" for i in range(2)]
    for k, r, n in zip(keys, rows, outs):
        assert b.upload(k, t, r, n_in, n)
    try:
        for m in (1, 6):
            x = normal(710 + m, (m, n_in), 1.0)
            ys = b.matmul_group(keys, x, outs)
            assert ys is not None, fh.last_error()
            for y, r, n in zip(ys, rows, outs):
                check(y, oracle.matmul_f32path(t, r, x, n), f"{fh.TYPE_NAMES[t]} backend M={m}")
    finally:
        for k in keys:
            b.release(k)


@pytest.mark.parametrize("t", [fh.Q4_1, fh.Q3_K, fh.MXFP4, fh.F16])
def test_full_size_gate_matrix(torch_dev, oracle, t):
    """14336 x 4096 (a Llama-3-8B gate) at one token and at 40 tokens: every row on the GPU,
    a sample of rows against the oracle, and the one-token launch (four rows per wavefront)
    bit-identical to the first token of the 40-token launch (same sums in the same order)."""
    torch, d = torch_dev
    n_out, n_in = 14336, 4096
    rows = rows_of(t, n_out, n_in, 900 + t)
    w = fh.repack(t, torch.from_numpy(rows).to(d), n_in, n_out)
    rb = fh.gguf_row_bytes(t, n_in)
    sel = np.unique(np.concatenate([np.arange(32), (uniform(901, 48) * n_out).astype(int), [n_out - 1]]))
    sub = np.concatenate([rows[i * rb:(i + 1) * rb] for i in sel])
    x = normal(902, (40, n_in), 1.0)
    ys = {}
    for m in (1, 40):
        y = fh.matmul_tensors(t, [w], torch.from_numpy(np.ascontiguousarray(x[:m])).to(d), [n_out])[0].cpu().numpy()
        check(y[:, sel], oracle.matmul_f32path(t, sub, x[:m], sel.size), f"{fh.TYPE_NAMES[t]} full size M={m}")
        ys[m] = y
    assert np.array_equal(ys[1][0], ys[40][0])
