"""Per-block integers through every matmul kernel, bit for bit, and full-range f16 scales.

The per-block int32 sums of FISH's kernels (quant_x86.cpp:280-495) are pinned
bit-exactly by fish_hip_block_ints, which shares its integer code with the
GEMV. The MFMA kernels (the 16x16 few-token batch kernel, the two-plane
32x32 GEMM, their grouped and work-list forms) form the same integers in
another way -- Q4_K: sc = 8a + b split into two int8 planes, I = 8H + L;
Q5_K / Q6_K: 64 hi + lo; the mins term J on an f16 MFMA -- and reach the
output only through f32 scaling. Here the scaling is made exact so that the
output IS the integer:
  - weights: random codes, sub-block scales and mins, but every f16 block
    scale d (and Q4_K / Q5_K dmin) is 1.0;
  - activations: integers in [-127, 127], every 32-value block holding a
    +-127, so FISH's Q8Act and Q8ActK scales are 127 / 127 = 1.0 and the
    int8 codes are the values themselves.
Then y[t][r] = sum over blocks of (sumi - mins) (Q6_K, Q8_0, Q4_0: of the
block integer), every term an integer; the test asserts beforehand that the
sum of their magnitudes is below 2^24, so any f32 summation order is exact,
and then requires the GPU output to equal that integer exactly.
"""
import numpy as np
import pytest

import imurun_amd as fh
from imurun_amd.synth import normal, uniform

pytestmark = pytest.mark.gpu

TYPES = [fh.Q8_0, fh.Q4_0, fh.Q4_K, fh.Q5_K, fh.Q6_K]
KQ = [fh.Q4_K, fh.Q5_K, fh.Q6_K]
ONE = np.array([1.0], np.float16).view(np.uint8)


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    fh.load()
    return torch, torch.device("cuda:0")


def dev(torch_dev, a):
    torch, d = torch_dev
    return torch.from_numpy(np.ascontiguousarray(a)).to(d)


def unit_scale_rows(t, n_out, n_in, seed):
    """GGUF rows of random bytes whose f16 block scales (and K-quant mins scales) are 1.0."""
    be, bb = fh.BLOCK_ELEMS[t], fh.BLOCK_BYTES[t]
    nb = n_out * n_in // be
    blocks = (uniform(seed, nb * bb) * 256).astype(np.uint8).reshape(nb, bb)
    if t == fh.Q6_K:
        blocks[:, 208:210] = ONE
    else:
        blocks[:, 0:2] = ONE
        if t in (fh.Q4_K, fh.Q5_K):
            blocks[:, 2:4] = ONE
    return blocks.reshape(-1)


def integer_acts(n_tok, n_in, seed):
    """Integer-valued f32 activations in [-24, 24] with one +-127 per 32-value block."""
    x = np.round(normal(seed, (n_tok, n_in)) * np.float32(8.0)).clip(-24, 24).astype(np.float32)
    pos = (uniform(seed + 1, n_tok * n_in // 32) * 32).astype(np.int64).clip(0, 31)
    sign = np.where(uniform(seed + 2, pos.size) < 0.5, -1.0, 1.0).astype(np.float32)
    xb = x.reshape(-1, 32)
    xb[np.arange(xb.shape[0]), pos] = 127.0 * sign
    return xb.reshape(n_tok, n_in)


def exact_outputs(oracle, t, rows, x, n_out):
    """The integer each output must equal, from the oracle's per-block integers."""
    n_tok, n_in = x.shape
    a32, a256 = oracle.act_batch(x)
    # the quantizer really has unit scales and identity codes on these inputs
    assert np.all(a32.reshape(-1, 40)[:, :4].copy().view(np.float32) == 1.0)
    rb = fh.gguf_row_bytes(t, n_in)
    k_layout = fh.BLOCK_ELEMS[t] == 256
    per_tok = (n_in // 256 * 276) if k_layout else (n_in // 32 * 40)
    acts = a256 if k_layout else a32
    out = np.zeros((n_tok, n_out), np.int64)
    mag = np.zeros((n_tok, n_out), np.int64)
    for i in range(n_tok):
        a = acts[i * per_tok:(i + 1) * per_tok]
        for r in range(n_out):
            ints = oracle.block_dots(t, rows[r * rb:(r + 1) * rb], a, n_in).astype(np.int64)
            if t in (fh.Q4_K, fh.Q5_K):
                out[i, r] = int(np.sum(ints[0::2]) - np.sum(ints[1::2]))
            else:
                out[i, r] = int(np.sum(ints))
            mag[i, r] = int(np.sum(np.abs(ints)))
    # precondition: every partial sum in any order is an integer below 2^24, so exact in f32
    assert int(mag.max()) < (1 << 24), f"test data too large for exact f32 sums: {int(mag.max())}"
    return out.astype(np.float32)


def check_exact(got, want, what):
    bad = np.argwhere(got != want)
    assert bad.size == 0, (f"{what}: {bad.shape[0]} outputs differ, first at {tuple(bad[0])}: "
                           f"got {got[tuple(bad[0])]!r} want {want[tuple(bad[0])]!r}")


# M <= 4: GEMV; 5..64: the 16x16 MFMA batch kernel; > 64 (K-quants): the two-plane GEMM
@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_tok", [1, 3, 5, 16, 33, 64, 65, 130, 300])
def test_kernel_integers_bit_exact(torch_dev, oracle, t, n_tok):
    n_in, n_out = 1024, 96
    rows = unit_scale_rows(t, n_out, n_in, 3000 + t)
    x = integer_acts(n_tok, n_in, 3100 + n_tok)
    want = exact_outputs(oracle, t, rows, x, n_out)
    w = fh.repack(t, dev(torch_dev, rows), n_in, n_out)
    got = fh.matmul_batch(t, w, dev(torch_dev, x), n_out).cpu().numpy()
    check_exact(got, want, f"{fh.TYPE_NAMES[t]} M={n_tok}")


@pytest.mark.parametrize("t", KQ)
@pytest.mark.parametrize("n_tok", [20, 200])
def test_grouped_launch_integers_bit_exact(torch_dev, oracle, t, n_tok):
    """matmul_group: tensors of different heights in one grouped GEMM launch (M > 64) or
    per-tensor batch launches, one quantization."""
    n_in, n_outs = 512, [64, 32, 160]
    rows = [unit_scale_rows(t, n, n_in, 3200 + i) for i, n in enumerate(n_outs)]
    x = integer_acts(n_tok, n_in, 3300 + n_tok)
    act = fh.quantize(dev(torch_dev, x))
    ws = [fh.repack(t, dev(torch_dev, r), n_in, n) for r, n in zip(rows, n_outs)]
    ys = fh.matmul_group(t, ws, act, n_tok, n_in, n_outs)
    for r, n, y in zip(rows, n_outs, ys):
        check_exact(y.cpu().numpy(), exact_outputs(oracle, t, r, x, n), f"{fh.TYPE_NAMES[t]} group n_out={n}")


@pytest.mark.parametrize("t", TYPES)
def test_one_token_fused_integers_bit_exact(torch_dev, oracle, t):
    """One token on f32 input: every workgroup quantizes x itself (gemv_x)."""
    n_in, n_outs = 2048, [130, 64]
    rows = [unit_scale_rows(t, n, n_in, 3400 + i) for i, n in enumerate(n_outs)]
    x = integer_acts(1, n_in, 3500)
    ws = [fh.repack(t, dev(torch_dev, r), n_in, n) for r, n in zip(rows, n_outs)]
    ys = fh.matmul_tensors(t, ws, dev(torch_dev, x), n_outs)
    for r, n, y in zip(rows, n_outs, ys):
        check_exact(y.cpu().numpy(), exact_outputs(oracle, t, r, x, n), f"{fh.TYPE_NAMES[t]} fused n_out={n}")


@pytest.mark.parametrize("n_tok,types", [(40, (fh.Q4_K, fh.Q5_K, fh.Q6_K)), (3, (fh.Q4_0, fh.Q8_0, fh.Q4_K)),
                                         (1, (fh.Q4_K, fh.Q4_K, fh.Q6_K))])
def test_expert_gate_up_integers_bit_exact(torch_dev, oracle, n_tok, types):
    """Expert FFN: the gate and up products of every (token, expert) slot -- the work-list
    batch kernel (40 tokens over 8 experts), the work-list GEMV (3 tokens, at most one per expert
    on average) and the one-token
    expert kernel -- equal the integers of the slot's expert rows against its token."""
    torch, d = torch_dev
    tg, tu, td = types
    n_embd, n_ff, n_expert, k = 512, 256, 8, 2
    pg = unit_scale_rows(tg, n_expert * n_ff, n_embd, 3600)
    pu = unit_scale_rows(tu, n_expert * n_ff, n_embd, 3601)
    pd = unit_scale_rows(td, n_expert * n_embd, n_ff, 3602)
    x = integer_acts(n_tok, n_embd, 3700 + n_tok)
    logits = normal(3800 + n_tok, (n_tok, n_expert))
    wg = fh.repack(tg, dev(torch_dev, pg), n_embd, n_expert * n_ff)
    wu = fh.repack(tu, dev(torch_dev, pu), n_embd, n_expert * n_ff)
    wd = fh.repack(td, dev(torch_dev, pd), n_ff, n_expert * n_embd)
    ws = torch.empty(fh.moe_workspace_bytes(n_tok, n_embd, n_ff, n_expert, k), dtype=torch.uint8, device=d)
    fh.moe_ffn(dev(torch_dev, x), dev(torch_dev, logits), n_ff, n_expert, k, True, tg, wg, tu, wu, td, wd,
               workspace=ws)
    p = {n: v.cpu().numpy() for n, v in fh.moe_parts(ws, n_tok, n_embd, n_ff, n_expert, k).items()}
    for name, t, packed in (("gate", tg, pg), ("up", tu, pu)):
        rb = fh.gguf_row_bytes(t, n_embd) * n_ff
        for tok in range(n_tok):
            for c in range(k):
                e, slot = int(p["sel"][tok, c]), int(p["tok_slot"][tok, c])
                want = exact_outputs(oracle, t, packed[e * rb:(e + 1) * rb], x[tok:tok + 1], n_ff)[0]
                check_exact(p[name][slot], want, f"{name} {fh.TYPE_NAMES[t]} token {tok} expert {e}")


# ------------------------------------------------------------------ full-range f16 scales

SCALE_CLASSES = {"subnormal": (0, 0), "tiny": (1, 4), "mid": (11, 19), "large": (26, 30)}


def full_range_rows(t, n_out, n_in, seed):
    """Random bytes whose f16 scales (d, and dmin for Q4_K / Q5_K) are random bit patterns of
    either sign; row r draws its exponent field from class r % 4: 0 (subnormal), 1..4, 11..19 or
    26..30 (up to 2^15 * 2047 / 1024). No infinity or NaN."""
    be, bb = fh.BLOCK_ELEMS[t], fh.BLOCK_BYTES[t]
    nb_row = n_in // be
    nb = n_out * nb_row
    blocks = (uniform(seed, nb * bb) * 256).astype(np.uint8).reshape(nb, bb)
    cls = np.repeat(np.arange(n_out) % 4, nb_row)
    lo = np.array([v[0] for v in SCALE_CLASSES.values()])[cls]
    hi = np.array([v[1] for v in SCALE_CLASSES.values()])[cls]

    def scales(s):
        e = lo + (uniform(s, nb) * (hi - lo + 1)).astype(np.int64).clip(0, hi - lo)
        m = (uniform(s + 1, nb) * 1024).astype(np.int64).clip(0, 1023)
        m = np.where((e == 0) & (m == 0), 1, m)  # subnormal class: never zero
        sgn = (uniform(s + 2, nb) < 0.5).astype(np.int64)
        return ((sgn << 15) | (e << 10) | m).astype(np.uint16).view(np.uint8).reshape(nb, 2)

    off = 208 if t == fh.Q6_K else 0
    blocks[:, off:off + 2] = scales(seed + 10)
    if t in (fh.Q4_K, fh.Q5_K):
        blocks[:, 2:4] = scales(seed + 20)
    return blocks.reshape(-1), np.arange(n_out) % 4


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_tok", [1, 20, 130])
def test_matmul_full_range_scales(torch_dev, oracle, t, n_tok):
    """Subnormal, tiny, mid-range and large f16 block scales of both signs reach the device
    decode: each class of rows is held to 1e-4 of its own largest output (rows of one class
    only, so large rows do not swamp subnormal ones)."""
    n_in, n_out = 1024, 64
    rows, cls = full_range_rows(t, n_out, n_in, 3900 + t)
    x = normal(3950 + n_tok, (n_tok, n_in))
    w = fh.repack(t, dev(torch_dev, rows), n_in, n_out)
    got = fh.matmul_batch(t, w, dev(torch_dev, x), n_out).cpu().numpy()
    want = oracle.matmul_f32(t, rows, x, n_out)
    assert np.all(np.isfinite(got))
    for c, name in enumerate(SCALE_CLASSES):
        sel = cls == c
        err = float(np.max(np.abs(got[:, sel] - want[:, sel])))
        scale = float(np.max(np.abs(want[:, sel])))
        assert scale > 0.0
        assert err <= 1e-4 * scale, f"{fh.TYPE_NAMES[t]} M={n_tok} {name} rows: err {err:.3e} vs 1e-4 * {scale:.3e}"
