"""Parity of the HIP path (through the C ABI) with the oracle and the golden vectors.

Bars: int8 activations, f32 activation scales and per-block int32 dot sums
bit-exact; f32 outputs within 1e-4 * max|y_ref| (max abs error over the
output), y_ref being FISH's CPU result on identical inputs.
"""
import numpy as np
import pytest

import imurun_amd as fh
from imurun_amd.synth import normal, uniform

pytestmark = pytest.mark.gpu

TOL = 1e-4
TYPES = [fh.Q8_0, fh.Q4_0, fh.Q4_K, fh.Q5_K, fh.Q6_K]
GOLDEN_TYPES = [fh.Q8_0, fh.Q4_0, fh.Q4_K, fh.Q6_K]  # tests/golden/matmul.npz


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    fh.load()
    return torch, torch.device("cuda:0")


def dev_u8(torch_dev, a):
    torch, d = torch_dev
    return torch.from_numpy(np.ascontiguousarray(a, np.uint8)).to(d)


def dev_f32(torch_dev, a):
    torch, d = torch_dev
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(d)


def packed_weights(oracle, t, n_out, n_in, seed, std=0.02):
    return oracle.quantize_rows(t, normal(seed, (n_out, n_in), std))


def random_rows(t, n_out, n_in, seed):
    """Random bytes with sane f16 scales: every code / scale bit pattern (test_kernels.cpp:89-107)."""
    be, bb = fh.BLOCK_ELEMS[t], fh.BLOCK_BYTES[t]
    nb = n_out * n_in // be
    blocks = (uniform(seed, nb * bb) * 256).astype(np.uint8).reshape(nb, bb)
    sc = (0.001 + uniform(seed + 1, 2 * nb) * 0.05).astype(np.float32).astype(np.float16).view(np.uint16)
    sc = sc.reshape(nb, 2)
    d_off = 208 if t == fh.Q6_K else 0
    blocks[:, d_off:d_off + 2] = sc[:, :1].view(np.uint8).reshape(nb, 2)
    if t in (fh.Q4_K, fh.Q5_K):
        blocks[:, 2:4] = sc[:, 1:].view(np.uint8).reshape(nb, 2)
    return blocks.reshape(-1)


def gpu_matmul(torch_dev, t, packed, x, n_out):
    n_tok, n_in = x.shape
    w = fh.repack(t, dev_u8(torch_dev, packed), n_in, n_out)
    y = fh.matmul_batch(t, w, dev_f32(torch_dev, x), n_out)
    return y.cpu().numpy()


def check_close(got, want, what):
    err = float(np.max(np.abs(got - want)))
    scale = float(np.max(np.abs(want)))
    assert err <= TOL * scale, f"{what}: max err {err:.3e} vs {TOL} * {scale:.3e}"


# ------------------------------------------------------------------ quantizer

@pytest.mark.parametrize("n", [256, 4096])
@pytest.mark.parametrize("kind", [0, 1, 2, 3])
def test_quantizer_matches_golden_bytes(torch_dev, golden, n, kind):
    g = golden("acts")
    x = dev_f32(torch_dev, g[f"x_{n}_{kind}"].reshape(1, n))
    _, q32, q256 = fh.quantize(x, fish_layouts=True)
    assert np.array_equal(q32.cpu().numpy(), g[f"q32_{n}_{kind}"])
    assert np.array_equal(q256.cpu().numpy(), g[f"q256_{n}_{kind}"])


@pytest.mark.parametrize("n_tok,n_in", [(1, 4096), (7, 14336), (64, 2048), (33, 768), (5, 96), (3, 32)])
def test_quantizer_batches_match_oracle(torch_dev, oracle, n_tok, n_in):
    x = normal(1000 + n_tok + n_in, (n_tok, n_in)) * np.float32(2.0)
    x[0, :32] = 0.0                                      # a zero block
    if n_in >= 64:
        x[-1, 32:64] *= np.float32(50.0)                 # an outlier block
    _, q32, q256 = fh.quantize(dev_f32(torch_dev, x), fish_layouts=True)
    w32, w256 = oracle.act_batch(x)
    assert np.array_equal(q32.cpu().numpy(), w32)
    if n_in % 256 == 0:
        assert np.array_equal(q256.cpu().numpy(), w256)
    else:
        assert q256 is None


# ------------------------------------------------------------------ per-block integers

@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_in", [256, 768, 4096])
@pytest.mark.parametrize("mode", ["packed", "random"])
def test_block_ints_bit_exact(torch_dev, oracle, t, n_in, mode):
    n_out = 48
    rows = packed_weights(oracle, t, n_out, n_in, 77 + n_in) if mode == "packed" else random_rows(t, n_out, n_in, 78)
    x = normal(90 + n_in, (1, n_in)) * np.float32(1.5)
    a32, a256 = oracle.act_batch(x)
    w = fh.repack(t, dev_u8(torch_dev, rows), n_in, n_out)
    act = fh.quantize(dev_f32(torch_dev, x))
    got = fh.block_ints(t, w, act, n_in, n_out).cpu().numpy()
    rb = fh.gguf_row_bytes(t, n_in)
    acts = a32 if fh.BLOCK_ELEMS[t] == 32 else a256
    want = np.concatenate([oracle.block_dots(t, rows[i * rb:(i + 1) * rb], acts, n_in) for i in range(n_out)])
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ matmul

@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_tok", [1, 2, 3, 4, 5, 8, 9, 16, 33, 130])
def test_matmul_matches_oracle(torch_dev, oracle, t, n_tok):
    n_in, n_out = (768 if fh.BLOCK_ELEMS[t] == 256 else 736), 96
    rows = packed_weights(oracle, t, n_out, n_in, 300 + n_tok)
    x = normal(400 + n_tok, (n_tok, n_in))
    got = gpu_matmul(torch_dev, t, rows, x, n_out)
    want = oracle.matmul_f32(t, rows, x, n_out)
    check_close(got, want, f"{fh.TYPE_NAMES[t]} M={n_tok}")


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_in", [1024, 736])
@pytest.mark.parametrize("n_tok", [1, 4, 5, 64, 65, 130])
def test_quantize_for_type_feeds_the_same_matmul(torch_dev, oracle, t, n_in, n_tok):
    """fish_hip_quantize_for writes only the planes that the type's kernel at n_tok reads:
    the matmul on it equals the matmul on the full quantization bit for bit. Its buffer
    starts as 0xA5 bytes, so a plane read but not written would show as a difference."""
    if fh.BLOCK_ELEMS[t] == 256 and n_in % 256:
        pytest.skip("K-quant rows are whole 256-value blocks")
    torch, d = torch_dev
    n_out = 96
    rows = packed_weights(oracle, t, n_out, n_in, 1300 + n_tok)
    x = dev_f32(torch_dev, normal(1400 + n_tok, (n_tok, n_in)))
    w = fh.repack(t, dev_u8(torch_dev, rows), n_in, n_out)
    full = fh.quantize(x)
    part = torch.full((fh.act_bytes(n_tok, n_in),), 0xA5, dtype=torch.uint8, device=d)
    fh.quantize(x, act=part, for_type=t)
    y_full = fh.matmul(t, w, full, n_tok, n_in, n_out).cpu().numpy()
    y_part = fh.matmul(t, w, part, n_tok, n_in, n_out).cpu().numpy()
    assert np.array_equal(y_full.view(np.uint32), y_part.view(np.uint32)), f"{fh.TYPE_NAMES[t]} M={n_tok}"
    check_close(y_part, oracle.matmul_f32(t, rows, x.cpu().numpy(), n_out), f"{fh.TYPE_NAMES[t]} M={n_tok}")


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_tok", [5, 16, 17, 33, 64, 100])
def test_batch_tiles_match_oracle(torch_dev, oracle, t, n_tok):
    """Token counts across the MFMA batch kernel's 16/32/64-token workgroups
    (and K split four or two ways), with 5 units of K and 80 rows."""
    n_in, n_out = 1280, 80
    rows = packed_weights(oracle, t, n_out, n_in, 800 + n_tok)
    x = normal(900 + n_tok, (n_tok, n_in))
    got = gpu_matmul(torch_dev, t, rows, x, n_out)
    check_close(got, oracle.matmul_f32(t, rows, x, n_out), f"{fh.TYPE_NAMES[t]} batch M={n_tok}")


@pytest.mark.parametrize("t", TYPES)
def test_matmul_random_codes(torch_dev, oracle, t):
    n_in, n_out, n_tok = 1024, 80, 20
    rows = random_rows(t, n_out, n_in, 501)
    x = normal(502, (n_tok, n_in))
    got = gpu_matmul(torch_dev, t, rows, x, n_out)
    want = oracle.matmul_f32(t, rows, x, n_out)
    check_close(got, want, f"{fh.TYPE_NAMES[t]} random codes")


@pytest.mark.parametrize("t", GOLDEN_TYPES)
@pytest.mark.parametrize("k", [512, 768])
def test_matmul_matches_reference_golden(torch_dev, golden, t, k):
    g = golden("matmul")
    for m in (1, 3, 17):
        want = g[f"y_{t}_{k}_{m}"]
        got = gpu_matmul(torch_dev, t, g[f"w_{t}_{k}"], g[f"x_{t}_{k}_{m}"], want.shape[1])
        check_close(got, want, f"{fh.TYPE_NAMES[t]} K={k} M={m}")


@pytest.mark.parametrize("t,n_out,n_in,n_tok", [
    (fh.Q8_0, 4096, 4096, 1),
    (fh.Q4_0, 14336, 4096, 1),
    (fh.Q4_0, 4096, 14336, 1),
    (fh.Q4_K, 14336, 4096, 512),
    (fh.Q6_K, 4096, 14336, 512),
    (fh.Q4_0, 14336, 4096, 512),
    (fh.Q4_K, 14336, 4096, 64),
    (fh.Q4_0, 32784, 512, 130),
    (fh.Q5_K, 14336, 4096, 512),
    (fh.Q5_K, 4096, 14336, 1),
    (fh.Q5_K, 14336, 4096, 40),
])
def test_full_size_shapes(torch_dev, oracle, t, n_out, n_in, n_tok):
    """Full-size shapes: all rows on the GPU; a row/token sample checked against
    the oracle, and row slicing must reproduce the full result: bit for bit, except
    where the slice's small grid takes the GEMM's two-part K split and the full one
    does not (the two halves' sums are then added once more at the end: f32
    rounding of the same sum, bounded here at 1e-6 of the largest output)."""
    torch, d = torch_dev
    rows_np = packed_weights(oracle, t, n_out, n_in, 7, 0.02)
    x = normal(8, (n_tok, n_in))
    w = fh.repack(t, dev_u8(torch_dev, rows_np), n_in, n_out)
    y = fh.matmul_batch(t, w, dev_f32(torch_dev, x), n_out).cpu().numpy()
    rb = fh.gguf_row_bytes(t, n_in)
    sel_rows = np.unique(np.concatenate([np.arange(64), (uniform(9, 64) * n_out).astype(int), [n_out - 1]]))
    sel_tok = np.unique(np.concatenate([np.arange(min(n_tok, 8)), (uniform(10, 8) * n_tok).astype(int)]))
    sub = np.concatenate([rows_np[i * rb:(i + 1) * rb] for i in sel_rows])
    want = oracle.matmul_f32(t, sub, x[sel_tok], sel_rows.size)
    check_close(y[np.ix_(sel_tok, sel_rows)], want, f"{fh.TYPE_NAMES[t]} {n_out}x{n_in} M={n_tok}")
    # row slicing: the first 1024 rows on their own give the same outputs
    w_part = fh.repack(t, dev_u8(torch_dev, rows_np[:1024 * rb]), n_in, 1024)
    y_part = fh.matmul_batch(t, w_part, dev_f32(torch_dev, x), 1024).cpu().numpy()
    split_differs = fh.BLOCK_ELEMS[t] == 256 and n_tok > 64 and (n_in // 256) % 2 == 0
    if split_differs:
        err = float(np.abs(y_part - y[:, :1024]).max())
        assert err <= 1e-6 * float(np.abs(y).max()), err
    else:
        assert np.array_equal(y_part, y[:, :1024])


@pytest.mark.parametrize("t,n_tok", [(fh.Q4_K, 130), (fh.Q6_K, 200), (fh.Q4_K, 512), (fh.Q4_K, 3), (fh.Q4_0, 70),
                                     (fh.Q5_K, 130), (fh.Q5_K, 20)])
def test_matmul_group_matches_single(torch_dev, oracle, t, n_tok):
    """matmul_group over tensors of different heights (one grouped GEMM launch
    for many-token K-quants, per-tensor launches otherwise): every output is
    bit-identical to its own matmul and close to the oracle."""
    n_in, n_outs = 768, [96, 32, 32, 160]
    rows = [packed_weights(oracle, t, n, n_in, 1000 + i) for i, n in enumerate(n_outs)]
    x = normal(1100 + n_tok, (n_tok, n_in))
    act = fh.quantize(dev_f32(torch_dev, x))
    ws = [fh.repack(t, dev_u8(torch_dev, r), n_in, n) for r, n in zip(rows, n_outs)]
    ys = fh.matmul_group(t, ws, act, n_tok, n_in, n_outs)
    for w, r, n, y in zip(ws, rows, n_outs, ys):
        single = fh.matmul(t, w, act, n_tok, n_in, n).cpu().numpy()
        got = y.cpu().numpy()
        assert np.array_equal(got, single)
        check_close(got, oracle.matmul_f32(t, r, x, n), f"{fh.TYPE_NAMES[t]} group n_out={n} M={n_tok}")


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_in", [96, 768, 2048, 4096, 14336])
def test_matmul_tensors_one_token_fused(torch_dev, oracle, t, n_in):
    """One token on f32 input: every workgroup quantizes x itself; the outputs
    are bit-identical to quantize + matmul and close to the oracle."""
    if fh.BLOCK_ELEMS[t] == 256 and n_in % 256:
        pytest.skip("K-quants need n_in % 256 == 0")
    n_outs = [200, 64]
    rows = [packed_weights(oracle, t, n, n_in, 1400 + i) for i, n in enumerate(n_outs)]
    x = normal(1500 + n_in, (1, n_in))
    xd = dev_f32(torch_dev, x)
    ws = [fh.repack(t, dev_u8(torch_dev, r), n_in, n) for r, n in zip(rows, n_outs)]
    ys = fh.matmul_tensors(t, ws, xd, n_outs)
    act = fh.quantize(xd)
    for w, r, n, y in zip(ws, rows, n_outs, ys):
        got = y.cpu().numpy()
        assert np.array_equal(got, fh.matmul(t, w, act, 1, n_in, n).cpu().numpy())
        check_close(got, oracle.matmul_f32(t, r, x, n), f"{fh.TYPE_NAMES[t]} fused K={n_in}")


@pytest.mark.parametrize("t", [fh.Q4_0, fh.Q8_0, fh.Q4_K, fh.Q5_K, fh.Q6_K])
@pytest.mark.parametrize("n_in", [2048, 4096])
def test_matmul_tensors_one_token_many_rows(torch_dev, oracle, t, n_in):
    """Gate/up-sized row counts (more workgroups than fit on the device at
    once), split unevenly between two tensors: bit-identical to quantize +
    matmul, close to the oracle."""
    n_outs = [12000, 9000]
    rows = [packed_weights(oracle, t, n, n_in, 1450 + i) for i, n in enumerate(n_outs)]
    x = normal(1550 + n_in, (1, n_in))
    xd = dev_f32(torch_dev, x)
    ws = [fh.repack(t, dev_u8(torch_dev, r), n_in, n) for r, n in zip(rows, n_outs)]
    ys = fh.matmul_tensors(t, ws, xd, n_outs)
    act = fh.quantize(xd)
    for w, r, n, y in zip(ws, rows, n_outs, ys):
        got = y.cpu().numpy()
        assert np.array_equal(got, fh.matmul(t, w, act, 1, n_in, n).cpu().numpy())
        check_close(got, oracle.matmul_f32(t, r, x, n), f"{fh.TYPE_NAMES[t]} many rows K={n_in}")


@pytest.mark.parametrize("t", [fh.Q4_0, fh.Q4_K])
@pytest.mark.parametrize("n_tok", [3, 130])
def test_matmul_tensors_batches(torch_dev, oracle, t, n_tok):
    """More tokens: quantized into the caller's workspace, then the group matmul."""
    n_in, n_outs = 512, [64, 32]
    rows = [packed_weights(oracle, t, n, n_in, 1600 + i) for i, n in enumerate(n_outs)]
    x = normal(1700 + n_tok, (n_tok, n_in))
    ws = [fh.repack(t, dev_u8(torch_dev, r), n_in, n) for r, n in zip(rows, n_outs)]
    ys = fh.matmul_tensors(t, ws, dev_f32(torch_dev, x), n_outs)
    for r, n, y in zip(rows, n_outs, ys):
        check_close(y.cpu().numpy(), oracle.matmul_f32(t, r, x, n), f"{fh.TYPE_NAMES[t]} tensors M={n_tok}")


# ------------------------------------------------------------------ backend surface

def test_backend_matmul_group_grouped_gemm(torch_dev, oracle):
    """q/k/v-shaped Q4_K tensors at a prefill batch: the backend's grouped launch."""
    be = fh.HipBackend()
    n_in, n_outs = 512, {"gq": 128, "gk": 32, "gv": 32}
    packed = {}
    for i, (name, n_out) in enumerate(n_outs.items()):
        packed[name] = packed_weights(oracle, fh.Q4_K, n_out, n_in, 1200 + i)
        assert be.upload(name, fh.Q4_K, packed[name], n_in, n_out)
    x = normal(1300, (150, n_in))
    ys = be.matmul_group(list(n_outs), x, list(n_outs.values()))
    for (name, n_out), y in zip(n_outs.items(), ys):
        check_close(y, oracle.matmul_f32(fh.Q4_K, packed[name], x, n_out), f"backend group {name}")
        assert np.array_equal(be.matmul(name, x, n_out), y)
    for name in n_outs:
        be.release(name)


def test_backend_upload_matmul_group(torch_dev, oracle):
    be = fh.HipBackend()
    assert be.available() and be.device_name()
    n_in = 1024
    ts = {"q": (fh.Q4_K, 256), "k": (fh.Q6_K, 128), "v": (fh.Q8_0, 64), "o": (fh.Q4_0, 96)}
    packed = {}
    for i, (name, (t, n_out)) in enumerate(ts.items()):
        packed[name] = packed_weights(oracle, t, n_out, n_in, 600 + i)
        before = be.bytes_resident()
        assert be.upload(name, t, packed[name], n_in, n_out)
        assert be.resident(name) and be.bytes_resident() > before
    for n_tok in (1, 6, 40):
        x = normal(700 + n_tok, (n_tok, n_in))
        ys = be.matmul_group(list(ts), x, [n for _, n in ts.values()])
        assert ys is not None
        for (name, (t, n_out)), y in zip(ts.items(), ys):
            check_close(y, oracle.matmul_f32(t, packed[name], x, n_out), f"backend {name} M={n_tok}")
        y1 = be.matmul("q", x, 256)
        assert np.array_equal(y1, ys[0])
    # refusals leave the caller to compute on the CPU
    assert be.matmul("missing", normal(1, (1, n_in)), 16) is None
    assert be.matmul("q", normal(1, (1, n_in)), 255) is None
    be.release("q")
    assert not be.resident("q")


@pytest.mark.parametrize("types", [(fh.Q4_K, fh.Q4_K, fh.Q6_K), (fh.Q5_K, fh.Q6_K, fh.Q5_K), (fh.Q6_K, fh.Q4_K, fh.Q5_K)],
                         ids=["q4k-q4k-q6k", "q5k-q6k-q5k", "three-types"])
@pytest.mark.parametrize("n_in,n_outs", [(2048, [1024, 256, 256]), (4096, [1024, 256, 256]),
                                         (8192, [1024, 256, 256]), (4096, [4096, 1024, 1024])])
def test_backend_one_token_mixed_types(torch_dev, oracle, types, n_in, n_outs):
    """One token through a q/k/v-shaped group of mixed K-quant types (a Q4_K_M layer's q, k in
    Q4_K and v in Q6_K): two types share one launch, each workgroup taking its tensor's type's
    path on the same quantized x; a third type falls back to one launch per type. Small groups
    run half the rows per wavefront, Llama-3-8B's q/k/v the default. Bit-identical to each
    tensor alone, and close to the oracle."""
    be = fh.HipBackend()
    names = [f"mx{i}_{n_in}_{n_outs[0]}" for i in range(3)]
    packed = []
    for i, (name, t, n_out) in enumerate(zip(names, types, n_outs)):
        packed.append(packed_weights(oracle, t, n_out, n_in, 1600 + i + n_in))
        assert be.upload(name, t, packed[-1], n_in, n_out)
    x = normal(1700 + n_in, (1, n_in))
    ys = be.matmul_group(names, x, n_outs)
    for name, t, p, n_out, y in zip(names, types, packed, n_outs, ys):
        assert np.array_equal(be.matmul(name, x, n_out), y), f"{name}: group differs from single"
        check_close(y, oracle.matmul_f32(t, p, x, n_out), f"mixed {fh.TYPE_NAMES[t]} K={n_in}")
    for name in names:
        be.release(name)


@pytest.mark.parametrize("n_tok", [5, 130, 256])
def test_backend_batch_mixed_types(torch_dev, oracle, n_tok):
    """A q/k/v-shaped group of a Q4_K_M layer (q, k Q4_K; v Q6_K) on a batch: at GEMM sizes the
    tensors of each type share one grouped launch (q with k), v runs alone; every output is
    bit-identical to the tensor's own matmul and close to the oracle."""
    be = fh.HipBackend()
    n_in, n_outs, types = 2048, [1024, 256, 256], [fh.Q4_K, fh.Q4_K, fh.Q6_K]
    names = [f"bm{i}_{n_tok}" for i in range(3)]
    packed = []
    for i, (name, t, n_out) in enumerate(zip(names, types, n_outs)):
        packed.append(packed_weights(oracle, t, n_out, n_in, 1800 + i))
        assert be.upload(name, t, packed[-1], n_in, n_out)
    x = normal(1810 + n_tok, (n_tok, n_in))
    ys = be.matmul_group(names, x, n_outs)
    for name, t, p, n_out, y in zip(names, types, packed, n_outs, ys):
        assert np.array_equal(be.matmul(name, x, n_out), y), f"{name}: group differs from single"
        check_close(y, oracle.matmul_f32(t, p, x, n_out), f"mixed batch {fh.TYPE_NAMES[t]} M={n_tok}")
    for name in names:
        be.release(name)


def test_backend_upload_keeps_the_vram_headroom(torch_dev, oracle, monkeypatch):
    """upload() leaves FISH's VRAM headroom free (vram_headroom_bytes, backend.h:171-187): with
    FISH_VRAM_HEADROOM_MB above the free memory the upload is refused (earlier uploads intact),
    also when FISH_VRAM_HEADROOM_PCT says 0 (the MB setting wins); with the percentage alone at 0,
    or the default rule, it succeeds."""
    be = fh.HipBackend()
    n_in, n_out = 1024, 256
    packed = packed_weights(oracle, fh.Q4_K, n_out, n_in, 1900)
    try:
        assert be.upload("headroom.a", fh.Q4_K, packed, n_in, n_out)
        before = be.bytes_resident()
        free_mb = be.memory_free() >> 20
        monkeypatch.setenv("FISH_VRAM_HEADROOM_MB", str(free_mb + 1024))
        assert not be.upload("headroom.b", fh.Q4_K, packed, n_in, n_out)
        assert be.bytes_resident() == before and be.resident("headroom.a") and not be.resident("headroom.b")
        monkeypatch.setenv("FISH_VRAM_HEADROOM_PCT", "0")
        assert not be.upload("headroom.b", fh.Q4_K, packed, n_in, n_out)
        monkeypatch.delenv("FISH_VRAM_HEADROOM_MB")
        assert be.upload("headroom.b", fh.Q4_K, packed, n_in, n_out)
        be.release("headroom.b")
        monkeypatch.delenv("FISH_VRAM_HEADROOM_PCT")
        assert be.upload("headroom.b", fh.Q4_K, packed, n_in, n_out)
        x = normal(1901, (3, n_in))
        assert np.array_equal(be.matmul("headroom.a", x, n_out), be.matmul("headroom.b", x, n_out))
    finally:
        be.release("headroom.a")
        be.release("headroom.b")
