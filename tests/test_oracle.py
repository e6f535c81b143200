"""Pins the CPU oracle (oracle/fish_oracle.c) before it is trusted as the checker.

Each function is checked against the reference's golden vectors
(tests/golden/, written by tests/golden/make_golden.py from FISH's own CPU
path) and against facts that do not come from the oracle: IEEE binary16
(numpy), the closed form of the activation quantizer, the Q4_K known-answer
block of test/test_m1.cpp:35-71, a second decoder of the block codes
(tests/fishref_np.py), and FISH's AVX2 dot products rebuilt from the
oracle's per-block integers.
"""
import numpy as np
import pytest

import fishref_np as F
from imurun_amd.synth import normal
from oracle.oracle import F32, F32_PATH_TYPES, Q4_0, Q4_1, Q4_K, Q5_K, Q6_K, Q8_0

TYPES = [Q8_0, Q4_0, Q4_K, Q5_K, Q6_K]


def test_fp16_decode_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.L.or_fp16_to_fp32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_fp16_encode_matches_ieee(oracle):
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(1e-3),
        rng.standard_normal(20000).astype(np.float32) * np.float32(300.0),
        rng.standard_normal(5000).astype(np.float32) * np.float32(3e-6),     # subnormal halves
        rng.standard_normal(2000).astype(np.float32) * np.float32(7e4),      # overflow
        # exact ties between two halves (round to even)
        (np.arange(1, 2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26], np.float32),
    ]).astype(np.float32)
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.L.or_fp32_to_fp16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n", [256, 4096])
@pytest.mark.parametrize("kind", [0, 1, 2, 3])
def test_quantizer_golden(oracle, golden, n, kind):
    g = golden("acts")
    x = g[f"x_{n}_{kind}"]
    assert np.array_equal(oracle.quantize_acts(x), g[f"q32_{n}_{kind}"])
    assert np.array_equal(oracle.quantize_acts_k(x), g[f"q256_{n}_{kind}"])


def test_quantizer_closed_form(oracle):
    xs = [normal(41, 4096) * np.float32(3.0),
          np.where(np.arange(4096) % 7 == 0, np.float32(0.0), normal(42, 4096)).astype(np.float32),
          np.zeros(512, np.float32)]
    # exact ties: one 127 per block pins d = 1, id = 1; k + 0.5 rounds to even
    t = (np.arange(1024) % 200 - 100).astype(np.float32) + np.float32(0.5)
    t[::32] = 127.0
    xs.append(t)
    for x in xs:
        assert np.array_equal(oracle.quantize_acts(x), F.quantize_acts(x, 32))
        assert np.array_equal(oracle.quantize_acts_k(x), F.quantize_acts(x, 256))


def test_tie_rounding_is_half_even(oracle):
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:6] = [0.5, 1.5, 2.5, -0.5, -2.5]
    q = oracle.quantize_acts(x)[8:40].view(np.int8)
    assert list(q[:6]) == [127, 0, 2, 2, 0, -2]


def test_q4k_known_answer_block(oracle):
    raw = np.zeros(144, np.uint8)
    raw[0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)   # d = 1.0, dmin = 0
    raw[4:8] = 1                                                        # scales 0..3 = 1
    raw[12:16] = 1                                                      # scales 4..7 = 1 (low nibble)
    n = (np.arange(128) & 15).astype(np.uint8)
    raw[16:] = n | (n << 4)
    y = oracle.dequant_row(Q4_K, raw, 256)
    want = np.concatenate([np.tile(np.arange(32) & 15, 8)]).astype(np.float32)
    assert np.array_equal(y, want)


@pytest.mark.parametrize("t", TYPES)
def test_packer_and_dequant_golden(oracle, golden, t):
    g = golden("pack")
    w, packed, deq = g[f"w_{t}"], g[f"packed_{t}"], g[f"deq_{t}"]
    assert np.array_equal(oracle.quantize_rows(t, w.reshape(1, -1)), packed)
    assert np.array_equal(oracle.dequant_row(t, packed, w.size).view(np.uint32), deq.view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
def test_dots_and_block_ints(oracle, golden, t):
    g = golden("dots")
    ns, rows, acts = g[f"n_{t}"], g[f"rows_{t}"], g[f"acts_{t}"]
    be, bb = F.BLOCK_ELEMS[t], F.BLOCK_BYTES[t]
    ab = 40 if be == 32 else 276
    ro = ao = 0
    for i, n in enumerate(ns):
        n = int(n)
        row = rows[ro:ro + n // be * bb]
        a = acts[ao:ao + n // (32 if be == 32 else 256) * ab]
        ro += row.size
        ao += a.size
        # f32 dot in FISH's scalar order: bit-identical to the reference's scalar table
        got = np.float32(oracle.vec_dot(t, row, a, n))
        assert got.view(np.uint32) == np.float32(g[f"scalar_{t}"][i]).view(np.uint32)
        # exact integers: oracle == an independent brute force
        ints = oracle.block_dots(t, row, a, n)
        assert np.array_equal(ints.astype(np.int64), F.block_ints(t, row, a, n))
        # and they rebuild FISH's AVX2 result (which is formed from these integers)
        xq = np.zeros(n)
        w = oracle.dequant_row(t, row, n).astype(np.float64)
        for b in range(n // (32 if be == 32 else 256)):
            blk = a[b * ab:(b + 1) * ab]
            d = float(blk[:4].view(np.float32)[0])
            off = 8 if be == 32 else 20
            span = 32 if be == 32 else 256
            xq[b * span:(b + 1) * span] = d * blk[off:off + span].view(np.int8)
        mass = np.abs(w * xq).sum() + 1e-9
        rebuilt = F.dot_from_ints(t, row, a, n, ints)
        assert abs(rebuilt - float(g[f"avx2_{t}"][i])) / mass < 1e-5


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q6_K])
@pytest.mark.parametrize("k", [512, 768])
def test_matmul_golden(oracle, golden, t, k):
    g = golden("matmul")
    w = g[f"w_{t}_{k}"]
    for m in (1, 3, 17):
        x = g[f"x_{t}_{k}_{m}"]
        want = g[f"y_{t}_{k}_{m}"]
        got = oracle.matmul_f32(t, w, x, want.shape[1])
        assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


def test_moe_golden(oracle, golden):
    g = golden("moe")
    E, F_, NE, K = int(g["E"]), int(g["F"]), int(g["NE"]), int(g["K"])
    sel, wsel = oracle.route(g["logits"], K, True)
    assert np.array_equal(sel, g["sel"])
    assert np.allclose(wsel, g["wsel"], rtol=0, atol=1e-6)
    out = oracle.moe_ffn(g["x"], g["logits"], E, F_, NE, K, True, Q4_K, g["gate"], Q4_K, g["up"], Q6_K, g["down"])
    want = g["out"]
    assert np.max(np.abs(out - want)) <= 1e-5 * np.max(np.abs(want))


def test_silu_mul_float64(oracle):
    """silu(g) * u in f32 steps (ops.cpp:25-30, model.cpp:1504-1508) against a float64
    restatement: exp, add, divide and multiply are four f32 roundings (each at most half
    an ulp, exp within one), so the result is within 4 ulps; a dropped factor of u, or
    sigmoid in place of silu, is off by orders of magnitude more."""
    g = normal(91, (4, 4096)) * np.float32(4.0)
    u = normal(92, (4, 4096))
    g[0, :6] = [0.0, -0.0, 80.0, -80.0, 1e-30, -1e-30]
    h = oracle.silu_mul(g, u)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    h64 = g64 / (1.0 + np.exp(-g64)) * u64
    ulp = np.spacing(np.abs(h64).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(h - h64) <= 4 * ulp + 1e-45)
    assert oracle.silu(np.float32(2.0)) == np.float32(2.0) / (np.float32(1.0) + np.exp(np.float32(-2.0)))
    wrong = (g64 / (1.0 + np.exp(-g64)))
    assert np.max(np.abs(h - wrong)) > 1e-2


def _abs_bound(x, w):
    """sum_k |x_k w_k| per (token, row): the scale of f32 rounding in a dot."""
    return np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T


@pytest.mark.parametrize("n", [256, 992])
def test_router_golden_and_float64(oracle, golden, n):
    g = golden("router")
    for t in (0, 1):
        w = g[f"w{t}_{n}"]
        wf = w if t == 0 else w.view(np.float16)
        for m in (1, 5):
            x = g[f"x_{n}_{m}"]
            want = g[f"y{t}_{n}_{m}"]
            got = oracle.router_logits(t, w, x)
            bound = _abs_bound(x, wf)
            if t == 1 and m == 1:
                # vec_dot's f16 branch uses the scalar four-sum dot on 64-value chunks
                # (quant.cpp:537-546), the same order as the oracle: bit-identical.
                assert np.array_equal(got, want)
            assert np.all(np.abs(got - want) <= 1e-6 * bound)
            exact = x.astype(np.float64) @ wf.astype(np.float64).T
            assert np.all(np.abs(got - exact) <= 1e-6 * bound)


def test_router_catches_a_dropped_term(oracle):
    # a dot that misses one product, or uses the transposed operand, is far outside the tolerance above
    n = 992
    x = normal(31, (3, n), 1.0)
    w = normal(32, (8, n), 0.05)
    got = oracle.router_logits(0, w, x)
    bound = _abs_bound(x, w)
    x2 = x.copy()
    x2[:, 17] = 0.0
    dropped = x2.astype(np.float64) @ w.astype(np.float64).T
    assert np.any(np.abs(got - dropped) > 1e-6 * bound)
    shifted = x.astype(np.float64) @ np.roll(w, 1, axis=0).astype(np.float64).T
    assert np.all(np.abs(got - shifted) > 1e-6 * bound)


@pytest.mark.parametrize("t", F32_PATH_TYPES)
def test_f32path_dequant_and_matmul_golden(oracle, golden, t):
    """Types FISH multiplies in f32: dequantised values bit-identical to FISH's
    dequant_row; one token bit-identical to vec_dot (scalar block dots; F32 rows
    go through FISH's AVX2 dot); more tokens within f32 rounding of the AVX2 dot."""
    g = golden("f32path")
    w = g[f"w_{t}"]
    n_out, n_in = 8, 512
    deq = oracle.dequant_row(t, w, n_out * n_in)
    assert np.array_equal(deq.view(np.uint32), g[f"deq_{t}"].view(np.uint32))
    for m in (1, 3):
        x = g[f"x_{t}_{m}"]
        got = oracle.matmul_f32path(t, w, x, n_out)
        want = g[f"y_{t}_{m}"]
        if m == 1 and t != F32:
            assert np.array_equal(got, want)
        bound = np.abs(x.astype(np.float64)) @ np.abs(deq.reshape(n_out, n_in).astype(np.float64)).T
        assert np.all(np.abs(got - want) <= 1e-6 * bound)
        exact = x.astype(np.float64) @ deq.reshape(n_out, n_in).astype(np.float64).T
        assert np.all(np.abs(got - exact) <= 1e-6 * bound)


def test_int8_matmul_refuses_f32_path_types(oracle):
    # FISH never gives these types to its int8 kernels (quant.cpp:475-481)
    x = np.zeros((1, 256), np.float32)
    q32, q256 = oracle.act_batch(x)
    with pytest.raises(ValueError):
        oracle.matmul(Q4_1, np.zeros(20 * 8, np.uint8), q32, q256, 1, 256, 1)
