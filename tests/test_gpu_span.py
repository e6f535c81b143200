"""Layer spans through the C ABI against a NumPy restatement of FISH's layer.

The span (fish_hip_span_prepare / _forward) runs dense llama layers on the
device. The reference below restates FISH's CPU forward for one layer
(model.cpp:1650-1801) step by step: rmsnorm (ops.cpp:18-23), the projections
as FISH's matmul_batch on int8-quantized activations (the oracle's
matmul_f32), RoPE from the same tables (ops.cpp:126-152, neox pairs here;
the adjacent-pair form is covered by the whole-model test), the KV cache,
causal GQA attention in float64 (ops.cpp:303-357), SiLU·up and the residual
adds. Calls: a 37-token prefill (batch kernel), three decode tokens (fused
GEMVs; the span replays one captured HIP graph per token, with the position
in device memory), a 100-token prefill (GEMM), then one more decode token,
so later calls attend over the cache the earlier ones wrote and every graph
replay is checked.

Bar: the layer's update x_out - x_in within 5e-3 of its L-inf norm. The
device rounds rmsnorm and attention in another order than FISH, so an
activation sitting on an int8 rounding boundary can quantize one code apart;
a wrong RoPE pairing, head mapping, mask or cache position is off by O(1).
"""
import numpy as np
import pytest

import imurun_amd as fh
from imurun_amd.synth import normal

pytestmark = pytest.mark.gpu

E, H, HKV, D, F, CTX = 512, 4, 2, 128, 1024, 256
Q, KV = H * D, HKV * D
TYPES = dict(wq=fh.Q4_K, wk=fh.Q4_K, wv=fh.Q6_K, wo=fh.Q4_K, wg=fh.Q4_K, wu=fh.Q4_K, wd=fh.Q6_K)
SHAPES = dict(wq=(Q, E), wk=(KV, E), wv=(KV, E), wo=(E, Q), wg=(F, E), wu=(F, E), wd=(E, F))


def rope_tables(rot_dim):
    half = rot_dim // 2
    inv = 10000.0 ** (-np.arange(half, dtype=np.float64) * 2 / rot_dim)
    th = np.arange(CTX, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(th).astype(np.float32), np.sin(th).astype(np.float32)


class RefLayer:
    def __init__(self, oracle, packed, an, fn, cos, sin, neox=True):
        self.o, self.w, self.an, self.fn, self.cos, self.sin = oracle, packed, an, fn, cos, sin
        self.neox = neox
        self.kc = np.zeros((CTX, KV), np.float32)
        self.vc = np.zeros((CTX, KV), np.float32)

    def mm(self, name, x):
        return self.o.matmul_f32(TYPES[name], self.w[name], x, SHAPES[name][0])

    @staticmethod
    def rms(x, w):
        s = (x.astype(np.float64) ** 2).sum(axis=1) / x.shape[1]
        scale = (np.float32(1.0) / np.sqrt((s.astype(np.float32) + np.float32(1e-5)))).astype(np.float32)
        return (x * scale[:, None]) * w[None, :]

    def rope(self, v, pos, nh):
        half = self.cos.shape[1]
        c, s = self.cos[pos][:, None, :], self.sin[pos][:, None, :]
        v = v.reshape(v.shape[0], nh, D).copy()
        if self.neox:
            x0, x1 = v[:, :, :half].copy(), v[:, :, half:2 * half].copy()
            v[:, :, :half] = x0 * c - x1 * s
            v[:, :, half:2 * half] = x0 * s + x1 * c
        else:  # adjacent pairs: a planted convention mistake for the bar to reject
            x0, x1 = v[:, :, 0:2 * half:2].copy(), v[:, :, 1:2 * half:2].copy()
            v[:, :, 0:2 * half:2] = x0 * c - x1 * s
            v[:, :, 1:2 * half:2] = x0 * s + x1 * c
        return v.reshape(v.shape[0], nh * D)

    def forward(self, x, pos0):
        n = x.shape[0]
        pos = np.arange(pos0, pos0 + n)
        xb = self.rms(x, self.an)
        q, k, v = self.mm("wq", xb), self.mm("wk", xb), self.mm("wv", xb)
        q, k = self.rope(q, pos, H), self.rope(k, pos, HKV)
        self.kc[pos], self.vc[pos] = k, v
        att = np.zeros((n, Q), np.float64)
        for t in range(n):
            p = pos0 + t
            for h in range(H):
                kh = h // (H // HKV)
                kk = self.kc[:p + 1, kh * D:(kh + 1) * D].astype(np.float64)
                vv = self.vc[:p + 1, kh * D:(kh + 1) * D].astype(np.float64)
                sc = kk @ q[t, h * D:(h + 1) * D].astype(np.float64) / np.sqrt(D)
                e = np.exp(sc - sc.max())
                att[t, h * D:(h + 1) * D] = (e / e.sum()) @ vv
        x = x + self.mm("wo", att.astype(np.float32))
        xb = self.rms(x, self.fn)
        g, u = self.mm("wg", xb), self.mm("wu", xb)
        h = (g / (1.0 + np.exp(-g))) * u
        return x + self.mm("wd", h.astype(np.float32))


@pytest.mark.parametrize("rot_dim", [D, D // 2])
def test_span_layer_matches_fish_forward(oracle, rot_dim):
    be = fh.HipBackend()
    assert be.available()
    packed = {n: fh.quantize_rows(TYPES[n], normal(600 + i, SHAPES[n], 0.03)) for i, n in enumerate(TYPES)}
    for n in TYPES:
        assert be.upload(f"span.{n}", TYPES[n], packed[n], SHAPES[n][1], SHAPES[n][0])
    an = (1.0 + 0.1 * normal(640, (E,), 1.0)).astype(np.float32)
    fn = (1.0 + 0.1 * normal(641, (E,), 1.0)).astype(np.float32)
    cos, sin = rope_tables(rot_dim)
    names = [f"span.{n}" for n in TYPES]
    assert be.span_prepare([(names, an, fn)], E, H, HKV, D, F, CTX, cos, sin, rope_neox=True)
    ref = RefLayer(oracle, packed, an, fn, cos, sin)
    try:
        pos0 = 0
        for i, n in enumerate((37, 1, 1, 1, 100, 1)):
            x = normal(650 + i, (n, E), 1.0)
            want = ref.forward(x, pos0)
            got = x.copy()
            assert be.span_forward(got, pos0), fh.load().fish_hip_last_error()
            d_ref, d_dev = want - x, got - x
            err = np.abs(d_dev - d_ref).max()
            assert err <= 5e-3 * np.abs(d_ref).max(), (n, pos0, err, np.abs(d_ref).max())
            if i == 0:
                # the bar rejects the other RoPE pairing (a plausible mistake)
                wrong = RefLayer(oracle, packed, an, fn, cos, sin, neox=False).forward(x, pos0) - x
                assert np.abs(d_dev - wrong).max() > 5e-3 * np.abs(d_ref).max()
            pos0 += n
        # past the context: refused, x untouched
        x = normal(660, (CTX - pos0 + 1, E), 1.0)
        x0 = x.copy()
        assert not be.span_forward(x, pos0)
        assert np.array_equal(x, x0)
    finally:
        be.span_release()
        for n in names:
            be.release(n)


def test_span_refuses_missing_or_misshaped_weights():
    be = fh.HipBackend()
    an = np.ones(E, np.float32)
    cos, sin = rope_tables(D)
    names = [f"absent.{n}" for n in TYPES]
    assert not be.span_prepare([(names, an, an)], E, H, HKV, D, F, CTX, cos, sin)
    # head_dim beyond the attention kernel's 256
    assert not be.span_prepare([(names, an, an)], E, 1, 1, 512, F, CTX, cos, sin)
    x = normal(661, (1, E), 1.0)
    assert not be.span_forward(x, 0)
