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
replay is checked. The KV cache holds f16 K and V, as FISH's own device span
does (vulkan_backend.cpp:1650); the reference stores them rounded to f16 the
same way. Layer variants: llama; Qwen-2 projection biases (q/k/v, and o);
Qwen-3 per-head q/k RMS norms before RoPE (model.cpp:1704-1719, :1749).

Bars, per call, on the device's own intermediate values of that call
(fish_hip_span_inspect), each stage against the reference applied to the
device's input of that stage: the RMS norms within 1e-6 of their largest
value; q / k / v, o, gate / up and down projections within 1e-4 of theirs
(FISH's int8 matmul on the same f32 input); q after bias / q-norm / RoPE and
the f16 cache rows of k and v within f32 rounding (cache rows: one f16 ulp);
attention (float64 softmax over the device's q and cache rows) within 1e-5;
silu * up within 1e-4; and the residual stream leaving the layer exactly
x + (o + bias_o) + down, in f32. End to end, the layer's update is also
compared with the reference layer run on its own (report, and a 2e-2 sanity
bar): the int8 requantization of the attention output and of the FFN hidden
state is discontinuous, so an f32 rounding difference can flip a code, which
moves the update by up to ~2e-3 of its L-inf norm here per flip; a wrong RoPE
pairing, head mapping, mask, cache position, bias or norm is off by O(1) and
fails the stage bars.
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


def rope_tables(rot_dim, ctx=CTX):
    half = rot_dim // 2
    inv = 10000.0 ** (-np.arange(half, dtype=np.float64) * 2 / rot_dim)
    th = np.arange(ctx, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(th).astype(np.float32), np.sin(th).astype(np.float32)


class RefLayer:
    def __init__(self, oracle, packed, an, fn, cos, sin, neox=True, extras=None):
        self.o, self.w, self.an, self.fn, self.cos, self.sin = oracle, packed, an, fn, cos, sin
        self.neox = neox
        self.x = extras or {}
        self.kc = np.zeros((cos.shape[0], KV), np.float32)
        self.vc = np.zeros((cos.shape[0], KV), np.float32)

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

    def head_rms(self, v, w, nh):
        """FISH's rmsnorm applied to each head of D values (model.cpp:1712-1719)."""
        return self.rms(v.reshape(-1, D), w).reshape(v.shape[0], nh * D)

    def prep(self, v, bias, norm_w, pos, nh):
        """Projection output -> + bias -> per-head RMS norm -> RoPE (model.cpp:1704-1724)."""
        if bias is not None:
            v = v + bias
        if norm_w is not None:
            v = self.head_rms(v, norm_w, nh)
        return self.rope(v, pos, nh)

    def forward(self, x, pos0):
        n = x.shape[0]
        pos = np.arange(pos0, pos0 + n)
        xb = self.rms(x, self.an)
        q, k, v = self.mm("wq", xb), self.mm("wk", xb), self.mm("wv", xb)
        if "bias_q" in self.x:
            q, k, v = q + self.x["bias_q"], k + self.x["bias_k"], v + self.x["bias_v"]
        if "q_norm" in self.x:
            q, k = self.head_rms(q, self.x["q_norm"], H), self.head_rms(k, self.x["k_norm"], HKV)
        q, k = self.rope(q, pos, H), self.rope(k, pos, HKV)
        # the cache holds f16 K and V (round to nearest even)
        self.kc[pos] = k.astype(np.float16).astype(np.float32)
        self.vc[pos] = v.astype(np.float16).astype(np.float32)
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
        proj = self.mm("wo", att.astype(np.float32))
        if "bias_o" in self.x:
            proj = proj + self.x["bias_o"]
        x = x + proj
        xb = self.rms(x, self.fn)
        g, u = self.mm("wg", xb), self.mm("wu", xb)
        h = (g / (1.0 + np.exp(-g))) * u
        return x + self.mm("wd", h.astype(np.float32))


def layer_extras(variant):
    """The optional per-layer vectors of a variant (backend.h:129-134)."""
    if variant == "qwen3":
        return {"q_norm": (1.0 + 0.2 * normal(670, (D,), 1.0)).astype(np.float32),
                "k_norm": (1.0 + 0.2 * normal(671, (D,), 1.0)).astype(np.float32)}
    if variant == "bias":
        return {"bias_q": normal(672, (Q,), 0.5), "bias_k": normal(673, (KV,), 0.5),
                "bias_v": normal(674, (KV,), 0.5), "bias_o": normal(675, (E,), 0.5)}
    return {}


def setup_span(oracle, be, rot_dim, variant, tag, ctx=CTX):
    packed = {n: fh.quantize_rows(TYPES[n], normal(600 + i, SHAPES[n], 0.03)) for i, n in enumerate(TYPES)}
    for n in TYPES:
        assert be.upload(f"{tag}.{n}", TYPES[n], packed[n], SHAPES[n][1], SHAPES[n][0])
    an = (1.0 + 0.1 * normal(640, (E,), 1.0)).astype(np.float32)
    fn = (1.0 + 0.1 * normal(641, (E,), 1.0)).astype(np.float32)
    cos, sin = rope_tables(rot_dim, ctx)
    names = [f"{tag}.{n}" for n in TYPES]
    extras = layer_extras(variant)
    assert be.span_prepare([(names, an, fn, extras)], E, H, HKV, D, F, ctx, cos, sin, rope_neox=True)
    return names, RefLayer(oracle, packed, an, fn, cos, sin, extras=extras), (packed, an, fn, cos, sin, extras)


def close(got, want, tol, what):
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    scale = float(np.max(np.abs(want)))
    assert err <= tol * scale, f"{what}: max err {err:.3e} vs {tol} * {scale:.3e}"


def check_stages(be, ref, x_in, x_out, pos0, what):
    """Every stage of the call that just ran, on the device's own stage inputs."""
    n = x_in.shape[0]
    X = ref.x
    sp = lambda part, w: be.span_inspect(part, w)  # noqa: E731
    xb, q, k, v, qr = sp("xb", E), sp("q", Q), sp("k", KV), sp("v", KV), sp("qr", Q)
    att, proj, xb2, h, u, dn = sp("att", Q), sp("proj", E), sp("xb2", E), sp("h", F), sp("u", F), sp("dn", E)
    assert xb.shape[0] == n, (what, xb.shape, n)
    pos = np.arange(pos0, pos0 + n)
    close(xb, ref.rms(x_in, ref.an), 1e-6, f"{what}: attention norm")
    for name, y in (("wq", q), ("wk", k), ("wv", v)):
        close(y, ref.mm(name, xb), 1e-4, f"{what}: {name}")
    # bias, q/k norm, RoPE; the cache rows hold f16(k'), f16(v + bias)
    q_want = ref.prep(q, X.get("bias_q"), X.get("q_norm"), pos, H)
    close(qr, q_want, 1e-5, f"{what}: q after bias / norm / RoPE")
    k_want = ref.prep(k, X.get("bias_k"), X.get("k_norm"), pos, HKV)
    v_want = v + X["bias_v"] if "bias_v" in X else v
    kc = be.span_inspect("kc", KV, 0, 0, pos0 + n)
    vc = be.span_inspect("vc", KV, 0, 0, pos0 + n)
    for got, want, nm in ((kc[pos0:], k_want, "k"), (vc[pos0:], v_want, "v")):
        ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
        assert np.all(np.abs(got - want.astype(np.float16).astype(np.float64)) <= ulp), f"{what}: {nm} cache rows"
    # attention over the device's q and cache rows, in float64
    a_want = np.zeros((n, Q))
    for t in range(n):
        p = pos0 + t
        for hh in range(H):
            kh = hh // (H // HKV)
            kk = kc[:p + 1, kh * D:(kh + 1) * D].astype(np.float64)
            vv = vc[:p + 1, kh * D:(kh + 1) * D].astype(np.float64)
            sc = kk @ qr[t, hh * D:(hh + 1) * D].astype(np.float64) / np.sqrt(D)
            e = np.exp(sc - sc.max())
            a_want[t, hh * D:(hh + 1) * D] = (e / e.sum()) @ vv
    close(att, a_want, 1e-5, f"{what}: attention")
    close(proj, ref.mm("wo", att), 1e-4, f"{what}: o projection")
    x1 = x_in + (proj + X["bias_o"] if "bias_o" in X else proj)
    close(xb2, ref.rms(x1, ref.fn), 1e-6, f"{what}: FFN norm")
    close(u, ref.mm("wu", xb2), 1e-4, f"{what}: up")
    g = ref.mm("wg", xb2)
    close(h, (g / (1.0 + np.exp(-g.astype(np.float64)))) * u, 1e-4, f"{what}: silu(gate) * up")
    close(dn, ref.mm("wd", h), 1e-4, f"{what}: down")
    assert np.array_equal(x_out, x1 + dn), f"{what}: residual stream"


def check_call(be, ref, x, pos0, what):
    want = ref.forward(x, pos0)
    got = x.copy()
    assert be.span_forward(got, pos0), fh.load().fish_hip_last_error()
    last = be.L.fish_hip_span_last_tokens()
    check_stages(be, ref, x[-last:], got[-last:], pos0 + x.shape[0] - last, what)
    d_ref, d_dev = want - x, got - x
    err = np.abs(d_dev - d_ref).max()
    print(f"span {what} n={x.shape[0]} pos0={pos0}: end-to-end update err {err:.3e} = "
          f"{err / np.abs(d_ref).max():.2e} of max|update|")
    assert err <= 2e-2 * np.abs(d_ref).max(), (what, x.shape[0], pos0, err, np.abs(d_ref).max())
    return d_dev, d_ref


@pytest.mark.parametrize("rot_dim,variant", [(D, "llama"), (D // 2, "llama"), (D, "qwen3"), (D, "bias")])
def test_span_layer_matches_fish_forward(oracle, rot_dim, variant):
    be = fh.HipBackend()
    assert be.available()
    names, ref, (packed, an, fn, cos, sin, extras) = setup_span(oracle, be, rot_dim, variant, "span")
    try:
        pos0 = 0
        for i, n in enumerate((37, 1, 1, 1, 100, 1)):
            x = normal(650 + i, (n, E), 1.0)
            d_dev, d_ref = check_call(be, ref, x, pos0, variant)
            if i == 0:
                # the stage bar rejects the other RoPE pairing (a plausible mistake), and a
                # variant's vectors left out
                q, qr = be.span_inspect("q", Q), be.span_inspect("qr", Q)
                pos = np.arange(pos0, pos0 + n)
                wrong = RefLayer(oracle, packed, an, fn, cos, sin, neox=False, extras=extras)
                bad = wrong.prep(q, extras.get("bias_q"), extras.get("q_norm"), pos, H)
                assert np.abs(qr - bad).max() > 1e-2 * np.abs(qr).max()
                if extras:
                    plain = ref.prep(q, None, None, pos, H)
                    assert np.abs(qr - plain).max() > 1e-2 * np.abs(qr).max()
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


def test_span_kv_rewind_then_new_tokens(oracle):
    """span_kv_truncate(n) then new tokens from position n (prefix reuse, backend.h:158): the
    rewritten positions replace the old ones for every later call; rows past n are never
    read before they are rewritten."""
    be = fh.HipBackend()
    names, ref, _ = setup_span(oracle, be, D, "llama", "rewind")
    try:
        check_call(be, ref, normal(680, (37, E), 1.0), 0, "prefill")
        for i in range(3):
            check_call(be, ref, normal(681 + i, (1, E), 1.0), 37 + i, "decode")
        be.span_kv_truncate(30)  # drop positions 30..39
        check_call(be, ref, normal(690, (5, E), 1.0), 30, "new prefill at 30")
        for i in range(3):
            check_call(be, ref, normal(691 + i, (1, E), 1.0), 35 + i, "new decode")
        be.span_kv_truncate(0)  # reset_kv()
        check_call(be, ref, normal(695, (1, E), 1.0), 0, "first token after reset")
        check_call(be, ref, normal(696, (1, E), 1.0), 1, "second token after reset")
    finally:
        be.span_release()
        for n in names:
            be.release(n)


def test_span_prefill_longer_than_one_chunk(oracle):
    """A batch of 300 tokens (more than FISH's 256-token forward batch) runs as two chunks, the
    second attending over the cache rows the first wrote."""
    be = fh.HipBackend()
    names, ref, _ = setup_span(oracle, be, D, "qwen3", "chunks", ctx=320)
    try:
        check_call(be, ref, normal(697, (300, E), 1.0), 0, "300-token prefill")
        check_call(be, ref, normal(698, (3, E), 1.0), 300, "3 more")
        check_call(be, ref, normal(699, (1, E), 1.0), 303, "decode")
    finally:
        be.span_release()
        for n in names:
            be.release(n)


def test_span_refuses_int8_kv_cache(oracle):
    """kv_q8 (backend.h:150-153) is refused: this backend keeps f16 K and V only."""
    be = fh.HipBackend()
    packed = {n: fh.quantize_rows(TYPES[n], normal(600 + i, SHAPES[n], 0.03)) for i, n in enumerate(TYPES)}
    names = [f"kvq8.{n}" for n in TYPES]
    for n, name in zip(TYPES, names):
        assert be.upload(name, TYPES[n], packed[n], SHAPES[n][1], SHAPES[n][0])
    an = np.ones(E, np.float32)
    cos, sin = rope_tables(D)
    try:
        assert not be.span_prepare([(names, an, an)], E, H, HKV, D, F, CTX, cos, sin, kv_q8=True)
        assert be.span_prepare([(names, an, an)], E, H, HKV, D, F, CTX, cos, sin)
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
