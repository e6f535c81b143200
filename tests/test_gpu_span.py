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
Qwen-3 per-head q/k RMS norms before RoPE (model.cpp:1704-1719, :1749);
Phi-3 fused q|k|v with its fused bias and fused gate|up, gate rows first
(model.cpp:1665-1674, 1481-1490; the fused tensors are the separate ones'
rows concatenated, so the reference keeps them apart); Gemma-2 post norms of
the attention and FFN outputs (model.cpp:1758-1760, 1791-1793), attention
logits soft-capped c tanh(s / c) and a sliding window (ops.cpp:327-335), and
FISH's tanh GELU in the FFN (ops.cpp:32-38).

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
    def __init__(self, oracle, packed, an, fn, cos, sin, neox=True, extras=None, types=None, opts=None):
        self.o, self.w, self.an, self.fn, self.cos, self.sin = oracle, packed, an, fn, cos, sin
        self.neox = neox
        self.x = extras or {}
        self.types = types or TYPES
        self.opts = opts or {}
        self.kc = np.zeros((cos.shape[0], KV), np.float32)
        self.vc = np.zeros((cos.shape[0], KV), np.float32)

    def mm(self, name, x):
        return self.o.matmul_f32(self.types[name], self.w[name], x, SHAPES[name][0])

    def act(self, g, u):
        """silu(g) * u, or FISH's tanh GELU (ops.cpp:32-38) when the variant has it."""
        if self.opts.get("gelu"):
            g64 = g.astype(np.float64)
            return (0.5 * g64 * (1.0 + np.tanh(0.7978845608028654 * (g64 + 0.044715 * g64 ** 3)))) * u
        return (g / (1.0 + np.exp(-g.astype(np.float64)))) * u

    def attend(self, q_row, kk, vv, p):
        """One head of one token over cache rows 0..p (float64), with the variant's soft cap
        and sliding window (ops.cpp:327-350)."""
        lo = max(0, p - self.opts["window"] + 1) if self.opts.get("window") else 0
        sc = kk[lo:p + 1] @ q_row / np.sqrt(D)
        if self.opts.get("softcap"):
            c = self.opts["softcap"]
            sc = c * np.tanh(sc / c)
        e = np.exp(sc - sc.max())
        return (e / e.sum()) @ vv[lo:p + 1]

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
        # the cache holds f16 K and V (round to nearest even), or their int8 form
        if self.opts.get("kv_q8"):
            self.kc[pos], self.vc[pos] = q8_rows(k)[0], q8_rows(v)[0]
        else:
            self.kc[pos] = k.astype(np.float16).astype(np.float32)
            self.vc[pos] = v.astype(np.float16).astype(np.float32)
        att = np.zeros((n, Q), np.float64)
        for t in range(n):
            p = pos0 + t
            for h in range(H):
                kh = h // (H // HKV)
                kk = self.kc[:p + 1, kh * D:(kh + 1) * D].astype(np.float64)
                vv = self.vc[:p + 1, kh * D:(kh + 1) * D].astype(np.float64)
                att[t, h * D:(h + 1) * D] = self.attend(q[t, h * D:(h + 1) * D].astype(np.float64), kk, vv, p)
        proj = self.mm("wo", att.astype(np.float32))
        if "bias_o" in self.x:
            proj = proj + self.x["bias_o"]
        if "post_attn_norm" in self.x:
            proj = self.rms(proj, self.x["post_attn_norm"])
        x = x + proj
        xb = self.rms(x, self.fn)
        g, u = self.mm("wg", xb), self.mm("wu", xb)
        dn = self.mm("wd", self.act(g, u).astype(np.float32))
        if "post_ffn_norm" in self.x:
            dn = self.rms(dn, self.x["post_ffn_norm"])
        return x + dn


# per variant: weight types (a fused tensor has one type), span options
VARIANT_TYPES = {"phi3": dict(TYPES, wv=fh.Q4_K)}
VARIANT_OPTS = {"gemma2": dict(softcap=5.0, window=24, gelu=True), "gelu": dict(gelu=True), "q8kv": dict(kv_q8=True)}


def q8_rows(x):
    """The int8 KV cache's value of each element (SpanParams::kv_q8, backend.h:152-156): per
    32 values d = amax / 127 (f32 division), codes clamp(rint(x * (1 / d)), -127, 127) with
    one f32 rounding of the product, value = code * d; and the d of each element's block."""
    x = np.ascontiguousarray(x, np.float32)
    b = x.reshape(x.shape[0], -1, 32)
    amax = np.abs(b).max(axis=2, keepdims=True)
    d = (amax / np.float32(127)).astype(np.float32)
    inv = np.where(d > 0, np.float32(1) / np.where(d > 0, d, np.float32(1)), np.float32(0)).astype(np.float32)
    q = np.clip(np.rint((b * inv).astype(np.float32)), -127, 127).astype(np.float32)
    return (q * d).reshape(x.shape).astype(np.float32), np.broadcast_to(d, b.shape).reshape(x.shape)


def layer_extras(variant):
    """The optional per-layer vectors of a variant (backend.h:129-134)."""
    if variant == "phi3":
        return {"bias_q": normal(676, (Q,), 0.5), "bias_k": normal(677, (KV,), 0.5),
                "bias_v": normal(678, (KV,), 0.5)}
    if variant == "gemma2":
        return {"post_attn_norm": (1.0 + 0.2 * normal(679, (E,), 1.0)).astype(np.float32),
                "post_ffn_norm": (1.0 + 0.2 * normal(680, (E,), 1.0)).astype(np.float32)}
    if variant == "qwen3":
        return {"q_norm": (1.0 + 0.2 * normal(670, (D,), 1.0)).astype(np.float32),
                "k_norm": (1.0 + 0.2 * normal(671, (D,), 1.0)).astype(np.float32)}
    if variant == "bias":
        return {"bias_q": normal(672, (Q,), 0.5), "bias_k": normal(673, (KV,), 0.5),
                "bias_v": normal(674, (KV,), 0.5), "bias_o": normal(675, (E,), 0.5)}
    return {}


def setup_span(oracle, be, rot_dim, variant, tag, ctx=CTX):
    types = VARIANT_TYPES.get(variant, TYPES)
    opts = VARIANT_OPTS.get(variant, {})
    packed = {n: fh.quantize_rows(types[n], normal(600 + i, SHAPES[n], 0.03)) for i, n in enumerate(types)}
    for n in types:
        assert be.upload(f"{tag}.{n}", types[n], packed[n], SHAPES[n][1], SHAPES[n][0])
    an = (1.0 + 0.1 * normal(640, (E,), 1.0)).astype(np.float32)
    fn = (1.0 + 0.1 * normal(641, (E,), 1.0)).astype(np.float32)
    cos, sin = rope_tables(rot_dim, ctx)
    names = [f"{tag}.{n}" for n in types]
    uploaded = list(names)
    extras = layer_extras(variant)
    span_extras = dict(extras)
    if variant == "phi3":
        # the fused tensors: rows of q, k, v (and of gate, up) concatenated, one bias for q|k|v
        fq = np.concatenate([packed["wq"], packed["wk"], packed["wv"]])
        fgu = np.concatenate([packed["wg"], packed["wu"]])
        assert be.upload(f"{tag}.wqkv", fh.Q4_K, fq, E, Q + 2 * KV)
        assert be.upload(f"{tag}.wgu", fh.Q4_K, fgu, E, 2 * F)
        uploaded += [f"{tag}.wqkv", f"{tag}.wgu"]
        span_extras = {"wqkv": f"{tag}.wqkv",
                       "bias_qkv": np.concatenate([extras["bias_q"], extras["bias_k"], extras["bias_v"]])}
        names_span = [None, None, None, names[3], None, f"{tag}.wgu", names[6]]
    else:
        names_span = names
    if opts.get("window"):
        span_extras["sliding_window"] = True
    assert be.span_prepare([(names_span, an, fn, span_extras)], E, H, HKV, D, F, ctx, cos, sin, rope_neox=True,
                           attn_softcap=opts.get("softcap", 0.0), window=opts.get("window", 0),
                           gelu=opts.get("gelu", False), kv_q8=opts.get("kv_q8", False))
    ref = RefLayer(oracle, packed, an, fn, cos, sin, extras=extras, types=types, opts=opts)
    return uploaded, ref, (packed, an, fn, cos, sin, extras)


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
        if ref.opts.get("kv_q8"):
            # int8 rows: within one code step of the form of the reference's values (the
            # device's own k and v differ from them in the last bits)
            val, dstep = q8_rows(want)
            assert np.all(np.abs(got - val) <= 1.01 * dstep + 1e-30), f"{what}: {nm} int8 cache rows"
            assert np.all(np.abs(got / np.where(dstep > 0, dstep, 1) - np.rint(got / np.where(dstep > 0, dstep, 1)))
                          < 1e-3), f"{what}: {nm} cache rows are codes x d"
            continue
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
            a_want[t, hh * D:(hh + 1) * D] = ref.attend(qr[t, hh * D:(hh + 1) * D].astype(np.float64), kk, vv, p)
    close(att, a_want, 1e-5, f"{what}: attention")
    if "post_attn_norm" in X:
        # proj holds rmsnorm(o + bias_o) * post_attn_norm
        p_want = ref.mm("wo", att) + (X["bias_o"] if "bias_o" in X else 0.0)
        close(proj, ref.rms(p_want.astype(np.float32), X["post_attn_norm"]), 1e-4, f"{what}: o projection, post norm")
        x1 = x_in + proj
    else:
        close(proj, ref.mm("wo", att), 1e-4, f"{what}: o projection")
        x1 = x_in + (proj + X["bias_o"] if "bias_o" in X else proj)
    close(xb2, ref.rms(x1, ref.fn), 1e-6, f"{what}: FFN norm")
    close(u, ref.mm("wu", xb2), 1e-4, f"{what}: up")
    g = ref.mm("wg", xb2)
    close(h, ref.act(g, u), 1e-4, f"{what}: act(gate) * up")
    d_want = ref.mm("wd", h)
    if "post_ffn_norm" in X:
        d_want = ref.rms(d_want, X["post_ffn_norm"])
    close(dn, d_want, 1e-4, f"{what}: down")
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


@pytest.mark.parametrize("rot_dim,variant", [(D, "llama"), (D // 2, "llama"), (D, "qwen3"), (D, "bias"),
                                             (D, "phi3"), (D, "gemma2"), (D, "gelu"), (D, "q8kv")])
def test_span_layer_matches_fish_forward(oracle, rot_dim, variant):
    be = fh.HipBackend()
    assert be.available()
    names, ref, (packed, an, fn, cos, sin, extras) = setup_span(oracle, be, rot_dim, variant, "span")
    try:
        pos0 = 0
        for i, n in enumerate((37, 1, 1, 3, 100, 1)):
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
                if "bias_q" in extras or "q_norm" in extras:
                    plain = ref.prep(q, None, None, pos, H)
                    assert np.abs(qr - plain).max() > 1e-2 * np.abs(qr).max()
            if i == 4 and ref.opts:
                # the bars reject attention without the soft cap or without the window, and SiLU
                # for GELU: each is far outside the 1e-5 / 1e-4 stage bars on this call
                att, qr = be.span_inspect("att", Q), be.span_inspect("qr", Q)
                kc = be.span_inspect("kc", KV, 0, 0, pos0 + n)
                vc = be.span_inspect("vc", KV, 0, 0, pos0 + n)
                for drop in [k for k in ("softcap", "window") if k in ref.opts]:
                    alt = RefLayer(oracle, packed, an, fn, cos, sin, extras=extras, types=ref.types,
                                   opts={k: v for k, v in ref.opts.items() if k != drop})
                    t, p = n - 1, pos0 + n - 1
                    a_alt = alt.attend(qr[t, :D].astype(np.float64), kc[:, :D].astype(np.float64),
                                       vc[:, :D].astype(np.float64), p)
                    assert np.abs(att[t, :D] - a_alt).max() > 1e-3 * np.abs(a_alt).max(), drop
                if ref.opts.get("gelu"):
                    g, u = be.span_inspect("h", F), be.span_inspect("u", F)
                    silu = RefLayer(oracle, packed, an, fn, cos, sin, extras=extras, types=ref.types, opts={})
                    xb2 = be.span_inspect("xb2", E)
                    gg = ref.mm("wg", xb2)
                    assert np.abs(silu.act(gg, u) - ref.act(gg, u)).max() > 1e-2 * np.abs(ref.act(gg, u)).max()
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


@pytest.mark.parametrize("e_dim,variant", [(2048, "gelu"), (4096, "llama")])
def test_span_decode_at_model_width(oracle, monkeypatch, e_dim, variant):
    """One-token calls at model widths: the gate/up launch then runs 64 lanes per row (one
    and two groups per lane) with the activation in its epilogue, SiLU and GELU; every stage
    is checked as above."""
    import sys
    mod = sys.modules[__name__]
    monkeypatch.setattr(mod, "E", e_dim)
    monkeypatch.setattr(mod, "SHAPES", dict(wq=(Q, e_dim), wk=(KV, e_dim), wv=(KV, e_dim), wo=(e_dim, Q),
                                            wg=(F, e_dim), wu=(F, e_dim), wd=(e_dim, F)))
    be = fh.HipBackend()
    assert be.available()
    names, ref, _ = setup_span(oracle, be, D, variant, f"wide{e_dim}")
    try:
        pos0 = 0
        for i, n in enumerate((5, 1, 1, 1)):
            x = normal(690 + i, (n, e_dim), 1.0)
            check_call(be, ref, x, pos0, f"{variant} E={e_dim}")
            pos0 += n
    finally:
        be.span_release()
        for n in names:
            be.release(n)


@pytest.mark.parametrize("variant", ["llama", "gemma2"])
def test_span_head_dim_256(oracle, monkeypatch, variant):
    """Head dim 256 (Gemma-2's): the prefill attention on f16 MFMA tiles of 256 values (no
    row prefetch), then one-token calls through the position chunks; every stage is checked
    as above, Gemma-2's soft cap and window included."""
    import sys
    mod = sys.modules[__name__]
    h, hkv, d = 2, 1, 256
    for name, val in (("H", h), ("HKV", hkv), ("D", d), ("Q", h * d), ("KV", hkv * d)):
        monkeypatch.setattr(mod, name, val)
    monkeypatch.setattr(mod, "SHAPES", dict(wq=(h * d, E), wk=(hkv * d, E), wv=(hkv * d, E), wo=(E, h * d),
                                            wg=(F, E), wu=(F, E), wd=(E, F)))
    be = fh.HipBackend()
    assert be.available()
    names, ref, _ = setup_span(oracle, be, d, variant, f"d256{variant}")
    try:
        pos0 = 0
        for i, n in enumerate((37, 100, 1, 1)):
            x = normal(720 + i, (n, E), 1.0)
            check_call(be, ref, x, pos0, f"{variant} D=256")
            pos0 += n
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


@pytest.mark.parametrize("variant", ["llama", "gemma2"])
def test_span_decode_at_long_positions(oracle, variant):
    """One-token calls with 6 and then 16-17 chunks of 64 positions behind the token, after
    prefills of more than one 256-token chunk: the combine then also reads chunks past the
    16 whose outputs it loads up front. Gemma-2's soft cap and 24-position window ride along;
    every stage is checked as above."""
    be = fh.HipBackend()
    names, ref, _ = setup_span(oracle, be, D, variant, f"long{variant}", ctx=1100)
    try:
        check_call(be, ref, normal(701, (383, E), 1.0), 0, "prefill to 383")
        for p in (383, 384, 385):
            check_call(be, ref, normal(702 + p, (1, E), 1.0), p, f"decode at {p}")
        check_call(be, ref, normal(703, (637, E), 1.0), 386, "prefill to 1023")
        for p in (1023, 1024, 1025):
            check_call(be, ref, normal(704 + p, (1, E), 1.0), p, f"decode at {p}")
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


def test_span_int8_kv_cache_needs_whole_blocks(oracle):
    """kv_q8 (backend.h:152-156) gives an int8 cache when kv_dim and head_dim are multiples of
    32 (FISH's planner sets it only then, model.cpp:1023); otherwise span_prepare refuses."""
    be = fh.HipBackend()
    packed = {n: fh.quantize_rows(TYPES[n], normal(600 + i, SHAPES[n], 0.03)) for i, n in enumerate(TYPES)}
    names = [f"kvq8.{n}" for n in TYPES]
    for n, name in zip(TYPES, names):
        assert be.upload(name, TYPES[n], packed[n], SHAPES[n][1], SHAPES[n][0])
    an = np.ones(E, np.float32)
    cos, sin = rope_tables(D)
    try:
        assert be.span_prepare([(names, an, an)], E, H, HKV, D, F, CTX, cos, sin, kv_q8=True)
        be.span_release()
        # head_dim 136 (not whole 32-value blocks) with q / o shaped to match: refused with kv_q8 only
        d2 = 136
        shp = dict(SHAPES, wq=(H * d2, E), wk=(HKV * d2, E), wv=(HKV * d2, E), wo=(E, H * d2))
        t2 = dict(TYPES, wo=fh.Q8_0)  # o's rows of 4 x 136 values: 32-value blocks
        p2 = {n: fh.quantize_rows(t2[n], normal(610 + i, shp[n], 0.03)) for i, n in enumerate(t2)}
        n2 = [f"kvq8b.{n}" for n in t2]
        for n, name in zip(t2, n2):
            assert be.upload(name, t2[n], p2[n], shp[n][1], shp[n][0])
        names += n2
        c2, s2 = rope_tables(d2)
        assert not be.span_prepare([(n2, an, an)], E, H, HKV, d2, F, CTX, c2, s2, kv_q8=True)
        assert be.span_prepare([(n2, an, an)], E, H, HKV, d2, F, CTX, c2, s2)
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


def test_span_refuses_inconsistent_fused_forms():
    """A fused q|k|v with separate q/k/v keys or separate biases, a fused bias without the fused
    tensor, a fused gate|up of the wrong height, and a sliding-window layer without a window
    size are refused (the descriptor contract of include/fish_hip.h)."""
    be = fh.HipBackend()
    types = VARIANT_TYPES["phi3"]
    packed = {n: fh.quantize_rows(types[n], normal(600 + i, SHAPES[n], 0.03)) for i, n in enumerate(types)}
    names = [f"fz.{n}" for n in types]
    for n, name in zip(types, names):
        assert be.upload(name, types[n], packed[n], SHAPES[n][1], SHAPES[n][0])
    assert be.upload("fz.wqkv", fh.Q4_K, np.concatenate([packed["wq"], packed["wk"], packed["wv"]]), E, Q + 2 * KV)
    assert be.upload("fz.wgu", fh.Q4_K, np.concatenate([packed["wg"], packed["wu"]]), E, 2 * F)
    an = np.ones(E, np.float32)
    cos, sin = rope_tables(D)
    fused = [None, None, None, names[3], None, "fz.wgu", names[6]]
    bqkv = np.zeros(Q + 2 * KV, np.float32)
    try:
        ok = be.span_prepare([(fused, an, an, {"wqkv": "fz.wqkv", "bias_qkv": bqkv})], E, H, HKV, D, F, CTX, cos,
                             sin)
        assert ok
        bad = [
            [(names, an, an, {"wqkv": "fz.wqkv"})],                                   # fused and separate
            [(fused, an, an, {"wqkv": "fz.wqkv", "bias_q": np.zeros(Q, np.float32)})],  # separate bias
            [(names, an, an, {"bias_qkv": bqkv})],                                    # fused bias alone
            [(names[:4] + [None, names[5], names[6]], an, an)],                      # gate|up of F rows
        ]
        for layers in bad:
            assert not be.span_prepare(layers, E, H, HKV, D, F, CTX, cos, sin)
        assert not be.span_prepare([(names, an, an, {"sliding_window": True})], E, H, HKV, D, F, CTX, cos, sin)
        assert be.span_prepare([(names, an, an, {"sliding_window": True})], E, H, HKV, D, F, CTX, cos, sin,
                               window=8)
    finally:
        be.span_release()
        for n in names + ["fz.wqkv", "fz.wgu"]:
            be.release(n)
