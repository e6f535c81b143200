"""Expert-routed FFN on the GPU (fish_hip_moe_*) against the oracle and the golden layer.

Every stage of a layer is checked on the GPU's own inputs to that stage:
routing (experts exact, weights within 1e-6), slot grouping (by expert,
tokens ascending), the gate and up products within 1e-4 * max|ref|, the
silu*up requantization bit-exact on the GPU's own f32 hidden values, the
down product within 1e-4 * max|ref| on those codes, and the combine
bit-exact (ascending expert order, separately rounded multiply and add).

The end-to-end comparison with FISH's composed layer (model.cpp:1523-1599)
is held to 1e-4 * max|out| plus a bound computed from the data: the hidden
state is requantized to int8 between the products, so an f32 rounding
difference in gate/up can move a hidden value across a rounding midpoint of
its code (or move its block's scale). The test requantizes FISH's own hidden
values (oracle gate/up on the same x, FISH's silu * up) and the GPU's, and
for each slot takes delta_k = |d' q'_k - d q_k|, the difference of the two
dequantized hidden values: nonzero where a code flipped or where the block's
scale differs (its absmax differs in the last bit). A down row i then moves by at most
sum_k delta_k |W_down[i][k]| <= sum_k delta_k colmax_k, colmax_k = max_i
|W_down[i][k]|; the combine weights it by the slot's routing weight. The
test prints the flipped codes, the observed error and the bound.
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


def dev(torch_dev, a, dtype=None):
    torch, d = torch_dev
    return torch.from_numpy(np.ascontiguousarray(a)).to(d)


def check_close(got, want, what, tol=TOL):
    err = float(np.max(np.abs(got - want)))
    scale = float(np.max(np.abs(want)))
    assert err <= tol * scale, f"{what}: max err {err:.3e} vs {tol} * {scale:.3e}"


@pytest.mark.parametrize("n_tok,n_expert,k", [(1, 8, 2), (64, 8, 2), (256, 128, 8), (7, 16, 4)])
def test_routing_matches_oracle(torch_dev, oracle, n_tok, n_expert, k):
    logits = normal(40 + n_tok + n_expert, (n_tok, n_expert))
    sel, wsel = fh.moe_route(dev(torch_dev, logits), k, True)
    want_sel, want_w = oracle.route(logits, k, True)
    assert np.array_equal(sel.cpu().numpy(), want_sel)
    assert np.allclose(wsel.cpu().numpy(), want_w, rtol=0, atol=1e-6)
    sel2, wsel2 = fh.moe_route(dev(torch_dev, logits), k, False)
    _, want_w2 = oracle.route(logits, k, False)
    assert np.array_equal(sel2.cpu().numpy(), want_sel)
    assert np.allclose(wsel2.cpu().numpy(), want_w2, rtol=0, atol=1e-6)


def _router_check(torch_dev, oracle, t, w, x):
    """GPU router logits against the oracle, per element within 1e-6 * sum|x w|
    (both sum in f32, in different orders), then the same top-k selection."""
    torch, _ = torch_dev
    wt = dev(torch_dev, w) if t == 0 else dev(torch_dev, w).view(torch.float16)
    got = fh.router_logits(dev(torch_dev, x), wt).cpu().numpy()
    want = oracle.router_logits(t, w, x)
    wf = w if t == 0 else w.view(np.float16)
    bound = np.abs(x.astype(np.float64)) @ np.abs(wf.astype(np.float64)).T
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= 1e-6 * bound), f"max err / bound {float(np.max(err / bound)):.3e}"
    return got, want


# tile shapes: one (token, expert) per wavefront below 1024 wavefronts' worth, then 2x4, then 8x8
# (100x128, 257x60 and 256x128 take 2x4; 1030x61 and 1100x67 take 8x8, ragged on both axes)
@pytest.mark.parametrize("t", [0, 1])
@pytest.mark.parametrize("n_tok,n_embd,n_expert", [(1, 4096, 8), (64, 4096, 8), (1, 2048, 128), (256, 2048, 128),
                                                   (5, 992, 8), (3, 260, 60), (33, 4, 3), (100, 1024, 128),
                                                   (257, 264, 60), (1030, 256, 61), (1100, 96, 67)])
def test_router_logits_match_oracle(torch_dev, oracle, t, n_tok, n_embd, n_expert):
    x = normal(50 + n_tok + n_embd, (n_tok, n_embd), 1.0)
    w = normal(60 + n_expert + n_embd, (n_expert, n_embd), 0.05)
    if t == 1:
        w = w.astype(np.float16).view(np.uint16)
    got, _ = _router_check(torch_dev, oracle, t, w, x)
    # every tile shape sums each (token, expert) in the same order: a token's logits are the
    # same bits whether it is routed alone or with the others
    torch, _ = torch_dev
    wt = dev(torch_dev, w) if t == 0 else dev(torch_dev, w).view(torch.float16)
    for r in sorted({0, n_tok // 2, n_tok - 1}):
        alone = fh.router_logits(dev(torch_dev, x[r:r + 1]), wt).cpu().numpy()
        assert np.array_equal(alone[0], got[r]), f"token {r}"
    # the device logits drive the device routing exactly as the oracle's routing
    k = min(2 if n_expert <= 8 else 8, n_expert)
    sel, _ = fh.moe_route(dev(torch_dev, got), k, True)
    assert np.array_equal(sel.cpu().numpy(), oracle.route(got, k, True)[0])


def test_router_logits_golden(torch_dev, oracle, golden):
    g = golden("router")
    for n in (256, 992):
        for t in (0, 1):
            for m in (1, 5):
                x = g[f"x_{n}_{m}"]
                got, _ = _router_check(torch_dev, oracle, t, g[f"w{t}_{n}"], x)
                wf = g[f"w{t}_{n}"] if t == 0 else g[f"w{t}_{n}"].view(np.float16)
                bound = np.abs(x.astype(np.float64)) @ np.abs(wf.astype(np.float64)).T
                assert np.all(np.abs(got - g[f"y{t}_{n}_{m}"]) <= 1e-6 * bound)


@pytest.mark.parametrize("n_rows,n_ff", [(20, 768), (3, 14336), (64, 256)])
def test_silu_mul_quantize_bit_exact_on_own_values(torch_dev, oracle, n_rows, n_ff):
    g = normal(51 + n_ff, (n_rows, n_ff)) * np.float32(2.0)
    u = normal(52 + n_ff, (n_rows, n_ff))
    _, q256, h = fh.silu_mul_quantize(dev(torch_dev, g), dev(torch_dev, u))
    h = h.cpu().numpy()
    # the values quantized are silu(g) * u to within float rounding of exp
    want = (g / (np.float32(1.0) + np.exp(-g.astype(np.float64)).astype(np.float32))) * u
    assert np.max(np.abs(h - want) / (np.abs(want) + 1e-30)) < 1e-5
    # and their int8 codes / scales / sums are exactly FISH's for those values
    assert np.array_equal(q256.cpu().numpy(), oracle.quantize_acts_k(h))


def repacked_experts(torch_dev, oracle, t, n_expert, rows, n_in, seed, distinct=None):
    """Expert tensor [n_expert][rows][n_in] packed like FISH (expert slices contiguous), repacked on device.
    With `distinct`, only that many experts are generated and the rest repeat them."""
    d = distinct or n_expert
    packed = np.concatenate([oracle.quantize_rows(t, normal(seed + e, (rows, n_in), 0.02)) for e in range(d)])
    if d < n_expert:
        packed = np.tile(packed, n_expert // d)
    return packed, fh.repack(t, dev(torch_dev, packed), n_in, n_expert * rows)


def check_stages(torch_dev, oracle, x, logits, parts, out, n_ff, k, types, packed):
    """Each stage of one layer against the oracle on the GPU's own stage inputs."""
    tg, tu, td = types
    pg, pu, pd = packed
    n_tok, n_embd = x.shape
    p = {name: v.cpu().numpy() for name, v in parts.items()}
    want_sel, want_w = oracle.route(logits, k, True)
    assert np.array_equal(p["sel"], want_sel)
    assert np.allclose(p["wsel"], want_w, rtol=0, atol=1e-6)
    # slots: every (token, choice) once, grouped by expert, tokens ascending within an expert
    tok_slot, slot_tok = p["tok_slot"], p["slot_tok"]
    assert np.array_equal(np.sort(tok_slot.reshape(-1)), np.arange(n_tok * k))
    assert np.array_equal(slot_tok[tok_slot], np.repeat(np.arange(n_tok)[:, None], k, axis=1))
    exp_of = np.empty(n_tok * k, np.int64)
    exp_of[tok_slot.reshape(-1)] = p["sel"].reshape(-1)
    key = exp_of * n_tok + slot_tok
    assert np.all(np.diff(key) > 0)
    # gate / up products of each expert's tokens
    bg, bu, bd = (fh.gguf_row_bytes(tg, n_embd) * n_ff, fh.gguf_row_bytes(tu, n_embd) * n_ff,
                  fh.gguf_row_bytes(td, n_ff) * n_embd)
    g_ref, u_ref = np.zeros_like(p["gate"]), np.zeros_like(p["up"])
    experts = np.unique(exp_of)
    for e in experts:
        sl = np.nonzero(exp_of == e)[0]
        g_ref[sl] = oracle.matmul_f32(tg, pg[e * bg:(e + 1) * bg], x[slot_tok[sl]], n_ff)
        u_ref[sl] = oracle.matmul_f32(tu, pu[e * bu:(e + 1) * bu], x[slot_tok[sl]], n_ff)
    check_close(p["gate"], g_ref, "gate products")
    check_close(p["up"], u_ref, "up products")
    # hidden rows: the requantization of the GPU's own silu(g)*u is FISH's, bit for bit
    _, q256, h = fh.silu_mul_quantize(dev(torch_dev, p["gate"]), dev(torch_dev, p["up"]))
    h = h.cpu().numpy()
    if q256 is not None:
        assert np.array_equal(q256.cpu().numpy(), oracle.quantize_acts_k(h))
    d_ref = np.zeros_like(p["down"])
    for e in experts:
        sl = np.nonzero(exp_of == e)[0]
        d_ref[sl] = oracle.matmul_f32(td, pd[e * bd:(e + 1) * bd], h[sl], n_embd)
    check_close(p["down"], d_ref, "down products")
    # combine in ascending expert order, w * down rounded, then added
    want = np.zeros((n_tok, n_embd), np.float32)
    for t in range(n_tok):
        acc = np.zeros(n_embd, np.float32)
        for i in np.argsort(p["sel"][t], kind="stable"):
            acc = acc + p["wsel"][t, i] * p["down"][tok_slot[t, i]]
        want[t] = acc
    assert np.array_equal(out, want)
    # what the hidden requantization may move: FISH's own hidden values (oracle gate/up on
    # the same x, FISH's silu * up) against the GPU's, code by code
    return hidden_bound(oracle, g_ref, u_ref, h, td, pd, exp_of, p["wsel"], tok_slot, n_embd, n_ff, k)


def hidden_bound(oracle, g_fish, u_fish, h_gpu, td, pd, exp_of, wsel, tok_slot, n_embd, n_ff, k):
    """Per-token bound on how far the layer output may move because the hidden values that reach
    the down projection differ: FISH's own (silu(g_fish) * u_fish, requantized) against the GPU's
    (h_gpu, requantized), both [slot][n_ff]. Returns (bound [n_tok], (flipped codes, differing block
    scales, blocks, differing dequantized values))."""
    n_tok = tok_slot.shape[0]
    k_layout = fh.BLOCK_ELEMS[td] == 256
    bd = fh.gguf_row_bytes(td, n_ff) * n_embd
    h_fish = oracle.silu_mul(g_fish, u_fish)
    a_gpu = oracle.act_batch(h_gpu)[1 if k_layout else 0]
    a_fish = oracle.act_batch(h_fish)[1 if k_layout else 0]
    delta = np.abs(act_values(a_gpu, k_layout) - act_values(a_fish, k_layout)).reshape(n_tok * k, n_ff)
    size, qoff = (276, 20) if k_layout else (40, 8)
    b_gpu, b_fish = a_gpu.reshape(-1, size), a_fish.reshape(-1, size)
    n_codes = int(np.count_nonzero(b_gpu[:, qoff:] != b_fish[:, qoff:]))
    n_scales = int(np.count_nonzero(np.any(b_gpu[:, :4] != b_fish[:, :4], axis=1)))
    slot_bound = np.zeros(n_tok * k)
    for e in np.unique(exp_of):
        sl = np.nonzero(exp_of == e)[0]
        sl = sl[np.any(delta[sl] > 0, axis=1)]
        if sl.size == 0:
            continue
        w_e = oracle.dequant_row(td, pd[e * bd:(e + 1) * bd], n_embd * n_ff).reshape(n_embd, n_ff)
        colmax = np.max(np.abs(w_e.astype(np.float64)), axis=0)
        slot_bound[sl] = delta[sl] @ colmax
    tok_bound = np.array([sum(abs(float(wsel[t, i])) * slot_bound[tok_slot[t, i]] for i in range(k))
                          for t in range(n_tok)])
    return tok_bound, (n_codes, n_scales, b_gpu.shape[0], int(np.count_nonzero(delta)))


def act_values(buf, k_layout):
    """Dequantized values d * q of FISH's Q8ActK (276-byte) or Q8Act (40-byte) blocks, float64."""
    size, qoff = (276, 20) if k_layout else (40, 8)
    blk = buf.reshape(-1, size)
    d = blk[:, :4].copy().view(np.float32).astype(np.float64)
    q = blk[:, qoff:].view(np.int8).astype(np.float64)
    return (d * q).reshape(-1)


def run_case(torch_dev, oracle, n_tok, n_embd, n_ff, n_expert, k, types, seed, distinct=None, favour=None):
    torch, d = torch_dev
    tg, tu, td = types
    pg, wg = repacked_experts(torch_dev, oracle, tg, n_expert, n_ff, n_embd, seed, distinct)
    pu, wu = repacked_experts(torch_dev, oracle, tu, n_expert, n_ff, n_embd, seed + 100, distinct)
    pd, wd = repacked_experts(torch_dev, oracle, td, n_expert, n_embd, n_ff, seed + 200, distinct)
    x = normal(seed + 300, (n_tok, n_embd))
    logits = normal(seed + 301, (n_tok, n_expert))
    if favour is not None:
        logits[:, favour] += np.float32(8.0)  # every token picks this expert (skewed counts)
    ws = torch.empty(fh.moe_workspace_bytes(n_tok, n_embd, n_ff, n_expert, k), dtype=torch.uint8, device=d)
    out = fh.moe_ffn(dev(torch_dev, x), dev(torch_dev, logits), n_ff, n_expert, k, True, tg, wg, tu, wu, td, wd,
                     workspace=ws).cpu().numpy()
    parts = fh.moe_parts(ws, n_tok, n_embd, n_ff, n_expert, k)
    tok_bound, (codes, scales, blocks, moved) = check_stages(torch_dev, oracle, x, logits, parts, out, n_ff, k, types,
                                                             (pg, pu, pd))
    want = oracle.moe_ffn(x, logits, n_embd, n_ff, n_expert, k, True, tg, pg, tu, pu, td, pd)
    err = np.abs(out.astype(np.float64) - want)
    scale = float(np.max(np.abs(want)))
    allowed = TOL * scale + np.broadcast_to(tok_bound[:, None], err.shape)
    worst = np.unravel_index(int(np.argmax(err / allowed)), err.shape)
    print(f"moe M={n_tok} E={n_embd} F={n_ff} NE={n_expert} k={k}: against FISH's requantization {codes} of "
          f"{n_tok * k * n_ff} hidden codes flipped, {scales} of {blocks} block scales differ; max err "
          f"{float(err.max()):.3e} = {float(err.max()) / scale:.2e} of max|out|; at the tightest element err "
          f"{float(err[worst]):.3e} vs allowed {float(allowed[worst]):.3e}")
    assert np.all(err <= allowed), f"moe M={n_tok}: err {float(err[worst]):.3e} > {float(allowed[worst]):.3e}"
    if moved == 0:  # nothing to excuse: the plain bar
        check_close(out, want, f"moe M={n_tok} E={n_embd} F={n_ff} NE={n_expert} k={k}")


def test_moe_matches_reference_golden(torch_dev, golden):
    g = golden("moe")
    E, F, NE, K = int(g["E"]), int(g["F"]), int(g["NE"]), int(g["K"])
    wg = fh.repack(fh.Q4_K, dev(torch_dev, g["gate"]), E, NE * F)
    wu = fh.repack(fh.Q4_K, dev(torch_dev, g["up"]), E, NE * F)
    wd = fh.repack(fh.Q6_K, dev(torch_dev, g["down"]), F, NE * E)
    out = fh.moe_ffn(dev(torch_dev, g["x"]), dev(torch_dev, g["logits"]), F, NE, K, True, fh.Q4_K, wg, fh.Q4_K, wu,
                     fh.Q6_K, wd)
    check_close(out.cpu().numpy(), g["out"], "golden MoE layer")


@pytest.mark.parametrize("n_tok", [1, 5, 20, 64, 160])
def test_moe_mixtral_like(torch_dev, oracle, n_tok):
    run_case(torch_dev, oracle, n_tok, 512, 1024, 8, 2, (fh.Q4_K, fh.Q4_K, fh.Q4_K), 1000 + n_tok)


@pytest.mark.parametrize("n_tok", [1, 33, 96])
def test_moe_qwen3_like(torch_dev, oracle, n_tok):
    run_case(torch_dev, oracle, n_tok, 512, 256, 32, 8, (fh.Q4_K, fh.Q4_K, fh.Q6_K), 2000 + n_tok)


@pytest.mark.parametrize("n_embd,n_ff,k,types", [
    (512, 4096, 4, (fh.Q4_K, fh.Q4_K, fh.Q6_K)),
    (256, 2560, 4, (fh.Q4_0, fh.Q4_0, fh.Q8_0)),
    (256, 512, 8, (fh.Q8_0, fh.Q8_0, fh.Q4_0)),
])
def test_moe_decode_hidden_sizes(torch_dev, oracle, n_embd, n_ff, k, types):
    """One token: hidden rows quantized by the down workgroups themselves
    (k * n_ff <= 8192) or once by the quantize kernel (larger)."""
    run_case(torch_dev, oracle, 1, n_embd, n_ff, 8, k, types, 6000 + n_ff + k)


@pytest.mark.parametrize("n_tok", [1, 20, 160])
def test_moe_q5_k_experts(torch_dev, oracle, n_tok):
    """Q5_K gate/up with Q6_K down (a Q5_K_M file's experts): the one-token
    kernels, the grouped few-token kernel and the grouped GEMM."""
    run_case(torch_dev, oracle, n_tok, 512, 1024, 8, 2, (fh.Q5_K, fh.Q5_K, fh.Q6_K), 8000 + n_tok)


@pytest.mark.parametrize("n_tok,n_expert,k,favour", [(100, 8, 2, 0), (96, 32, 8, 5), (40, 8, 2, 7)])
def test_moe_skewed_routing(torch_dev, oracle, n_tok, n_expert, k, favour):
    """One expert chosen by every token: its slots span several work-list items
    (more than one 32-token item), the other experts get few or none."""
    run_case(torch_dev, oracle, n_tok, 512, 512, n_expert, k, (fh.Q4_K, fh.Q4_K, fh.Q6_K), 7000 + n_tok,
             favour=favour)


def test_moe_mixed_types(torch_dev, oracle):
    run_case(torch_dev, oracle, 9, 256, 512, 4, 2, (fh.Q8_0, fh.Q4_0, fh.Q6_K), 3000)


def test_moe_mixtral_full_size_decode(torch_dev, oracle):
    """Mixtral-8x7B expert shapes at M=1 (one distinct expert, replicated)."""
    run_case(torch_dev, oracle, 1, 4096, 14336, 8, 2, (fh.Q4_K, fh.Q4_K, fh.Q4_K), 4000, distinct=1)


def test_moe_qwen3_full_size(torch_dev, oracle):
    """Qwen3-30B-A3B expert shapes, 128 experts (8 distinct, repeated), M=24."""
    run_case(torch_dev, oracle, 24, 2048, 768, 128, 8, (fh.Q4_K, fh.Q4_K, fh.Q6_K), 5000, distinct=8)


def test_moe_mixtral_full_size_batched(torch_dev, oracle):
    """Mixtral-8x7B expert shapes at M=64 (E=4096, F=14336, 8 experts, top-2; two distinct
    experts, repeated): the grouped MFMA batch kernel in work-list mode at K=4096 and K=14336."""
    run_case(torch_dev, oracle, 64, 4096, 14336, 8, 2, (fh.Q4_K, fh.Q4_K, fh.Q4_K), 4100, distinct=2)


def test_moe_qwen3_full_size_decode(torch_dev, oracle):
    """Qwen3-30B-A3B expert shapes at M=1 (E=2048, F=768, 128 experts, top-8): the one-token
    expert kernels."""
    run_case(torch_dev, oracle, 1, 2048, 768, 128, 8, (fh.Q4_K, fh.Q4_K, fh.Q6_K), 5100, distinct=16)


def test_moe_qwen3_full_size_prefill(torch_dev, oracle):
    """Qwen3-30B-A3B expert shapes at M=256 (128 experts, top-8, skewed per-expert counts from
    N(0, 1) logits): grouped batch-kernel items over all 128 experts."""
    run_case(torch_dev, oracle, 256, 2048, 768, 128, 8, (fh.Q4_K, fh.Q4_K, fh.Q6_K), 5200, distinct=16)


@pytest.mark.parametrize("n_tok", [1, 20, 64])
def test_backend_moe_ffn_on_host_buffers(torch_dev, oracle, n_tok):
    """fish_hip_backend_moe_ffn: the expert tensors uploaded through the backend as 3-D tensors
    (n_expert = ne[2]), x / logits / out in host memory. Bit-identical to fish_hip_moe_ffn on
    device pointers; with a resident f32 router tensor the logits are computed on the device
    (= router_logits then moe_ffn); refusals leave out untouched."""
    torch, d = torch_dev
    be = fh.HipBackend()
    E, F, NE, K = 512, 1024, 8, 2
    types = (fh.Q4_K, fh.Q4_K, fh.Q6_K)
    tg, tu, td = types
    pg, wg = repacked_experts(torch_dev, oracle, tg, NE, F, E, 8100)
    pu, wu = repacked_experts(torch_dev, oracle, tu, NE, F, E, 8200)
    pd, wd = repacked_experts(torch_dev, oracle, td, NE, E, F, 8300)
    names = [f"bmoe{n_tok}.{n}" for n in ("gate", "up", "down")]
    assert be.upload(names[0], tg, pg, E, F, NE) and be.upload(names[1], tu, pu, E, F, NE)
    assert be.upload(names[2], td, pd, F, E, NE)
    wr = normal(8400, (NE, E), 0.05)
    assert be.upload(f"bmoe{n_tok}.router", fh.F32, wr.view(np.uint8), E, NE)
    try:
        x = normal(8500 + n_tok, (n_tok, E))
        logits = normal(8600 + n_tok, (n_tok, NE))
        served = int(fh.load().fish_hip_backend_served())
        got = be.moe_ffn(names, x, logits, F, NE, K)
        assert got is not None, fh.last_error()
        assert int(fh.load().fish_hip_backend_served()) == served + 1
        want = fh.moe_ffn(dev(torch_dev, x), dev(torch_dev, logits), F, NE, K, True, tg, wg, tu, wu, td, wd)
        assert np.array_equal(got, want.cpu().numpy())
        # router logits on the device from the resident router tensor
        got_r = be.moe_ffn(names, x, None, F, NE, K, router=f"bmoe{n_tok}.router")
        lg = fh.router_logits(dev(torch_dev, x), dev(torch_dev, wr))
        want_r = fh.moe_ffn(dev(torch_dev, x), lg, F, NE, K, True, tg, wg, tu, wu, td, wd)
        assert np.array_equal(got_r, want_r.cpu().numpy())
        # refusals: expert count or widths that do not match the resident tensors
        assert be.moe_ffn(names, x, logits[:, :4], F, 4, K) is None
        assert be.moe_ffn(names, x, logits, F // 2, NE, K) is None
        assert be.moe_ffn([names[0], names[1], "bmoe.absent"], x, logits, F, NE, K) is None
        # a 2-D tensor is not an expert tensor: the router as gate is refused
        assert be.moe_ffn([f"bmoe{n_tok}.router", names[1], names[2]], x, logits, F, NE, K) is None
    finally:
        for n in names + [f"bmoe{n_tok}.router"]:
            be.release(n)
