"""FISH's own host code driving the HIP path: the drop-in test.

oracle/_ref/libfishref_hip.so holds the reference's ops/quant/gguf sources
(compiled where they lie) and the FISH-side backend binding
(imurun_amd/fish_side/hip_backend.cpp), which registers itself with FISH at
load like the Vulkan backend (vulkan_backend.cpp:2168-2177). The tests do
what FISH's loader and forward pass do -- supports() and upload() per weight
tensor, then matmul_tensor / matmul_tensors (ops.cpp:283-299) -- and compare
with FISH's CPU matmul_batch on the same bytes (max error <= 1e-4 of the
output's L-inf norm). The library exists only where the reference sources
were present at build time; without it these tests skip.
"""
import numpy as np
import pytest

import imurun_amd as fh
from imurun_amd.synth import normal, uniform
from oracle.oracle import DropIn

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not DropIn.available(), reason="oracle/_ref/libfishref_hip.so not built")]

TOL = 1e-4
Q8_1 = 9  # a type in FISH's size table that neither FISH's matmul nor this backend multiplies


@pytest.fixture(scope="module")
def drop():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    d = DropIn()
    assert d.backend_name() == "hip", "the HIP binding did not register with FISH"
    return d


def served() -> int:
    """Device matmuls computed so far (the backend's own count, same library instance)."""
    return int(fh.load().fish_hip_backend_served())


def check(got, want, what):
    err = float(np.max(np.abs(got - want)))
    scale = float(np.max(np.abs(want)))
    assert err <= TOL * scale, f"{what}: max err {err:.3e} vs {TOL} * {scale:.3e}"


@pytest.mark.parametrize("t", [fh.Q8_0, fh.Q4_0, fh.Q4_K, fh.Q5_K, fh.Q6_K])
@pytest.mark.parametrize("n_in,n_out", [(1024, 384), (4096, 512)])
def test_matmul_tensor_through_fish_routing(drop, t, n_in, n_out):
    packed = fh.quantize_rows(t, normal(300 + t + n_in, (n_out, n_in), 0.02))
    h = drop.tensor(t, packed, n_in, n_out)
    try:
        before = drop.bytes_resident()
        assert drop.upload(h) and drop.resident(h)
        assert drop.bytes_resident() > before
        for m in (1, 4, 17, 64, 130):
            x = normal(310 + m + t, (m, n_in), 1.0)
            n0 = served()
            y = drop.matmul_tensor(h, x)
            assert served() == n0 + 1, "FISH did not get this matmul from the device"
            check(y, drop.matmul_cpu(h, x), f"type {t} {n_out}x{n_in} M={m}")
        drop.release(h)
        assert not drop.resident(h)
    finally:
        drop.free(h)


@pytest.mark.parametrize("t", [fh.Q4_0, fh.Q4_K])
@pytest.mark.parametrize("m", [1, 5, 96])
def test_matmul_tensors_gate_up_group(drop, t, m):
    # gate and up on the same x: matmul_tensors -> ComputeBackend::matmul_group
    n_in, n_out = 2048, 1536
    hs = [drop.tensor(t, fh.quantize_rows(t, normal(320 + i + t, (n_out, n_in), 0.02)), n_in, n_out)
          for i in range(2)]
    try:
        for h in hs:
            assert drop.upload(h)
        x = normal(330 + m, (m, n_in), 1.0)
        n0 = served()
        ys = drop.matmul_tensors(hs, x)
        assert served() == n0 + 1, "the group was not one device call"
        for i, h in enumerate(hs):
            check(ys[i], drop.matmul_cpu(h, x), f"group member {i}, M={m}")
    finally:
        for h in hs:
            drop.release(h)
            drop.free(h)


@pytest.mark.parametrize("t", [fh.Q4_1, fh.Q3_K, fh.MXFP4, fh.F16])
def test_f32_path_types_through_fish_routing(drop, t):
    # types FISH multiplies in f32 go to the device as well (their GGUF bytes, dequantised there)
    from test_gpu_f32path import rows_of
    n_in, n_out = 1024, 96
    h = drop.tensor(t, rows_of(t, n_out, n_in, 350 + t), n_in, n_out)
    try:
        assert drop.upload(h) and drop.resident(h)
        for m in (1, 7):
            x = normal(351 + m, (m, n_in), 1.0)
            n0 = served()
            y = drop.matmul_tensor(h, x)
            assert served() == n0 + 1
            check(y, drop.matmul_cpu(h, x), f"{fh.TYPE_NAMES[t]} M={m}")
        drop.release(h)
    finally:
        drop.free(h)


def test_unsupported_type_stays_on_the_cpu(drop):
    # supports() is false, upload() is never attempted, matmul_tensor takes FISH's CPU path
    n_in, n_out = 512, 64
    packed = (uniform(340, n_out * n_in // 32 * 36) * 256).astype(np.uint8)
    h = drop.tensor(Q8_1, packed, n_in, n_out)
    try:
        assert not drop.upload(h) and not drop.resident(h)
        x = normal(341, (3, n_in), 1.0)
        n0 = served()
        assert np.array_equal(drop.matmul_tensor(h, x), drop.matmul_cpu(h, x))
        assert served() == n0
    finally:
        drop.free(h)


@pytest.mark.parametrize("n_tok,types", [(9, (fh.Q4_K, fh.Q4_K, fh.Q6_K)), (40, (fh.Q4_K, fh.Q5_K, fh.Q6_K)),
                                         (1, (fh.Q4_K, fh.Q4_K, fh.Q4_K)), (5, (fh.Q8_0, fh.Q4_0, fh.Q6_K))])
def test_moe_ffn_through_fish_expert_tensors(drop, oracle, n_tok, types):
    """FISH's three 3-D expert TensorInfos uploaded through FISH's backend (upload() with
    ne[2] experts), then the expert hook as the patched model.cpp calls it after the router
    matmul: bit-identical to the device-pointer expert FFN, and against FISH's own CPU
    moe_ffn composition (compiled from the reference, AVX2 matmul_batch) within 1e-4 of
    max|out| plus the movement FISH's own hidden values explain (their int8 requantization
    is discontinuous: FISH's scalar and AVX2 paths differ by 1e-3 on the 9-token case)."""
    import torch
    from oracle.oracle import Ref
    from test_gpu_moe import hidden_bound
    tg, tu, td = types
    E, F, NE, K = 256, 512, 8, 2
    d = torch.device("cuda:0")
    pg = np.concatenate([fh.quantize_rows(tg, normal(9000 + e, (F, E), 0.02)) for e in range(NE)])
    pu = np.concatenate([fh.quantize_rows(tu, normal(9100 + e, (F, E), 0.02)) for e in range(NE)])
    pd = np.concatenate([fh.quantize_rows(td, normal(9200 + e, (E, F), 0.02)) for e in range(NE)])
    hs = [drop.tensor3(tg, pg, E, F, NE), drop.tensor3(tu, pu, E, F, NE), drop.tensor3(td, pd, F, E, NE)]
    try:
        for h in hs:
            assert drop.upload(h) and drop.resident(h)
        x = normal(9300 + n_tok, (n_tok, E))
        logits = normal(9400 + n_tok, (n_tok, NE))
        before = served()
        got = drop.moe_ffn(hs, x, logits, F, NE, K)
        assert got is not None and served() == before + 1
        # the device-pointer path on the same bytes, with its intermediate buffers
        tx, tl = torch.from_numpy(x).to(d), torch.from_numpy(logits).to(d)
        wg, wu, wd = (fh.repack(t, torch.from_numpy(p).to(d), n_in, NE * n_out)
                      for t, p, n_in, n_out in ((tg, pg, E, F), (tu, pu, E, F), (td, pd, F, E)))
        ws = torch.empty(fh.moe_workspace_bytes(n_tok, E, F, NE, K), dtype=torch.uint8, device=d)
        dev_out = fh.moe_ffn(tx, tl, F, NE, K, True, tg, wg, tu, wu, td, wd, workspace=ws).cpu().numpy()
        assert np.array_equal(got, dev_out)
        # FISH's own CPU composition, and the bound from FISH's AVX2 gate / up products
        ref = Ref()
        want, _, _ = ref.moe_ffn(x, logits, E, F, NE, K, True, tg, pg, tu, pu, td, pd)
        p = {n: v.cpu().numpy() for n, v in fh.moe_parts(ws, n_tok, E, F, NE, K).items()}
        exp_of = np.empty(n_tok * K, np.int64)
        exp_of[p["tok_slot"].reshape(-1)] = p["sel"].reshape(-1)
        bg, bu = fh.gguf_row_bytes(tg, E) * F, fh.gguf_row_bytes(tu, E) * F
        g_f, u_f = np.zeros_like(p["gate"]), np.zeros_like(p["up"])
        for e in np.unique(exp_of):
            sl = np.nonzero(exp_of == e)[0]
            g_f[sl] = ref.matmul_f32(tg, pg[e * bg:(e + 1) * bg], x[p["slot_tok"][sl]], F)
            u_f[sl] = ref.matmul_f32(tu, pu[e * bu:(e + 1) * bu], x[p["slot_tok"][sl]], F)
        _, _, h_gpu = fh.silu_mul_quantize(torch.from_numpy(p["gate"]).to(d), torch.from_numpy(p["up"]).to(d))
        bound, (codes, scales, blocks, _) = hidden_bound(oracle, g_f, u_f, h_gpu.cpu().numpy(), td, pd, exp_of,
                                                         p["wsel"], p["tok_slot"], E, F, K)
        err = np.abs(got.astype(np.float64) - want)
        allowed = TOL * float(np.max(np.abs(want))) + np.broadcast_to(bound[:, None], err.shape)
        print(f"drop-in moe M={n_tok}: {codes} codes / {scales} of {blocks} scales differ from FISH's AVX2 "
              f"requantization; max err {float(err.max()):.3e}, max allowed {float(allowed.max()):.3e}")
        assert np.all(err <= allowed)
    finally:
        for h in hs:
            drop.release(h)
            drop.free(h)
