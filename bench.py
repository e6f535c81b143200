"""Benchmark of the MI355X quantized-matmul path (one GPU).

Workload (one step): the Llama-3-8B FFN at decode, Q4_0 weights, M = 1:
  gate + up GEMV (2 x 14336 x 4096) on x (1 x 4096, int8-quantized in the
  same launch) -> down GEMV (4096 x 14336) on h (1 x 14336, likewise)
Weights are f32 N(0, 0.02) packed to Q4_0 by FISH's block writer; inputs are
N(0, 1); every step uses the next of several weight copies so the 256 MB
Infinity Cache never holds the step's weights. value = algorithmic bytes of
the step (weights + f32 x read + f32 y written) / step time.

Also reported: the M = 512 prefill of one Llama-3-8B layer in Q4_K / Q6_K
(int8 TOPS), and the reference's own AVX2 CPU path on the host cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S]
"""
from __future__ import annotations

import argparse
import json

import numpy as np
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA
MALL_BYTES = 256 << 20

E, F = 4096, 14336             # Llama-3-8B hidden / FFN width


def gemv_step_bytes():
    """Algorithmic bytes of the step and of its dominant launch (gate + up on one x)."""
    import imurun_amd as fh
    w = fh.gguf_row_bytes(fh.Q4_0, E) * F
    gate_up = 2 * w + E * 4 + 2 * F * 4
    down = fh.gguf_row_bytes(fh.Q4_0, F) * E + F * 4 + E * 4
    return gate_up + down, gate_up


def run_gemv(args, torch, fh, dev):
    from imurun_amd.synth import normal
    t = fh.Q4_0
    wg = fh.quantize_rows(t, normal(101, (F, E), 0.02))
    wu = fh.quantize_rows(t, normal(102, (F, E), 0.02))
    wd = fh.quantize_rows(t, normal(103, (E, F), 0.02))
    step_w = wg.size + wu.size + wd.size
    copies = max(2, int(2 * MALL_BYTES // step_w) + 2)
    sets = []
    for c in range(copies):
        sets.append(tuple(fh.repack(t, torch.from_numpy(a).to(dev), n_in, n_out)
                          for a, n_in, n_out in ((wg, E, F), (wu, E, F), (wd, F, E))))
    x = torch.from_numpy(normal(104, (1, E))).to(dev)
    h = torch.from_numpy(normal(105, (1, F))).to(dev)
    yg = torch.empty((1, F), dtype=torch.float32, device=dev)
    yu = torch.empty((1, F), dtype=torch.float32, device=dev)
    yd = torch.empty((1, E), dtype=torch.float32, device=dev)

    def step(c):
        # matmul_tensors on f32 input: gate and up share one launch that
        # quantizes x per workgroup; down quantizes h the same way
        g, u, d = sets[c]
        fh.matmul_tensors(t, [g, u], x, [F, F], ys=[yg, yu])
        fh.matmul_tensors(t, [d], h, [E], ys=[yd])

    # HIP graphs of whole rotations: one graph runs `copies` consecutive steps
    # (2 launches each) so host launch latency stays out of the GPU's way; a
    # second graph runs the remaining K mod copies steps -> exactly K steps
    for c in range(copies):
        step(c)
    torch.cuda.synchronize()
    cs = torch.cuda.Stream()

    def capture(n_steps):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(cs):
            with torch.cuda.graph(g, stream=cs):
                for c in range(n_steps):
                    step(c % copies)
        return g

    full = capture(copies)
    rest = capture(args.steps % copies) if args.steps % copies else None
    torch.cuda.synchronize()
    with torch.cuda.stream(cs):
        for _ in range(max(1, args.warmup // copies)):
            full.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps // copies):
            full.replay()
        if rest is not None:
            rest.replay()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0

    # the dominant kernel alone: the fused gate+up GEMV, one graph of
    # back-to-back launches over every weight copy, HIP events around the
    # replays on the graph's stream -> average duration per launch
    def gates():
        for c in range(copies):
            fh.matmul_tensors(t, [sets[c][0], sets[c][1]], x, [F, F], ys=[yg, yu])
    gate_us = graph_time(torch, [gates], max(20, args.steps // 2)) / copies
    return elapsed, copies, gate_us


def run_prefill(args, torch, fh, dev):
    """One Llama-3-8B layer's projections at M = 512 (Q4_K; down in Q6_K): q/k/v and
    gate/up each as one grouped launch on the same activations, as FISH's matmul_tensors.
    Successive layer steps use the next of several weight copies, so no step finds the
    previous step's weights in the 256 MB MALL."""
    from imurun_amd.synth import normal
    M = 512
    shapes = [("q", fh.Q4_K, E, E), ("k", fh.Q4_K, 1024, E), ("v", fh.Q4_K, 1024, E), ("o", fh.Q4_K, E, E),
              ("gate", fh.Q4_K, F, E), ("up", fh.Q4_K, F, E), ("down", fh.Q6_K, E, F)]
    # 1024 distinct packed rows per tensor, repeated to the full height (timing does not depend on values)
    base, layer_bytes = {}, 0
    for i, (name, t, n_out, n_in) in enumerate(shapes):
        base[name] = torch.from_numpy(fh.quantize_rows(t, normal(200 + i, (1024, n_in), 0.02))).to(dev)
        layer_bytes += base[name].numel() * (n_out // 1024)
    copies = max(2, int(2 * MALL_BYTES // layer_bytes) + 2)
    ws = [{name: (t, n_out, n_in, fh.repack(t, base[name].repeat(n_out // 1024), n_in, n_out))
           for name, t, n_out, n_in in shapes} for _ in range(copies)]
    x = torch.from_numpy(normal(210, (M, E))).to(dev)
    hx = torch.from_numpy(normal(211, (M, F))).to(dev)
    ax = torch.empty(fh.act_bytes(M, E), dtype=torch.uint8, device=dev)
    ah = torch.empty(fh.act_bytes(M, F), dtype=torch.uint8, device=dev)
    ys = {name: torch.empty((M, n_out), dtype=torch.float32, device=dev) for name, _, n_out, _ in shapes}
    ops = sum(2 * M * n_out * n_in for _, _, n_out, n_in in shapes)

    def group(c, names, act):
        t, _, n_in, _ = ws[c][names[0]]
        fh.matmul_group(t, [ws[c][n][3] for n in names], act, M, n_in, [ws[c][n][1] for n in names],
                        ys=[ys[n] for n in names])

    parts = {
        "quantize_x": lambda c: fh.quantize(x, act=ax, for_type=fh.Q4_K),
        "qkv": lambda c: group(c, ["q", "k", "v"], ax),
        "o": lambda c: group(c, ["o"], ax),
        "gate_up": lambda c: group(c, ["gate", "up"], ax),
        "quantize_h": lambda c: fh.quantize(hx, act=ah, for_type=fh.Q6_K),
        "down": lambda c: group(c, ["down"], ah),
    }
    reps = max(10, args.steps // 4)
    layer_us = graph_time(torch, [lambda c=c: [f(c) for f in parts.values()] for c in range(copies)],
                          max(reps, 2 * copies))
    # each part as back-to-back calls over the copies in one graph: a one-launch graph per replay
    # would time the host's graph launches for the short parts, not the kernels
    per = {name: graph_time_seq(torch, [lambda c=c, f=f: f(c) for c in range(copies)] * 2, reps)
           for name, f in parts.items()}
    return ops, layer_us, per, copies


def graph_time(torch, fns, reps):
    """Average time (us) per replay of fns[i % len(fns)] captured as HIP graphs,
    HIP events recorded on the stream the graphs replay on."""
    for f in fns:
        f()
    torch.cuda.synchronize()
    cs = torch.cuda.Stream()
    graphs = []
    with torch.cuda.stream(cs):
        for f in fns:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cs):
                f()
            graphs.append(g)
    torch.cuda.synchronize()
    with torch.cuda.stream(cs):
        for g in graphs:
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(cs)
        for i in range(reps):
            graphs[i % len(graphs)].replay()
        e1.record(cs)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps * 1e3


def graph_time_seq(torch, fns, reps):
    """Average time (us) per call when all of fns run back to back in one HIP graph."""
    return graph_time(torch, [lambda: [f() for f in fns]], reps) / len(fns)


def run_q8_gemv(args, torch, fh, dev):
    """4096 x 4096 Q8_0 GEMV at M = 1 (x quantized per call), rotating copies past the MALL."""
    from imurun_amd.synth import normal
    t, N, K = fh.Q8_0, 4096, 4096
    p = fh.quantize_rows(t, normal(121, (N, K), 0.02))
    copies = int(2 * MALL_BYTES // p.size) + 2
    g = torch.from_numpy(p).to(dev)
    ws = [fh.repack(t, g, K, N) for _ in range(copies)]
    x = torch.from_numpy(normal(122, (1, K))).to(dev)
    a = torch.empty(fh.act_bytes(1, K), dtype=torch.uint8, device=dev)
    y = torch.empty((1, N), dtype=torch.float32, device=dev)
    fns = [lambda w=w: fh.matmul_tensors(t, [w], x, [N], ys=[y]) for w in ws]
    us = graph_time_seq(torch, fns, 40)
    b = p.size + K * 4 + N * 4
    return {"workload": "Q8_0 GEMV 4096x4096, M=1, f32 x quantized in-kernel", "us": round(us, 3),
            "gbs": round(b / us / 1e3, 1), "pct_hbm": round(100 * b / us / 1e3 / HBM_PEAK_GBS, 2)}


def run_kquant_gemv(args, torch, fh, dev, t, name):
    """Llama-3-8B FFN decode (M = 1) on K-quant weights: the fused gate+up GEMV
    (2 x 14336x4096) and the down GEMV (4096x14336), x / h quantized in-kernel,
    rotating copies past the MALL; each kernel graph-timed on its own."""
    from imurun_amd.synth import normal
    wg = fh.quantize_rows(t, normal(141, (F, E), 0.02))
    wu = fh.quantize_rows(t, normal(142, (F, E), 0.02))
    wd = fh.quantize_rows(t, normal(143, (E, F), 0.02))
    copies = max(2, int(2 * MALL_BYTES // (wg.size + wu.size + wd.size)) + 2)
    sets = [tuple(fh.repack(t, torch.from_numpy(a).to(dev), n_in, n_out)
                  for a, n_in, n_out in ((wg, E, F), (wu, E, F), (wd, F, E))) for _ in range(copies)]
    x = torch.from_numpy(normal(144, (1, E))).to(dev)
    h = torch.from_numpy(normal(145, (1, F))).to(dev)
    yg, yu = (torch.empty((1, F), dtype=torch.float32, device=dev) for _ in range(2))
    yd = torch.empty((1, E), dtype=torch.float32, device=dev)
    gu = [lambda s_=s_: fh.matmul_tensors(t, [s_[0], s_[1]], x, [F, F], ys=[yg, yu]) for s_ in sets]
    dn = [lambda s_=s_: fh.matmul_tensors(t, [s_[2]], h, [E], ys=[yd]) for s_ in sets]
    gu_us = graph_time_seq(torch, gu, max(20, args.steps // 4))
    dn_us = graph_time_seq(torch, dn, max(20, args.steps // 4))
    b_gu = wg.size + wu.size + E * 4 + 2 * F * 4
    b_dn = wd.size + F * 4 + E * 4
    return {"workload": f"Llama-3-8B FFN decode, {name}, M=1: gate+up 2x14336x4096 fused, down 4096x14336; "
                        "f32 x / h quantized in-kernel",
            "gate_up_us": round(gu_us, 3), "gate_up_gbs": round(b_gu / gu_us / 1e3, 1),
            "gate_up_pct_hbm": round(100 * b_gu / gu_us / 1e3 / HBM_PEAK_GBS, 2),
            "down_us": round(dn_us, 3), "down_gbs": round(b_dn / dn_us / 1e3, 1),
            "down_pct_hbm": round(100 * b_dn / dn_us / 1e3 / HBM_PEAK_GBS, 2)}


def run_f32path_gemv(args, torch, fh, dev):
    """Types FISH multiplies in f32: one 14336x4096 (Llama-3-8B gate) matrix at M = 1, GGUF
    bytes dequantised in the kernel, f32 x; random code bytes with sane scales (the kernel's work
    does not depend on the values); copies rotated past the MALL."""
    from imurun_amd.synth import uniform
    out = {"workload": "14336x4096 GEMV, M=1, f32 x, weights dequantised in-kernel (FISH's f32 path)"}
    x = torch.randn((1, E), device=dev)
    y = torch.empty((1, F), dtype=torch.float32, device=dev)
    for t in (fh.Q4_1, fh.Q5_0, fh.Q3_K, fh.IQ4_NL, fh.MXFP4, fh.F16):
        nbytes = fh.gguf_row_bytes(t, E) * F
        raw = (uniform(230 + t, nbytes) * 256).astype(np.uint8)
        be, bb = fh.BLOCK_ELEMS[t], fh.BLOCK_BYTES[t]
        blocks = raw.reshape(-1, bb)
        h = np.array([0.01], np.float16).view(np.uint8)
        if t == fh.MXFP4:
            blocks[:, 0] = 127
        elif t == fh.F16:
            blocks[:] = h
        else:  # f16 scale fields set to a sane value
            off = 108 if t == fh.Q3_K else 0
            blocks[:, off:off + 2] = h
        copies = int(2 * MALL_BYTES // nbytes) + 2
        g = torch.from_numpy(raw).to(dev)
        ws = [fh.repack(t, g, E, F) for _ in range(copies)]
        us = graph_time_seq(torch, [lambda w=w: fh.matmul_tensors(t, [w], x, [F], ys=[y]) for w in ws], 20)
        out[fh.TYPE_NAMES[t]] = {"us": round(us, 2), "gbs": round(nbytes / us / 1e3, 1),
                                 "pct_hbm": round(100 * nbytes / us / 1e3 / HBM_PEAK_GBS, 2)}
    return out


def run_q5k_prefill(args, torch, fh, dev):
    """Q5_K gate+up (2 x 14336x4096, a Q5_K_M layer's FFN input side) at M = 512 as one
    grouped GEMM launch on activations quantized once; 1024 distinct packed rows repeated."""
    from imurun_amd.synth import normal
    M, t = 512, fh.Q5_K
    ws = []
    for seed in (221, 222):
        base = fh.quantize_rows(t, normal(seed, (1024, E), 0.02))
        ws.append(fh.repack(t, torch.from_numpy(base).to(dev).repeat(F // 1024), E, F))
    act = fh.quantize(torch.from_numpy(normal(223, (M, E))).to(dev))
    ys = [torch.empty((M, F), dtype=torch.float32, device=dev) for _ in range(2)]
    us = graph_time_seq(torch, [lambda: fh.matmul_group(t, ws, act, M, E, [F, F], ys=ys)] * 4, 10)
    ops = 2 * 2 * M * F * E
    return {"workload": "Q5_K gate+up GEMM 2 x 14336x4096, M=512, one grouped launch", "us": round(us, 2),
            "tops": round(ops / us / 1e6, 1), "pct_int8_peak": round(100 * ops / us / 1e6 / INT8_PEAK_TOPS, 2)}


def run_span_decode(args, torch, fh, dev):
    """Llama-3-8B layers as one layer span (Q4_K_M mix: q, k, o, gate, up Q4_K; v, down Q6_K) through
    the backend's C ABI: a 512-token prefill, then decode tokens at position 512, each call moving x
    host -> device -> host. Beside it, the same layer routed per matmul (four synchronous backend calls
    with host round trips, FISH's path without spans; its CPU attention is not counted)."""
    from imurun_amd.synth import normal
    L_, H_, HKV_, D_, CTX = 4, 32, 8, 128, 2048
    Qd, KVd = H_ * D_, HKV_ * D_
    types = dict(wq=fh.Q4_K, wk=fh.Q4_K, wv=fh.Q6_K, wo=fh.Q4_K, wg=fh.Q4_K, wu=fh.Q4_K, wd=fh.Q6_K)
    shapes = dict(wq=(Qd, E), wk=(KVd, E), wv=(KVd, E), wo=(E, Qd), wg=(F, E), wu=(F, E), wd=(E, F))
    be = fh.HipBackend()
    host, layer_bytes = {}, 0
    for i, n in enumerate(types):
        n_out, n_in = shapes[n]
        base = fh.quantize_rows(types[n], normal(300 + i, (min(1024, n_out), n_in), 0.02))
        host[n] = np.tile(base, n_out // min(1024, n_out))
        layer_bytes += host[n].size
    layers = []
    for l in range(L_):
        names = []
        for n in types:
            assert be.upload(f"span{l}.{n}", types[n], host[n], shapes[n][1], shapes[n][0])
            names.append(f"span{l}.{n}")
        layers.append((names, np.ones(E, np.float32), np.ones(E, np.float32)))
    half = D_ // 2
    th = np.arange(CTX)[:, None] * (500000.0 ** (-np.arange(half) * 2 / D_))[None, :]
    assert be.span_prepare(layers, E, H_, HKV_, D_, F, CTX, np.cos(th), np.sin(th), rope_neox=False)
    try:
        assert be.span_forward(normal(309, (512, E), 1.0), 0)  # first call sizes the scratch
        x = normal(310, (512, E), 1.0)
        t0 = time.perf_counter()
        assert be.span_forward(x, 0)
        prefill_ms = (time.perf_counter() - t0) * 1e3
        xs = [normal(311 + i, (1, E), 1.0) for i in range(24)]
        times = []
        for xi in xs:
            t0 = time.perf_counter()
            assert be.span_forward(xi, 512)
            times.append(time.perf_counter() - t0)
        dec_us = float(np.median(times[4:])) * 1e6
        # the same layer routed per matmul with host round trips
        x1 = normal(330, (1, E), 1.0)
        h1 = normal(331, (1, F), 1.0)
        a1 = normal(332, (1, Qd), 1.0)
        names = layers[0][0]
        rt = []
        for _ in range(20):
            t0 = time.perf_counter()
            be.matmul_group(names[0:3], x1, [Qd, KVd, KVd])
            be.matmul_group(names[3:4], a1, [E])
            be.matmul_group(names[4:6], x1, [F, F])
            be.matmul_group(names[6:7], h1, [E])
            rt.append(time.perf_counter() - t0)
        routed_us = float(np.median(rt[4:])) * 1e6
    finally:
        be.span_release()
        for names, _, _ in layers:
            for n in names:
                be.release(n)
    per_layer = dec_us / L_
    return {"workload": f"Llama-3-8B layer span, {L_} layers, Q4_K_M mix, decode at position 512 "
                        "(x host->device->host per call)",
            "decode_us_per_token": round(dec_us, 1), "us_per_layer": round(per_layer, 2),
            "layer_weight_bytes": layer_bytes, "gbs": round(layer_bytes / per_layer / 1e3, 1),
            "routed_per_matmul_us_per_layer": round(routed_us, 2),
            "prefill_512_ms": round(prefill_ms, 2),
            "prefill_tok_per_s": round(512 / prefill_ms * 1e3, 1)}


def run_moe(args, torch, fh, dev, name, NE, K, E, F_, types, cases):
    """Expert FFN layer at the given token counts; one distinct expert replicated (same traffic)."""
    from imurun_amd.synth import normal
    tg, tu, td = types
    rows = lambda t, n_out, n_in, seed: fh.quantize_rows(t, normal(seed, (n_out, n_in), 0.02))  # noqa: E731
    pg, pu, pd = rows(tg, F_, E, 131), rows(tu, F_, E, 132), rows(td, E, F_, 133)
    wg = fh.repack(tg, torch.from_numpy(pg).to(dev).repeat(NE), E, NE * F_)
    wu = fh.repack(tu, torch.from_numpy(pu).to(dev).repeat(NE), E, NE * F_)
    wd = fh.repack(td, torch.from_numpy(pd).to(dev).repeat(NE), F_, NE * E)
    per_expert = pg.size + pu.size + pd.size
    wr = torch.from_numpy(normal(136, (NE, E), 0.05)).to(dev)
    out = {"workload": f"{name} expert layer: {NE} experts, top-{K}, hidden {E}, expert FFN {F_}",
           "weights_per_expert_bytes": per_expert}
    for M in cases:
        x = torch.from_numpy(normal(134 + M, (M, E))).to(dev)
        ws = torch.empty(fh.moe_workspace_bytes(M, E, F_, NE, K), dtype=torch.uint8, device=dev)
        y = torch.empty((M, E), dtype=torch.float32, device=dev)
        if M == 1:
            # rotate the chosen experts so successive steps read disjoint weight sets
            sets = NE // K
            logit_sets = []
            for s_ in range(sets):
                lg = np.full((1, NE), -4.0, np.float32)
                lg[0, s_ * K:(s_ + 1) * K] = 4.0 + np.arange(K, dtype=np.float32) * 0.1
                logit_sets.append(torch.from_numpy(lg).to(dev))
            active = K
        else:
            logit_sets = [torch.from_numpy(normal(135 + M, (M, NE))).to(dev)]
            sel, _ = fh.moe_route(logit_sets[0], K, True)
            active = int(np.unique(sel.cpu().numpy()).size)
        fns = [lambda lg=lg: fh.moe_ffn(x, lg, F_, NE, K, True, tg, wg, tu, wu, td, wd, out=y, workspace=ws)
               for lg in logit_sets]
        us = graph_time_seq(torch, fns, max(20, 80 // len(fns)))
        b = active * per_expert + M * E * 8
        ops = 2 * M * K * 3 * E * F_
        # the router matmul before it (model.cpp:1529), f32 router rows [NE][E], timed on its own
        lg_out = torch.empty((M, NE), dtype=torch.float32, device=dev)
        # (16 calls per graph: one short kernel per replay would time the replay, not the kernel)
        router_us = graph_time_seq(torch, [lambda: fh.router_logits(x, wr, out=lg_out)] * 16, 20)
        out[f"M{M}"] = {"us": round(us, 2), "active_experts": active, "bytes": b, "gbs": round(b / us / 1e3, 1),
                        "pct_hbm": round(100 * b / us / 1e3 / HBM_PEAK_GBS, 2), "tops": round(ops / us / 1e6, 2),
                        "router_f32_us": round(router_us, 2)}
    return out


def host_topology():
    """Physical cores and sockets of this host (from /proc/cpuinfo), logical CPUs and the CPUs this
    process may run on: FISH sizes its pool from the physical core count (threadpool.cpp:47-60)."""
    pairs, sockets = set(), set()
    phys = core = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k = k.strip()
                if k == "physical id":
                    phys = v.strip()
                elif k == "core id":
                    core = v.strip()
                elif not k:
                    if phys is not None and core is not None:
                        pairs.add((phys, core))
                        sockets.add(phys)
                    phys = core = None
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"physical_cores": len(pairs) or None, "sockets": len(sockets) or None,
            "logical_cpus": os.cpu_count(), "affinity_cpus": affinity}


def timed_loop(fn, seconds, n_sets=1):
    """Run fn(i) once untimed, then until `seconds` have passed (at least once); (calls, elapsed s)."""
    fn(0)
    n, t0 = 0, time.perf_counter()
    while True:
        fn(n % n_sets)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            return n, el


def run_cpu_baseline(args, step_bytes):
    """The reference's own CPU path (FISH's quantize + threaded AVX2 matmul_batch and its moe_ffn
    loop), one bounded sample per workload. FISH picks its thread count itself (FISH_THREADS unset:
    min(physical cores, 32), threadpool.cpp:47-60); FISH_LOW_PRIORITY=0 keeps the pool un-niced."""
    os.environ.pop("FISH_THREADS", None)
    os.environ["FISH_LOW_PRIORITY"] = "0"
    from imurun_amd.synth import normal
    import imurun_amd as fh
    from oracle.oracle import Oracle, Ref
    kind = "reference" if Ref.available() else "port"
    if kind == "reference":
        ref = Ref()
        threads = ref.threads()
        mm = lambda t, w, v, n_out: ref.matmul_f32(t, w, v, n_out)  # noqa: E731
        moe = ref.moe_ffn
    else:
        orc = Oracle()
        orc.threads = 1
        threads = 1
        mm = lambda t, w, v, n_out: orc.matmul_f32(t, w, v, n_out)  # noqa: E731
        moe = orc.moe_ffn
    t = fh.Q4_0
    copies = 4  # > 4x any host LLC: weights come from DRAM like a real decode step
    base = (fh.quantize_rows(t, normal(101, (F, E), 0.02)), fh.quantize_rows(t, normal(102, (F, E), 0.02)),
            fh.quantize_rows(t, normal(103, (E, F), 0.02)))
    sets = [tuple(a.copy() for a in base) for _ in range(copies)]
    x = normal(104, (1, E))
    h = normal(105, (1, F))

    def ffn(i):
        g, u, d = sets[i]
        mm(t, g, x, F)
        mm(t, u, x, F)
        mm(t, d, h, E)
    n, el = timed_loop(ffn, args.cpu_seconds, copies)
    del sets
    out = {"value": round(step_bytes * n / el / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": kind,
           "sample": f"{n} decode FFN steps (Q4_0 gate+up 14336x4096, down 4096x14336, M=1, int8 activations "
                     f"quantized per call) over {copies} weight copies, {el:.1f} s",
           "host": dict(host_topology(), threads_used=threads,
                        thread_policy="FISH default_threads(): min(physical cores, 32), FISH_THREADS unset")}
    if args.no_extras:
        return out
    per = {}
    budget = max(1.0, args.cpu_seconds / 4)

    # Q8_0 GEMV 4096x4096, M=1
    q8 = [fh.quantize_rows(fh.Q8_0, normal(121, (4096, 4096), 0.02)) for _ in range(1)]
    q8 = [q8[0].copy() for _ in range(8)]  # 8 x 17.8 MB copies rotated past the host caches
    xq = normal(122, (1, 4096))
    n, el = timed_loop(lambda i: mm(fh.Q8_0, q8[i], xq, 4096), budget, len(q8))
    us = el / n * 1e6
    b = q8[0].size + 4096 * 8
    per["q8_0_gemv"] = {"us": round(us, 1), "gbs": round(b / us / 1e3, 2),
                        "sample": f"{n} calls over 8 weight copies, {el:.1f} s"}
    del q8

    # Llama-3-8B layer projections at M = 512 (Q4_K; down Q6_K), each matmul quantizing its input
    M = 512
    shapes = [("q", fh.Q4_K, E, E), ("k", fh.Q4_K, 1024, E), ("v", fh.Q4_K, 1024, E), ("o", fh.Q4_K, E, E),
              ("gate", fh.Q4_K, F, E), ("up", fh.Q4_K, F, E), ("down", fh.Q6_K, E, F)]
    lw = {}
    for i, (name, tt, n_out, n_in) in enumerate(shapes):
        lw[name] = np.tile(fh.quantize_rows(tt, normal(200 + i, (1024, n_in), 0.02)), n_out // 1024)
    xp = normal(210, (M, E))
    hp = normal(211, (M, F))

    def layer(_):
        for name, tt, n_out, n_in in shapes:
            mm(tt, lw[name], hp if n_in == F else xp, n_out)
    n, el = timed_loop(layer, budget)
    ops = sum(2 * M * n_out * n_in for _, _, n_out, n_in in shapes)
    per["prefill_layer_m512"] = {"ms": round(el / n * 1e3, 2), "tops": round(ops * n / el / 1e12, 3),
                                 "sample": f"{n} layers (7 matmuls each, M=512), {el:.1f} s"}
    del lw

    # expert layers through FISH's moe_ffn loop (model.cpp:1523-1599)
    for key, NE, K, E_, F_, types, cases in (("moe_mixtral", 8, 2, 4096, 14336, (fh.Q4_K, fh.Q4_K, fh.Q4_K), (1, 64)),
                                             ("moe_qwen3", 128, 8, 2048, 768, (fh.Q4_K, fh.Q4_K, fh.Q6_K), (1, 256))):
        tg, tu, td = types
        pg = fh.quantize_rows(tg, normal(131, (F_, E_), 0.02))
        pu = fh.quantize_rows(tu, normal(132, (F_, E_), 0.02))
        pd = fh.quantize_rows(td, normal(133, (E_, F_), 0.02))
        per_expert = pg.size + pu.size + pd.size
        wg, wu, wd = np.tile(pg, NE), np.tile(pu, NE), np.tile(pd, NE)
        res = {}
        for M_ in cases:
            xm = normal(134 + M_, (M_, E_))
            if M_ == 1:
                lsets = []
                for s_ in range(NE // K):
                    lg = np.full((1, NE), -4.0, np.float32)
                    lg[0, s_ * K:(s_ + 1) * K] = 4.0 + np.arange(K, dtype=np.float32) * 0.1
                    lsets.append(lg)
                active = K
            else:
                lsets = [normal(135 + M_, (M_, NE))]
                active = int(np.unique(Oracle().route(lsets[0], K, True)[0]).size)
            n, el = timed_loop(lambda i: moe(xm, lsets[i], E_, F_, NE, K, True, tg, wg, tu, wu, td, wd),
                               budget, len(lsets))
            us = el / n * 1e6
            b = active * per_expert + M_ * E_ * 8
            res[f"M{M_}"] = {"us": round(us, 1), "gbs": round(b / us / 1e3, 2),
                             "tops": round(2 * M_ * K * 3 * E_ * F_ / us / 1e6, 3),
                             "sample": f"{n} layer calls, {el:.1f} s"}
        per[key] = res
        del wg, wu, wd
    out["per_config"] = per
    return out


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
COPY_BYTES = 256 << 20


def calibration_copy(torch, dev):
    """A plain device copy of COPY_BYTES: what FETCH_SIZE / WRITE_SIZE (and the EA request counters)
    read for known bytes, the factor that turns their per-dispatch values into HBM bytes."""
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()


def kernel_only_launches(name, torch, fh, dev):
    """(description, algorithmic bytes per launch, launch closures) of one decode kernel over weight
    copies rotated past the MALL: the counter passes see the kernels the bench times, on the same
    shapes, each launch reading weights that are not cache resident."""
    from imurun_amd.synth import normal
    if name in ("gemv_gate_up", "q4k_gate_up", "q4k_down"):
        t = fh.Q4_0 if name == "gemv_gate_up" else fh.Q4_K
        down = name == "q4k_down"
        mats = [(103 if t == fh.Q4_0 else 143, F, E)] if down else \
            [(101 if t == fh.Q4_0 else 141, E, F), (102 if t == fh.Q4_0 else 142, E, F)]
        packed = [fh.quantize_rows(t, normal(seed, (n_out, n_in), 0.02)) for seed, n_in, n_out in mats]
        wbytes = sum(p.size for p in packed)
        copies = max(2, int(2 * MALL_BYTES // wbytes) + 2)
        sets = [[fh.repack(t, torch.from_numpy(p).to(dev), n_in, n_out) for p, (_, n_in, n_out) in zip(packed, mats)]
                for _ in range(copies)]
        n_in = mats[0][1]
        x = torch.from_numpy(normal(104, (1, n_in))).to(dev)
        n_outs = [m[2] for m in mats]
        ys = [torch.empty((1, n), dtype=torch.float32, device=dev) for n in n_outs]
        desc = (f"gemv_x_kernel<{fh.TYPE_NAMES[t]}> " +
                ("down 4096x14336" if down else "gate+up 2 x 14336x4096") + ", one token, x quantized in-kernel")
        return desc, wbytes + n_in * 4 + sum(n_outs) * 4, \
            [lambda w=w: fh.matmul_tensors(t, w, x, n_outs, ys=ys) for w in sets]
    if name == "q8_gemv":
        t, N, K = fh.Q8_0, 4096, 4096
        p = fh.quantize_rows(t, normal(121, (N, K), 0.02))
        g = torch.from_numpy(p).to(dev)
        ws = [fh.repack(t, g, K, N) for _ in range(int(2 * MALL_BYTES // p.size) + 2)]
        x = torch.from_numpy(normal(122, (1, K))).to(dev)
        y = torch.empty((1, N), dtype=torch.float32, device=dev)
        return "gemv_x_kernel<Q8_0> 4096x4096, one token, x quantized in-kernel", p.size + K * 4 + N * 4, \
            [lambda w=w: fh.matmul_tensors(t, [w], x, [N], ys=[y]) for w in ws]
    # expert layers: moe_mixtral_m1 / _m64, moe_qwen3_m1 / _m256
    fam, m = name[4:].rsplit("_m", 1)
    M = int(m)
    NE, K, E_, F_, (tg, tu, td) = {"mixtral": (8, 2, 4096, 14336, (fh.Q4_K, fh.Q4_K, fh.Q4_K)),
                                   "qwen3": (128, 8, 2048, 768, (fh.Q4_K, fh.Q4_K, fh.Q6_K))}[fam]
    pg = fh.quantize_rows(tg, normal(131, (F_, E_), 0.02))
    pu = fh.quantize_rows(tu, normal(132, (F_, E_), 0.02))
    pd = fh.quantize_rows(td, normal(133, (E_, F_), 0.02))
    wg = fh.repack(tg, torch.from_numpy(pg).to(dev).repeat(NE), E_, NE * F_)
    wu = fh.repack(tu, torch.from_numpy(pu).to(dev).repeat(NE), E_, NE * F_)
    wd = fh.repack(td, torch.from_numpy(pd).to(dev).repeat(NE), F_, NE * E_)
    per_expert = pg.size + pu.size + pd.size
    x = torch.from_numpy(normal(134 + M, (M, E_))).to(dev)
    ws = torch.empty(fh.moe_workspace_bytes(M, E_, F_, NE, K), dtype=torch.uint8, device=dev)
    y = torch.empty((M, E_), dtype=torch.float32, device=dev)
    if M == 1:
        logit_sets = []
        for s_ in range(NE // K):
            lg = np.full((1, NE), -4.0, np.float32)
            lg[0, s_ * K:(s_ + 1) * K] = 4.0 + np.arange(K, dtype=np.float32) * 0.1
            logit_sets.append(torch.from_numpy(lg).to(dev))
        active = K
    else:
        logit_sets = [torch.from_numpy(normal(135 + M, (M, NE))).to(dev)]
        sel, _ = fh.moe_route(logit_sets[0], K, True)
        active = int(np.unique(sel.cpu().numpy()).size)
    desc = f"{fam} expert layer ({NE} experts, top-{K}, hidden {E_}, FFN {F_}), M={M}"
    return desc, active * per_expert + M * E_ * 8, \
        [lambda lg=lg: fh.moe_ffn(x, lg, F_, NE, K, True, tg, wg, tu, wu, td, wd, out=y, workspace=ws)
         for lg in logit_sets]


KERNEL_ONLY = ["gemv_gate_up", "q8_gemv", "q4k_gate_up", "q4k_down", "moe_mixtral_m1", "moe_mixtral_m64",
               "moe_qwen3_m1", "moe_qwen3_m256", "gemm_gate", "gemm_down"]


def run_kernel_only(args, torch, fh, dev):
    """For rocprofv3 counter passes: one workload's launches `--steps` times over rotated weight
    copies, then the calibration copy."""
    desc, algo, fns = kernel_only_launches(args.kernel_only, torch, fh, dev)
    for i in range(args.steps):
        fns[i % len(fns)]()
    calibration_copy(torch, dev)
    print(json.dumps({"kernel_only": desc, "launches": args.steps, "algorithmic_bytes": algo,
                      "copy_bytes": COPY_BYTES}))
    return 0


def run_kernel_only_gemm(args, torch, fh, dev):
    """For rocprofv3 counter passes: one M = 512 prefill GEMM (Q4_K gate 14336x4096 or Q6_K down
    4096x14336, the prefill layer's weights: 1024 distinct packed rows, repeated) on activations
    quantized once, `--steps` times back to back."""
    from imurun_amd.synth import normal
    M = 512
    t, n_out, n_in, seed = {"gemm_gate": (fh.Q4_K, F, E, 204), "gemm_down": (fh.Q6_K, E, F, 206)}[args.kernel_only]
    base = fh.quantize_rows(t, normal(seed, (1024, n_in), 0.02))
    w = fh.repack(t, torch.from_numpy(base).to(dev).repeat(n_out // 1024), n_in, n_out)
    x = torch.from_numpy(normal(210, (M, n_in))).to(dev)
    act = fh.quantize(x)
    y = torch.empty((M, n_out), dtype=torch.float32, device=dev)
    for _ in range(args.steps):
        fh.matmul_group(t, [w], act, M, n_in, [n_out], ys=[y])
    torch.cuda.synchronize()
    print(json.dumps({"kernel_only": f"gemm_kq_kernel {fh.TYPE_NAMES[t]} {n_out}x{n_in}, M={M}",
                      "launches": args.steps}))
    return 0


# the device sources each counter-pass workload depends on: a traffic figure is reported only for
# the sources it was measured on
_CSRC = os.path.join("imurun_amd", "csrc")
TRAFFIC_SOURCES = {
    "gemv": ["gemv.hip", "rowdot.h", "dots.h", "qact.h", "common.h", "repack.hip"],
    "moe": ["moe.hip", "batch.hip", "quantize.hip", "rowdot.h", "dots.h", "qact.h", "common.h", "repack.hip"],
}


def sources_sha(group):
    import hashlib
    h = hashlib.sha256()
    for f in TRAFFIC_SOURCES[group]:
        with open(os.path.join(ROOT, _CSRC, f), "rb") as fh_:
            h.update(fh_.read())
    return h.hexdigest()[:16]


def measured_traffic(workload):
    """HBM bytes per call of a counter-pass workload from profiles/traffic.json (FETCH_SIZE and
    WRITE_SIZE scaled by a plain copy), with the commit-independent hash of the sources it was
    measured on; (None, reason) when absent or measured on other sources."""
    try:
        with open(TRAFFIC_FILE) as f:
            e = json.load(f)["workloads"][workload]
    except (OSError, ValueError, KeyError):
        return None, "not measured"
    group = "moe" if workload.startswith("moe") else "gemv"
    if e.get("sources_sha") != sources_sha(group):
        return None, f"stale: measured on sources {e.get('sources_sha')}, now {sources_sha(group)}"
    return e, (f"rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes of bench.py --kernel-only {workload}, scaled by "
               f"a 256 MiB copy; sources {e['sources_sha']}")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--kernel-only", nargs="?", const="gemv_gate_up", default=None, choices=KERNEL_ONLY,
                    help="run only one workload's launches --steps times (for rocprofv3 --pmc): a decode "
                         "GEMV or expert layer over rotated weight copies, then a calibration copy; or the "
                         "M=512 Q4_K gate / Q6_K down GEMM")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the path shards by rows/experts "
              "across GPUs but no multi-GPU figure is produced", file=sys.stderr)
        return 2

    import torch
    import imurun_amd as fh
    assert torch.cuda.is_available(), "bench needs a ROCm GPU"
    dev = torch.device("cuda:0")
    fh.load()
    if args.kernel_only in ("gemm_gate", "gemm_down"):
        return run_kernel_only_gemm(args, torch, fh, dev)
    if args.kernel_only:
        return run_kernel_only(args, torch, fh, dev)

    step_bytes, gate_bytes = gemv_step_bytes()
    elapsed, copies, gate_us = run_gemv(args, torch, fh, dev)
    ms = elapsed / args.steps * 1e3
    value = step_bytes / (elapsed / args.steps) / 1e9
    gate_gbs = gate_bytes / (gate_us * 1e-6) / 1e9

    out = {
        "metric": "quant GEMV GB/s (% HBM peak) at M=1; prefill int8 TOPS (% peak) at M=512",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": f"synthetic: W ~ N(0,0.02) packed to Q4_0 by FISH's block writer, x ~ N(0,1); "
                f"{copies} weight copies rotated per step (> 2x the 256 MB MALL)",
        "config": {"workload": "Llama-3-8B FFN decode, Q4_0, M=1: gate+up GEMV 2x14336x4096 and down GEMV "
                               "4096x14336, int8 activations quantized in the same launches",
                   "n_tok": 1, "hidden": E, "ffn": F,
                   "weight_type": "Q4_0", "hbm_pct_of_peak": round(100 * value / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "kernel": "gemv_x_kernel<Q4_0> gate+up 2 x 14336x4096, x quantized in-kernel",
                     "achieved": round(gate_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gate_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "median_kernel_us": round(gate_us, 3), "algorithmic_bytes": gate_bytes},
    }
    tr, why = measured_traffic("gemv_gate_up")
    out["roofline"]["traffic"] = tr["bytes_per_call"] if tr else None
    out["roofline"]["traffic_source"] = why
    if not args.no_extras:
        out["q8_0_gemv"] = run_q8_gemv(args, torch, fh, dev)
        out["q4_k_gemv"] = run_kquant_gemv(args, torch, fh, dev, fh.Q4_K, "Q4_K")
        out["q5_k_gemv"] = run_kquant_gemv(args, torch, fh, dev, fh.Q5_K, "Q5_K")
        out["q6_k_gemv"] = run_kquant_gemv(args, torch, fh, dev, fh.Q6_K, "Q6_K")
        out["f32_path_gemv"] = run_f32path_gemv(args, torch, fh, dev)
        out["span_decode"] = run_span_decode(args, torch, fh, dev)
        out["moe_mixtral"] = run_moe(args, torch, fh, dev, "Mixtral-8x7B", 8, 2, 4096, 14336,
                                     (fh.Q4_K, fh.Q4_K, fh.Q4_K), (1, 64))
        out["moe_qwen3"] = run_moe(args, torch, fh, dev, "Qwen3-30B-A3B", 128, 8, 2048, 768,
                                   (fh.Q4_K, fh.Q4_K, fh.Q6_K), (1, 256))
        # measured HBM bytes over algorithmic bytes, where a counter pass covers these sources
        for key, sub, wl in (("q8_0_gemv", None, "q8_gemv"), ("q4_k_gemv", "gate_up", "q4k_gate_up"),
                             ("q4_k_gemv", "down", "q4k_down"), ("moe_mixtral", "M1", "moe_mixtral_m1"),
                             ("moe_mixtral", "M64", "moe_mixtral_m64"), ("moe_qwen3", "M1", "moe_qwen3_m1"),
                             ("moe_qwen3", "M256", "moe_qwen3_m256")):
            tr, why = measured_traffic(wl)
            dst = out[key] if sub is None or sub not in out[key] else out[key][sub]
            name = "traffic_over_algorithmic" if sub is None or sub in out[key] else f"{sub}_traffic_over_algorithmic"
            dst[name] = tr["traffic_over_algorithmic"] if tr else why
    if not args.no_prefill:
        if not args.no_extras:
            out["q5_k_prefill"] = run_q5k_prefill(args, torch, fh, dev)
        ops, layer_us, per, pcopies = run_prefill(args, torch, fh, dev)
        tops = ops / layer_us / 1e6
        proj_ops = {"qkv": 2 * 512 * 6144 * E, "o": 2 * 512 * E * E, "gate_up": 2 * 512 * 2 * F * E,
                    "down": 2 * 512 * E * F}
        out["prefill"] = {"workload": "Llama-3-8B layer projections, M=512 (q,k,v,o,gate,up Q4_K; down Q6_K) + "
                                      "activation quantization; q/k/v and gate/up as grouped launches",
                          "weight_copies": pcopies, "int_ops": ops, "us": round(layer_us, 2), "tops": round(tops, 2),
                          "pct_int8_peak": round(100 * tops / INT8_PEAK_TOPS, 2),
                          "parts_us": {k: round(v, 2) for k, v in per.items()},
                          "parts_tops": {k: round(proj_ops[k] / per[k] / 1e6, 1) for k in proj_ops}}
    if not args.no_cpu:
        out["cpu_baseline"] = run_cpu_baseline(args, step_bytes)
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
