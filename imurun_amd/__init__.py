"""MI355X (gfx950) quantized-matmul path of FISH, driven from Python.

The product is libfish_hip.so (C ABI in include/fish_hip.h); this module
binds it with ctypes the way IMURUN's model/fish_native.py binds libfish.so,
and adds thin helpers that pass torch device tensors as raw pointers. There
is no fallback: if the library or a gfx950 device is missing, calls raise.

Operator names follow FISH (model/fish/include/fish/ops.h, quant.h):
  quantize(x)                     ActBatch::quantize  (ops.cpp:158-175)
  repack(type, gguf, n_in, n_out) ComputeBackend::upload's device copy (backend.h:41-42)
  matmul(type, w, act, ...)       matmul_batch's int8 path (ops.cpp:177-216)
  matmul_batch(type, w, x, n_out) the convenience overload (ops.cpp:254-264)
  HipBackend                      ComputeBackend over host buffers (backend.h:26-163)
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfish_hip.so")

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 8, 12, 13, 14
# types FISH multiplies in f32 (no int8 kernel; kept as GGUF bytes on the device)
F32, F16, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, BF16, MXFP4 = 0, 1, 3, 6, 7, 10, 11, 20, 30, 39
F32_PATH_TYPES = (Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, MXFP4, F32, F16, BF16)
TYPE_NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", F32: "F32", F16: "F16",
              Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1", Q2_K: "Q2_K", Q3_K: "Q3_K", IQ4_NL: "IQ4_NL", BF16: "BF16",
              MXFP4: "MXFP4"}
BLOCK_ELEMS = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, F32: 1, F16: 1, BF16: 1, Q4_1: 32, Q5_0: 32,
               Q5_1: 32, Q2_K: 256, Q3_K: 256, IQ4_NL: 32, MXFP4: 32}
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, F32: 4, F16: 2, BF16: 2, Q4_1: 20, Q5_0: 22,
               Q5_1: 24, Q2_K: 84, Q3_K: 110, IQ4_NL: 18, MXFP4: 17}

_P = ctypes.c_void_p
_lib = None


class FishHipError(RuntimeError):
    pass


def gguf_row_bytes(t: int, n_in: int) -> int:
    return (n_in // BLOCK_ELEMS[t]) * BLOCK_BYTES[t]


def load() -> ctypes.CDLL:
    """The loaded libfish_hip.so with argument types set (raises if absent)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FishHipError(f"{LIB_PATH} is missing: run __graft_entry__.build() (hipcc --offload-arch=gfx950)")
    L = ctypes.CDLL(LIB_PATH)
    sig = {
        "fish_hip_abi_version": ([], ctypes.c_int),
        "fish_hip_kernel_name": ([], ctypes.c_char_p),
        "fish_hip_last_error": ([], ctypes.c_char_p),
        "fish_hip_weight_bytes": ([ctypes.c_uint32, ctypes.c_int, ctypes.c_int], ctypes.c_uint64),
        "fish_hip_act_bytes": ([ctypes.c_int, ctypes.c_int], ctypes.c_uint64),
        "fish_hip_quantize": ([_P, ctypes.c_int, ctypes.c_int, _P, _P, _P, _P], ctypes.c_int),
        "fish_hip_quantize_for": ([ctypes.c_uint32, _P, ctypes.c_int, ctypes.c_int, _P, _P], ctypes.c_int),
        "fish_hip_repack": ([ctypes.c_uint32, _P, ctypes.c_int, ctypes.c_int, _P, _P], ctypes.c_int),
        "fish_hip_matmul": ([ctypes.c_uint32, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P, _P], ctypes.c_int),
        "fish_hip_matmul_group": ([ctypes.c_uint32, ctypes.c_int, _P, _P, ctypes.c_int, ctypes.c_int, _P, _P, _P],
                                  ctypes.c_int),
        "fish_hip_matmul_tensors": ([ctypes.c_uint32, ctypes.c_int, _P, _P, ctypes.c_int, ctypes.c_int, _P, _P, _P,
                                     ctypes.c_uint64, _P], ctypes.c_int),
        "fish_hip_matmul_tensors_noalloc": ([ctypes.c_uint32, ctypes.c_int, _P, _P, ctypes.c_int, ctypes.c_int, _P,
                                             _P, _P], ctypes.c_int),
        "fish_hip_noalloc_scratch_bytes": ([], ctypes.c_uint64),
        "fish_hip_block_ints": ([ctypes.c_uint32, _P, _P, ctypes.c_int, ctypes.c_int, _P, _P], ctypes.c_int),
        "fish_hip_quantize_rows": ([ctypes.c_uint32, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int], ctypes.c_int),
        "fish_hip_moe_workspace_bytes": ([ctypes.c_int] * 5, ctypes.c_uint64),
        "fish_hip_moe_workspace_layout": ([ctypes.c_int] * 5 + [ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
        "fish_hip_moe_ffn": ([_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                              ctypes.c_int, ctypes.c_uint32, _P, ctypes.c_uint32, _P, ctypes.c_uint32, _P, _P,
                              ctypes.c_uint64, _P, _P], ctypes.c_int),
        "fish_hip_moe_route": ([_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P, ctypes.c_uint64, _P,
                                _P, _P], ctypes.c_int),
        "fish_hip_router_logits": ([_P, ctypes.c_int, ctypes.c_int, ctypes.c_uint32, _P, ctypes.c_int, _P, _P],
                                   ctypes.c_int),
        "fish_hip_silu_mul_quantize": ([_P, _P, ctypes.c_int, ctypes.c_int, _P, _P, _P, _P], ctypes.c_int),
        "fish_hip_backend_available": ([], ctypes.c_int),
        "fish_hip_device_name": ([], ctypes.c_char_p),
        "fish_hip_memory_total": ([], ctypes.c_uint64),
        "fish_hip_memory_free": ([], ctypes.c_uint64),
        "fish_hip_supports": ([ctypes.c_uint32], ctypes.c_int),
        "fish_hip_upload": ([_P, ctypes.c_uint32, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int], ctypes.c_int),
        "fish_hip_resident": ([_P], ctypes.c_int),
        "fish_hip_release": ([_P], None),
        "fish_hip_bytes_resident": ([], ctypes.c_uint64),
        "fish_hip_backend_served": ([], ctypes.c_uint64),
        "fish_hip_backend_matmul": ([_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P], ctypes.c_int),
        "fish_hip_backend_matmul_group": ([_P, ctypes.c_int, _P, ctypes.c_int, ctypes.c_int, _P, _P], ctypes.c_int),
        "fish_hip_backend_moe_ffn": ([_P, _P, _P, _P, _P, _P] + [ctypes.c_int] * 6 + [_P], ctypes.c_int),
        "fish_hip_span_prepare": ([_P], ctypes.c_int),
        "fish_hip_span_forward": ([_P, ctypes.c_int, ctypes.c_int], ctypes.c_int),
        "fish_hip_span_kv_truncate": ([ctypes.c_int], None),
        "fish_hip_span_inspect": ([ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P, ctypes.c_uint64],
                                  ctypes.c_int),
        "fish_hip_span_last_tokens": ([], ctypes.c_int),
        "fish_hip_span_release": ([], None),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def last_error() -> str:
    return (load().fish_hip_last_error() or b"").decode()


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise FishHipError(f"{what} failed ({rc}): {last_error()}")


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream or None
    return stream


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------------ block writer (host)

def quantize_rows(t: int, w: np.ndarray, n_threads: int | None = None) -> np.ndarray:
    """FISH's quantize_row over the rows of w (f32 [n_rows, n_in]) -> GGUF bytes."""
    w = np.ascontiguousarray(w, np.float32)
    n_rows, n_in = w.shape
    out = np.empty(gguf_row_bytes(t, n_in) * n_rows, np.uint8)
    threads = n_threads or min(16, os.cpu_count() or 1)
    _check(load().fish_hip_quantize_rows(t, w.ctypes.data, out.ctypes.data, n_rows, n_in, threads), "quantize_rows")
    return out


# ------------------------------------------------------------------ device operators (torch tensors)

def weight_bytes(t: int, n_in: int, n_out: int) -> int:
    return int(load().fish_hip_weight_bytes(t, n_in, n_out))


def act_bytes(n_tok: int, n_in: int) -> int:
    return int(load().fish_hip_act_bytes(n_tok, n_in))


def quantize(x, act=None, fish_layouts: bool = False, stream=None, for_type: int | None = None):
    """ActBatch::quantize on the device. x: f32 cuda [n_tok, n_in].
    Returns act (uint8 cuda) or (act, q32 bytes, q256 bytes) with FISH's layouts.
    for_type: only the planes the matmuls of that weight type read at n_tok tokens."""
    import torch
    assert x.is_cuda and x.dtype == torch.float32 and x.dim() == 2 and x.is_contiguous()
    n_tok, n_in = x.shape
    if act is None:
        act = torch.empty(act_bytes(n_tok, n_in), dtype=torch.uint8, device=x.device)
    if for_type is not None:
        if fish_layouts:
            raise FishHipError("quantize: for_type writes no FISH layouts")
        _check(load().fish_hip_quantize_for(for_type, x.data_ptr(), n_tok, n_in, act.data_ptr(), _stream(stream)),
               "quantize_for")
        return act
    q32 = q256 = None
    if fish_layouts:
        q32 = torch.empty(n_tok * (n_in // 32) * 40, dtype=torch.uint8, device=x.device)
        if n_in % 256 == 0:
            q256 = torch.empty(n_tok * (n_in // 256) * 276, dtype=torch.uint8, device=x.device)
    _check(load().fish_hip_quantize(x.data_ptr(), n_tok, n_in, act.data_ptr(), _ptr(q32), _ptr(q256),
                                    _stream(stream)), "quantize")
    return (act, q32, q256) if fish_layouts else act


def repack(t: int, gguf, n_in: int, n_out: int, stream=None):
    """GGUF rows (uint8 cuda tensor) -> repacked device tensor."""
    import torch
    assert gguf.is_cuda and gguf.dtype == torch.uint8
    if gguf.numel() < gguf_row_bytes(t, n_in) * n_out:
        raise FishHipError("repack: source smaller than n_out GGUF rows")
    nb = weight_bytes(t, n_in, n_out)
    if nb == 0:
        raise FishHipError(f"repack: type {t} with n_in={n_in} unsupported")
    w = torch.empty(nb, dtype=torch.uint8, device=gguf.device)
    _check(load().fish_hip_repack(t, gguf.data_ptr(), n_in, n_out, w.data_ptr(), _stream(stream)), "repack")
    return w


def matmul(t: int, w, act, n_tok: int, n_in: int, n_out: int, y=None, stream=None):
    """y[n_tok, n_out] = W . x on a repacked tensor and a quantized activation buffer."""
    import torch
    if w.numel() < weight_bytes(t, n_in, n_out) or act.numel() < act_bytes(n_tok, n_in):
        raise FishHipError("matmul: buffer smaller than its layout")
    if y is None:
        y = torch.empty((n_tok, n_out), dtype=torch.float32, device=w.device)
    assert y.numel() >= n_tok * n_out and y.is_contiguous()
    _check(load().fish_hip_matmul(t, w.data_ptr(), act.data_ptr(), n_tok, n_in, n_out, y.data_ptr(),
                                  _stream(stream)), "matmul")
    return y


def matmul_group(t: int, ws, act, n_tok: int, n_in: int, n_outs, ys=None, stream=None):
    """Several repacked tensors of one type applied to the same activations (matmul_tensors)."""
    import torch
    n = len(ws)
    if n != len(n_outs) or not 1 <= n <= 4:
        raise FishHipError("matmul_group: 1..4 tensors with one n_out each")
    for w, n_out in zip(ws, n_outs):
        if w.numel() < weight_bytes(t, n_in, n_out):
            raise FishHipError("matmul_group: weight buffer smaller than its layout")
    if act.numel() < act_bytes(n_tok, n_in):
        raise FishHipError("matmul_group: activation buffer smaller than its layout")
    if ys is None:
        ys = [torch.empty((n_tok, n_out), dtype=torch.float32, device=ws[0].device) for n_out in n_outs]
    for y, n_out in zip(ys, n_outs):
        assert y.numel() >= n_tok * n_out and y.is_contiguous()
    wp = (ctypes.c_void_p * n)(*[w.data_ptr() for w in ws])
    yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
    no = (ctypes.c_int * n)(*n_outs)
    _check(load().fish_hip_matmul_group(t, n, wp, act.data_ptr(), n_tok, n_in, no, yp, _stream(stream)),
           "matmul_group")
    return ys


def matmul_tensors(t: int, ws, x, n_outs, ys=None, act=None, stream=None):
    """f32 x [n_tok, n_in] quantized and multiplied by 1..4 tensors (matmul_tensors / the
    convenience matmul_batch); one token runs as one fused launch without a workspace.
    Types FISH multiplies in f32 (F32_PATH_TYPES) take x as it is."""
    import torch
    assert x.is_cuda and x.dtype == torch.float32 and x.dim() == 2 and x.is_contiguous()
    n_tok, n_in = x.shape
    n = len(ws)
    if n != len(n_outs) or not 1 <= n <= 4:
        raise FishHipError("matmul_tensors: 1..4 tensors with one n_out each")
    for w, n_out in zip(ws, n_outs):
        if w.numel() < weight_bytes(t, n_in, n_out):
            raise FishHipError("matmul_tensors: weight buffer smaller than its layout")
    if ys is None:
        ys = [torch.empty((n_tok, n_out), dtype=torch.float32, device=x.device) for n_out in n_outs]
    for y, n_out in zip(ys, n_outs):
        assert y.numel() >= n_tok * n_out and y.is_contiguous()
    if act is None and n_tok > 1 and t not in F32_PATH_TYPES:
        act = torch.empty(act_bytes(n_tok, n_in), dtype=torch.uint8, device=x.device)
    wp = (ctypes.c_void_p * n)(*[w.data_ptr() for w in ws])
    yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
    no = (ctypes.c_int * n)(*n_outs)
    _check(load().fish_hip_matmul_tensors(t, n, wp, x.data_ptr(), n_tok, n_in, no, yp, _ptr(act),
                                          act.numel() if act is not None else 0, _stream(stream)), "matmul_tensors")
    return ys


def matmul_tensors_noalloc(t: int, ws, x, n_outs, ys, stream=None):
    """matmul_tensors with the activation workspace in the library's fixed device array
    (fish_hip_matmul_tensors_noalloc): the call allocates nothing; ys must be given."""
    import torch
    assert x.is_cuda and x.dtype == torch.float32 and x.dim() == 2 and x.is_contiguous()
    n_tok, n_in = x.shape
    n = len(ws)
    if n != len(n_outs) or n != len(ys) or not 1 <= n <= 4:
        raise FishHipError("matmul_tensors_noalloc: 1..4 tensors with one n_out and one y each")
    for w, y, n_out in zip(ws, ys, n_outs):
        if w.numel() < weight_bytes(t, n_in, n_out):
            raise FishHipError("matmul_tensors_noalloc: weight buffer smaller than its layout")
        assert y.numel() >= n_tok * n_out and y.is_contiguous()
    wp = (ctypes.c_void_p * n)(*[w.data_ptr() for w in ws])
    yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
    no = (ctypes.c_int * n)(*n_outs)
    _check(load().fish_hip_matmul_tensors_noalloc(t, n, wp, x.data_ptr(), n_tok, n_in, no, yp, _stream(stream)),
           "matmul_tensors_noalloc")
    return ys


def noalloc_scratch_bytes() -> int:
    return int(load().fish_hip_noalloc_scratch_bytes())


def matmul_batch(t: int, w, x, n_out: int, stream=None):
    """Quantize x then multiply (the convenience matmul_batch, ops.cpp:254-264)."""
    act = quantize(x, stream=stream)
    return matmul(t, w, act, x.shape[0], x.shape[1], n_out, stream=stream)


def block_ints(t: int, w, act, n_in: int, n_out: int, stream=None):
    """Per-block integer dots of every row with token 0 (int32 cuda tensor)."""
    import torch
    per_row = (2 * (n_in // 256)) if t in (Q4_K, Q5_K) else ((n_in // 256) if t == Q6_K else n_in // 32)
    out = torch.empty(n_out * per_row, dtype=torch.int32, device=w.device)
    _check(load().fish_hip_block_ints(t, w.data_ptr(), act.data_ptr(), n_in, n_out, out.data_ptr(),
                                      _stream(stream)), "block_ints")
    return out


# ------------------------------------------------------------------ expert FFN (torch tensors)

def moe_workspace_bytes(n_tok: int, n_embd: int, n_ff: int, n_expert: int, k: int) -> int:
    return int(load().fish_hip_moe_workspace_bytes(n_tok, n_embd, n_ff, n_expert, k))


def moe_ffn(x, logits, n_ff: int, n_expert: int, k: int, norm: bool, tg: int, wg, tu: int, wu, td: int, wd,
            out=None, workspace=None, stream=None):
    """LlamaModel::moe_ffn with given router logits; weights repacked (n_expert * rows)."""
    import torch
    n_tok, n_embd = x.shape
    nb = moe_workspace_bytes(n_tok, n_embd, n_ff, n_expert, k)
    if nb == 0:
        raise FishHipError("moe_ffn: unsupported sizes")
    if workspace is None:
        workspace = torch.empty(nb, dtype=torch.uint8, device=x.device)
    if out is None:
        out = torch.empty((n_tok, n_embd), dtype=torch.float32, device=x.device)
    _check(load().fish_hip_moe_ffn(x.data_ptr(), logits.data_ptr(), n_tok, n_embd, n_ff, n_expert, k, int(norm), tg,
                                   wg.data_ptr(), tu, wu.data_ptr(), td, wd.data_ptr(), workspace.data_ptr(),
                                   workspace.numel(), out.data_ptr(), _stream(stream)), "moe_ffn")
    return out


MOE_PARTS = ("sel", "wsel", "tok_slot", "slot_tok", "gate", "up", "down")


def moe_parts(workspace, n_tok: int, n_embd: int, n_ff: int, n_expert: int, k: int) -> dict:
    """Views of the intermediate buffers a moe_ffn call left in `workspace`."""
    import torch
    offs = (ctypes.c_uint64 * len(MOE_PARTS))()
    _check(load().fish_hip_moe_workspace_layout(n_tok, n_embd, n_ff, n_expert, k, offs), "moe_workspace_layout")
    slots = n_tok * k
    shapes = {"sel": ((n_tok, k), torch.int32), "wsel": ((n_tok, k), torch.float32),
              "tok_slot": ((n_tok, k), torch.int32), "slot_tok": ((slots,), torch.int32),
              "gate": ((slots, n_ff), torch.float32), "up": ((slots, n_ff), torch.float32),
              "down": ((slots, n_embd), torch.float32)}
    out = {}
    for name, off in zip(MOE_PARTS, offs):
        shape, dt = shapes[name]
        n = int(np.prod(shape)) * 4
        out[name] = workspace[int(off):int(off) + n].view(dt).view(shape)
    return out


def moe_route(logits, k: int, norm: bool = True, stream=None):
    import torch
    n_tok, n_expert = logits.shape
    ws = torch.empty(moe_workspace_bytes(n_tok, 32, 32, n_expert, k), dtype=torch.uint8, device=logits.device)
    sel = torch.empty((n_tok, k), dtype=torch.int32, device=logits.device)
    wsel = torch.empty((n_tok, k), dtype=torch.float32, device=logits.device)
    _check(load().fish_hip_moe_route(logits.data_ptr(), n_tok, n_expert, k, int(norm), ws.data_ptr(), ws.numel(),
                                     sel.data_ptr(), wsel.data_ptr(), _stream(stream)), "moe_route")
    return sel, wsel


def router_logits(x, w, out=None, stream=None):
    """logits [n_tok][n_expert] = x @ w.T in f32 for f32 or f16 router rows w
    [n_expert][n_embd] (model.cpp:1529); written into `out` when given."""
    import torch
    if w.dtype not in (torch.float32, torch.float16):
        raise ValueError("router_logits: weights must be float32 or float16")
    n_tok, n_embd = x.shape
    n_expert = w.shape[0]
    if w.shape[1] != n_embd or x.dtype != torch.float32 or not x.is_contiguous() or not w.is_contiguous():
        raise ValueError("router_logits: x f32 [n_tok][n_embd], w [n_expert][n_embd], both contiguous")
    logits = torch.empty((n_tok, n_expert), dtype=torch.float32, device=x.device) if out is None else out
    if logits.shape != (n_tok, n_expert) or logits.dtype != torch.float32 or not logits.is_contiguous():
        raise ValueError("router_logits: out must be contiguous f32 [n_tok][n_expert]")
    t = 0 if w.dtype == torch.float32 else 1
    _check(load().fish_hip_router_logits(x.data_ptr(), n_tok, n_embd, t, w.data_ptr(), n_expert, logits.data_ptr(),
                                         _stream(stream)), "router_logits")
    return logits


def silu_mul_quantize(g, u, stream=None):
    """(act, FISH Q8ActK bytes or None, h) for h = silu(g) * u."""
    import torch
    n_rows, n_ff = g.shape
    act = torch.empty(act_bytes(n_rows, n_ff), dtype=torch.uint8, device=g.device)
    q256 = torch.empty(n_rows * (n_ff // 256) * 276, dtype=torch.uint8, device=g.device) if n_ff % 256 == 0 else None
    h = torch.empty((n_rows, n_ff), dtype=torch.float32, device=g.device)
    _check(load().fish_hip_silu_mul_quantize(g.data_ptr(), u.data_ptr(), n_rows, n_ff, act.data_ptr(), _ptr(q256),
                                             h.data_ptr(), _stream(stream)), "silu_mul_quantize")
    return act, q256, h


# ------------------------------------------------------------------ backend (host buffers)

SPAN_VECS = ("q_norm", "k_norm", "bias_q", "bias_k", "bias_v", "bias_o")
SPAN_VECS2 = ("bias_qkv", "post_attn_norm", "post_ffn_norm")  # after the wqkv key


class SpanLayer(ctypes.Structure):
    """fish_hip_span_layer (include/fish_hip.h)."""
    _fields_ = [(n, ctypes.c_void_p) for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")] + \
               [("attn_norm", ctypes.c_void_p), ("ffn_norm", ctypes.c_void_p)] + \
               [(n, ctypes.c_void_p) for n in SPAN_VECS] + [("wqkv", ctypes.c_void_p)] + \
               [(n, ctypes.c_void_p) for n in SPAN_VECS2] + [("sliding_window", ctypes.c_int)]


class SpanParams(ctypes.Structure):
    """fish_hip_span_params (include/fish_hip.h)."""
    _fields_ = [("n_layers", ctypes.c_int), ("n_embd", ctypes.c_int), ("n_head", ctypes.c_int),
                ("n_head_kv", ctypes.c_int), ("head_dim", ctypes.c_int), ("n_ff", ctypes.c_int),
                ("n_ctx", ctypes.c_int), ("eps", ctypes.c_float), ("attn_scale", ctypes.c_float),
                ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p), ("rot_dim", ctypes.c_int),
                ("rope_neox", ctypes.c_int), ("layers", ctypes.c_void_p), ("kv_q8", ctypes.c_int),
                ("attn_softcap", ctypes.c_float), ("window", ctypes.c_int), ("gelu", ctypes.c_int)]


class HipBackend:
    """ComputeBackend over host numpy buffers (backend.h:26-163).

    Tensors are named by strings; each name maps to one key pointer for the life of
    the process (shared by every instance), so a name always addresses the same
    resident tensor and no key address is ever reused for another name."""

    _keys: dict[str, ctypes.c_void_p] = {}
    _anchors: list = []

    def __init__(self):
        self.L = load()

    def available(self) -> bool:
        return bool(self.L.fish_hip_backend_available())

    def name(self) -> str:
        return "hip"

    def device_name(self) -> str:
        return (self.L.fish_hip_device_name() or b"").decode()

    def memory_total(self) -> int:
        return int(self.L.fish_hip_memory_total())

    def memory_free(self) -> int:
        return int(self.L.fish_hip_memory_free())

    def supports(self, t: int) -> bool:
        return bool(self.L.fish_hip_supports(t))

    def _key(self, name: str) -> ctypes.c_void_p:
        if name not in self._keys:
            buf = ctypes.create_string_buffer(1)
            self._anchors.append(buf)
            self._keys[name] = ctypes.cast(buf, ctypes.c_void_p)
        return self._keys[name]

    def upload(self, name: str, t: int, data: np.ndarray, n_in: int, n_out: int, n_expert: int = 1) -> bool:
        data = np.ascontiguousarray(data, dtype=np.uint8)
        if data.size < gguf_row_bytes(t, n_in) * n_out * n_expert:
            return False
        return bool(self.L.fish_hip_upload(self._key(name), t, data.ctypes.data, n_in, n_out, n_expert))

    def resident(self, name: str) -> bool:
        return name in self._keys and bool(self.L.fish_hip_resident(self._keys[name]))

    def release(self, name: str) -> None:
        if name in self._keys:
            self.L.fish_hip_release(self._keys[name])

    def bytes_resident(self) -> int:
        return int(self.L.fish_hip_bytes_resident())

    def matmul(self, name: str, x: np.ndarray, n_out: int):
        """y[n_tok, n_out] or None when the device call failed (caller uses the CPU)."""
        x = np.ascontiguousarray(x, np.float32)
        n_tok, n_in = x.shape
        y = np.empty((n_tok, n_out), np.float32)
        ok = self.L.fish_hip_backend_matmul(self._key(name), x.ctypes.data, n_tok, n_in, n_out, y.ctypes.data)
        return y if ok else None

    def span_prepare(self, layers, n_embd, n_head, n_head_kv, head_dim, n_ff, n_ctx, rope_cos, rope_sin,
                     rope_neox=False, eps=1e-5, attn_scale=0.0, kv_q8=False, attn_softcap=0.0, window=0,
                     gelu=False) -> bool:
        """ComputeBackend::span_prepare over uploaded tensors: layers = [(names of
        wq, wk, wv, wo, wg, wu, wd), attn_norm, ffn_norm] or [(names, attn_norm, ffn_norm,
        extras)] with extras a dict of the optional SPAN_VECS / SPAN_VECS2 vectors (Qwen-3 q/k
        norms, biases, Gemma-2 post norms), "wqkv" (the fused q|k|v tensor's name, with wq, wk,
        wv None) and "sliding_window"; a None wg makes wu the fused gate|up. RoPE tables
        [n_ctx][rot_dim / 2]."""
        arr = (SpanLayer * len(layers))()
        keep = []

        def vec(v):
            if v is None:
                return None
            v = np.ascontiguousarray(v, np.float32)
            keep.append(v)
            return v.ctypes.data

        for i, layer in enumerate(layers):
            names, an, fn = layer[:3]
            extras = layer[3] if len(layer) > 3 else {}
            keys = [self._key(n).value if n is not None else None for n in names]
            wqkv = self._key(extras["wqkv"]).value if extras.get("wqkv") else None
            arr[i] = SpanLayer(*keys, vec(an), vec(fn), *[vec(extras.get(n)) for n in SPAN_VECS], wqkv,
                               *[vec(extras.get(n)) for n in SPAN_VECS2], 1 if extras.get("sliding_window") else 0)
        rc = np.ascontiguousarray(rope_cos, np.float32)
        rs = np.ascontiguousarray(rope_sin, np.float32)
        p = SpanParams(len(layers), n_embd, n_head, n_head_kv, head_dim, n_ff, n_ctx, eps, attn_scale,
                       rc.ctypes.data, rs.ctypes.data, 2 * rc.shape[1], 1 if rope_neox else 0,
                       ctypes.cast(arr, ctypes.c_void_p), 1 if kv_q8 else 0, attn_softcap, window,
                       1 if gelu else 0)
        return bool(self.L.fish_hip_span_prepare(ctypes.byref(p)))

    def span_kv_truncate(self, n_past: int) -> None:
        self.L.fish_hip_span_kv_truncate(n_past)

    SPAN_PARTS = ("x", "xb", "q", "k", "v", "qr", "att", "proj", "xb2", "h", "u", "dn")

    def span_inspect(self, part: str, width: int, layer: int = 0, pos0: int = 0, n: int = 0):
        """An intermediate buffer of the last span_forward call, [tokens][width] f32; part "kc" /
        "vc" returns cache rows pos0 .. pos0 + n - 1 of `layer` ([n][width], width = kv_dim)."""
        if part in ("kc", "vc"):
            out = np.empty((n, width), np.float32)
            ok = self.L.fish_hip_span_inspect(100 if part == "kc" else 101, layer, pos0, n, out.ctypes.data, out.size)
        else:
            t = int(self.L.fish_hip_span_last_tokens())
            out = np.empty((t, width), np.float32)
            ok = t > 0 and self.L.fish_hip_span_inspect(self.SPAN_PARTS.index(part), 0, 0, 0, out.ctypes.data,
                                                        out.size)
        if not ok:
            raise FishHipError(f"span_inspect({part}) refused")
        return out

    def moe_ffn(self, names, x: np.ndarray, logits, n_ff: int, n_expert: int, k: int, norm: bool = True,
                router: str | None = None):
        """fish_hip_backend_moe_ffn over uploaded 3-D expert tensors (gate, up, down names) on host
        buffers; `logits` [n_tok][n_expert] or None with a resident router tensor. out or None."""
        x = np.ascontiguousarray(x, np.float32)
        n_tok, n_embd = x.shape
        lg = None if logits is None else np.ascontiguousarray(logits, np.float32)
        out = np.empty((n_tok, n_embd), np.float32)
        keys = [self._key(n).value for n in names]
        kr = self._key(router).value if router else None
        ok = self.L.fish_hip_backend_moe_ffn(keys[0], keys[1], keys[2], kr, x.ctypes.data,
                                             None if lg is None else lg.ctypes.data, n_tok, n_embd, n_ff, n_expert, k,
                                             int(norm), out.ctypes.data)
        return out if ok else None

    def span_forward(self, x: np.ndarray, pos0: int) -> bool:
        """ComputeBackend::span_forward: x [n_tok, n_embd] float32, updated in place."""
        assert x.dtype == np.float32 and x.flags.c_contiguous
        return bool(self.L.fish_hip_span_forward(x.ctypes.data, x.shape[0], pos0))

    def span_release(self) -> None:
        self.L.fish_hip_span_release()

    def matmul_group(self, names, x: np.ndarray, n_outs):
        x = np.ascontiguousarray(x, np.float32)
        n_tok, n_in = x.shape
        ys = [np.empty((n_tok, n), np.float32) for n in n_outs]
        keys = (ctypes.c_void_p * len(names))(*[self._key(n).value for n in names])
        outs = (ctypes.c_int * len(names))(*n_outs)
        yp = (ctypes.c_void_p * len(names))(*[y.ctypes.data for y in ys])
        ok = self.L.fish_hip_backend_matmul_group(keys, len(names), x.ctypes.data, n_tok, n_in, outs, yp)
        return ys if ok else None
