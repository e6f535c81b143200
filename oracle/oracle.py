"""ctypes bindings of the checker libraries -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product path (imurun_amd) never does.

  Oracle  -> oracle/liboracle.so, the C restatement of FISH's CPU path
  Ref     -> oracle/_ref/libfishref.so, the reference's own CPU path compiled
             from its sources (None when it was not built)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libfishref.so")

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 8, 12, 13, 14
# weight types FISH multiplies on its f32 path (no int8 kernel). IQ4_XS has a
# dequantiser (quant.cpp:299-316) but no entry in FISH's type-size table
# (gguf.cpp:216-241), so matmul_batch cannot address its rows: not listed.
F32, F16, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, IQ4_XS, BF16, MXFP4 = 0, 1, 3, 6, 7, 10, 11, 20, 23, 30, 39
F32_PATH_TYPES = [Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, MXFP4, F32, F16, BF16]
BLOCK_ELEMS = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q4_1: 32, Q5_0: 32, Q5_1: 32, Q2_K: 256,
               Q3_K: 256, IQ4_NL: 32, IQ4_XS: 256, MXFP4: 32, F32: 1, F16: 1, BF16: 1}
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q2_K: 84,
               Q3_K: 110, IQ4_NL: 18, IQ4_XS: 136, MXFP4: 17, F32: 4, F16: 2, BF16: 2}
ACT32, ACT256 = 40, 276

_P = ctypes.c_void_p
_F = ctypes.POINTER(ctypes.c_float)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def row_bytes(t: int, n: int) -> int:
    return (n // BLOCK_ELEMS[t]) * BLOCK_BYTES[t]


def uses_k_layout(t: int) -> bool:
    return BLOCK_ELEMS[t] == 256


def build(quiet: bool = True) -> None:
    """Compile liboracle.so (and _ref when the reference sources exist)."""
    out = subprocess.run(["make", "-C", HERE, "all"], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + out.stdout + out.stderr)
    if not quiet:
        print(out.stdout)


class Oracle:
    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        self.L = L
        L.or_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.or_fp16_to_fp32.restype = ctypes.c_float
        L.or_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.or_fp32_to_fp16.restype = ctypes.c_uint16
        L.or_quantize_acts.argtypes = [_P, ctypes.c_uint64, _P]
        L.or_quantize_acts_k.argtypes = [_P, ctypes.c_uint64, _P]
        L.or_dequant_row.argtypes = [ctypes.c_uint32, _P, _P, ctypes.c_uint64]
        L.or_block_dots.argtypes = [ctypes.c_uint32, _P, _P, ctypes.c_uint64, _P]
        L.or_block_dots.restype = ctypes.c_int64
        L.or_vec_dot_q8.argtypes = [ctypes.c_uint32, _P, _P, ctypes.c_uint64]
        L.or_vec_dot_q8.restype = ctypes.c_float
        L.or_matmul_batch.argtypes = [ctypes.c_uint32, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P, ctypes.c_int]
        L.or_act_batch.argtypes = [_P, ctypes.c_int, ctypes.c_int, _P, _P]
        L.or_quantize_row.argtypes = [ctypes.c_uint32, _P, _P, ctypes.c_uint64]
        L.or_quantize_rows.argtypes = [ctypes.c_uint32, _P, _P, ctypes.c_int64, ctypes.c_uint64, ctypes.c_int]
        L.or_route.argtypes = [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P, _P]
        L.or_silu.argtypes = [ctypes.c_float]
        L.or_silu.restype = ctypes.c_float
        L.or_silu_mul.argtypes = [_P, _P, ctypes.c_uint64, _P]
        L.or_moe_ffn.argtypes = [_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_uint32, _P, ctypes.c_uint32, _P, ctypes.c_uint32, _P, _P,
                                 ctypes.c_int]
        L.or_router_logits.argtypes = [ctypes.c_uint32, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]
        L.or_matmul_f32path.argtypes = [ctypes.c_uint32, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]
        self.threads = min(16, os.cpu_count() or 1)

    # activations -----------------------------------------------------------
    def quantize_acts(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        n = x.size
        out = np.zeros(n // 32 * ACT32, np.uint8)
        self.L.or_quantize_acts(_ptr(x), n, _ptr(out))
        return out

    def quantize_acts_k(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        n = x.size
        out = np.zeros(n // 256 * ACT256, np.uint8)
        self.L.or_quantize_acts_k(_ptr(x), n, _ptr(out))
        return out

    def act_batch(self, x: np.ndarray):
        """ActBatch::quantize: (q32 bytes, q256 bytes or None) for x[n_tok][n_in]."""
        x = np.ascontiguousarray(x, np.float32)
        n_tok, n_in = x.shape
        q32 = np.zeros(n_tok * (n_in // 32) * ACT32, np.uint8)
        q256 = np.zeros(n_tok * (n_in // 256) * ACT256, np.uint8) if n_in % 256 == 0 else None
        self.L.or_act_batch(_ptr(x), n_tok, n_in, _ptr(q32), _ptr(q256) if q256 is not None else None)
        return q32, q256

    # weights ---------------------------------------------------------------
    def quantize_rows(self, t: int, w: np.ndarray) -> np.ndarray:
        w = np.ascontiguousarray(w, np.float32)
        n_rows, n_in = w.shape
        out = np.zeros(n_rows * row_bytes(t, n_in), np.uint8)
        if not self.L.or_quantize_rows(t, _ptr(w), _ptr(out), n_rows, n_in, self.threads):
            raise ValueError("bad type/shape")
        return out

    def dequant_row(self, t: int, row: np.ndarray, n: int) -> np.ndarray:
        out = np.zeros(n, np.float32)
        if not self.L.or_dequant_row(t, _ptr(np.ascontiguousarray(row)), _ptr(out), n):
            raise ValueError("bad type/shape")
        return out

    def block_dots(self, t: int, row: np.ndarray, acts: np.ndarray, n: int) -> np.ndarray:
        per = 2 if t in (Q4_K, Q5_K) else 1
        out = np.zeros((n // BLOCK_ELEMS[t]) * per, np.int32)
        k = self.L.or_block_dots(t, _ptr(np.ascontiguousarray(row)), _ptr(np.ascontiguousarray(acts)), n, _ptr(out))
        assert k == out.size
        return out

    def vec_dot(self, t: int, row: np.ndarray, acts: np.ndarray, n: int) -> float:
        return self.L.or_vec_dot_q8(t, _ptr(np.ascontiguousarray(row)), _ptr(np.ascontiguousarray(acts)), n)

    def matmul(self, t: int, w: np.ndarray, q32, q256, n_tok: int, n_in: int, n_out: int) -> np.ndarray:
        y = np.zeros((n_tok, n_out), np.float32)
        ok = self.L.or_matmul_batch(t, _ptr(w), _ptr(q32) if q32 is not None else None,
                                    _ptr(q256) if q256 is not None else None, n_tok, n_in, n_out, _ptr(y),
                                    self.threads)
        if not ok:
            raise ValueError("bad matmul arguments")
        return y

    def matmul_f32(self, t: int, w: np.ndarray, x: np.ndarray, n_out: int) -> np.ndarray:
        q32, q256 = self.act_batch(x)
        return self.matmul(t, w, q32, q256, x.shape[0], x.shape[1], n_out)

    # MoE ---------------------------------------------------------------------
    def route(self, logits: np.ndarray, k: int, norm: bool = True):
        logits = np.ascontiguousarray(logits, np.float32)
        n_tok, ne = logits.shape
        sel = np.zeros((n_tok, k), np.int32)
        wsel = np.zeros((n_tok, k), np.float32)
        self.L.or_route(_ptr(logits), n_tok, ne, k, int(norm), _ptr(sel), _ptr(wsel))
        return sel, wsel

    def router_logits(self, t: int, w: np.ndarray, x: np.ndarray) -> np.ndarray:
        """matmul_batch on f32 (t=0) or f16 (t=1, w as uint16 bits) router rows
        w [n_expert][n_embd] (ops.cpp:219-250)."""
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32 if t == 0 else np.uint16)
        n_tok, n_embd = x.shape
        out = np.zeros((n_tok, w.shape[0]), np.float32)
        if not self.L.or_router_logits(t, _ptr(w), _ptr(x), n_tok, n_embd, w.shape[0], _ptr(out)):
            raise ValueError("bad router arguments")
        return out

    def matmul_f32path(self, t: int, w: np.ndarray, x: np.ndarray, n_out: int) -> np.ndarray:
        """matmul_batch on a type without an int8 kernel: y [n_tok][n_out] (ops.cpp:219-250)."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros((x.shape[0], n_out), np.float32)
        if not self.L.or_matmul_f32path(t, _ptr(np.ascontiguousarray(w)), _ptr(x), x.shape[0], x.shape[1], n_out,
                                        _ptr(y)):
            raise ValueError("bad f32-path arguments")
        return y

    def silu(self, v: float) -> float:
        return self.L.or_silu(v)

    def silu_mul(self, g: np.ndarray, u: np.ndarray) -> np.ndarray:
        """h = silu(g) * u in FISH's f32 steps (ops.cpp:25-30, model.cpp:1504-1508)."""
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        assert g.shape == u.shape
        h = np.empty_like(g)
        self.L.or_silu_mul(_ptr(g), _ptr(u), g.size, _ptr(h))
        return h

    def moe_ffn(self, x, logits, E, F, NE, K, norm, tg, wg, tu, wu, td, wd) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        logits = np.ascontiguousarray(logits, np.float32)
        n_tok = x.shape[0]
        out = np.zeros((n_tok, E), np.float32)
        self.L.or_moe_ffn(_ptr(x), _ptr(logits), n_tok, E, F, NE, K, int(norm), tg, _ptr(wg), tu, _ptr(wu), td,
                          _ptr(wd), _ptr(out), self.threads)
        return out


class Ref:
    """The reference's compiled CPU path (FISH's installed kernel table)."""

    def __init__(self, path: str = REF_SO):
        L = ctypes.CDLL(path)
        self.L = L
        L.ref_kernel_name.restype = ctypes.c_char_p
        L.ref_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.ref_fp16_to_fp32.restype = ctypes.c_float
        L.ref_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.ref_fp32_to_fp16.restype = ctypes.c_uint16
        L.ref_quantize_acts.argtypes = [_P, ctypes.c_uint64, _P, ctypes.c_int]
        L.ref_quantize_acts_k.argtypes = [_P, ctypes.c_uint64, _P, ctypes.c_int]
        L.ref_dequant_row.argtypes = [ctypes.c_uint32, _P, _P, ctypes.c_uint64]
        L.ref_quantize_row.argtypes = [ctypes.c_uint32, _P, _P, ctypes.c_uint64]
        L.ref_vec_dot_q8.argtypes = [ctypes.c_uint32, _P, _P, ctypes.c_uint64, ctypes.c_int]
        L.ref_vec_dot_q8.restype = ctypes.c_float
        L.ref_matmul_f32.argtypes = [ctypes.c_uint32, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]
        L.ref_matmul_acts.argtypes = [ctypes.c_uint32, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]
        L.ref_moe_ffn.argtypes = [_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_int, ctypes.c_uint32, _P, ctypes.c_uint32, _P, ctypes.c_uint32, _P, _P, _P,
                                  _P]

    @staticmethod
    def available() -> bool:
        return os.path.exists(REF_SO)

    def kernel_name(self) -> str:
        return self.L.ref_kernel_name().decode()

    def threads(self) -> int:
        return self.L.ref_threads()

    def quantize_acts(self, x, scalar=False):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(x.size // 32 * ACT32, np.uint8)
        self.L.ref_quantize_acts(_ptr(x), x.size, _ptr(out), int(scalar))
        return out

    def quantize_acts_k(self, x, scalar=False):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(x.size // 256 * ACT256, np.uint8)
        self.L.ref_quantize_acts_k(_ptr(x), x.size, _ptr(out), int(scalar))
        return out

    def quantize_row(self, t, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(row_bytes(t, x.size), np.uint8)
        assert self.L.ref_quantize_row(t, _ptr(x), _ptr(out), x.size)
        return out

    def dequant_row(self, t, row, n):
        out = np.zeros(n, np.float32)
        assert self.L.ref_dequant_row(t, _ptr(np.ascontiguousarray(row)), _ptr(out), n)
        return out

    def vec_dot(self, t, row, acts, n, scalar=False):
        return self.L.ref_vec_dot_q8(t, _ptr(np.ascontiguousarray(row)), _ptr(np.ascontiguousarray(acts)), n,
                                     int(scalar))

    def matmul_f32(self, t, w, x, n_out):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros((x.shape[0], n_out), np.float32)
        self.L.ref_matmul_f32(t, _ptr(w), _ptr(x), x.shape[0], x.shape[1], n_out, _ptr(y))
        return y

    def matmul_acts(self, t, w, q32, q256, n_tok, n_in, n_out):
        y = np.zeros((n_tok, n_out), np.float32)
        self.L.ref_matmul_acts(t, _ptr(w), _ptr(q32), _ptr(q256) if q256 is not None else None, n_tok, n_in, n_out,
                               _ptr(y))
        return y

    def moe_ffn(self, x, logits, E, F, NE, K, norm, tg, wg, tu, wu, td, wd):
        x = np.ascontiguousarray(x, np.float32)
        logits = np.ascontiguousarray(logits, np.float32)
        n_tok = x.shape[0]
        out = np.zeros((n_tok, E), np.float32)
        sel = np.zeros((n_tok, K), np.int32)
        wsel = np.zeros((n_tok, K), np.float32)
        self.L.ref_moe_ffn(_ptr(x), _ptr(logits), n_tok, E, F, NE, K, int(norm), tg, _ptr(wg), tu, _ptr(wu), td,
                           _ptr(wd), _ptr(out), _ptr(sel), _ptr(wsel))
        return out, sel, wsel


DROPIN_SO = os.path.join(HERE, "_ref", "libfishref_hip.so")


class DropIn:
    """FISH's own routing (ops.cpp:283-299) with the HIP backend binding
    registered, from _ref/libfishref_hip.so. Weight bytes stay owned by the
    caller (numpy arrays kept alive in self._keep)."""

    @staticmethod
    def available() -> bool:
        return os.path.exists(DROPIN_SO)

    def __init__(self, path: str = DROPIN_SO):
        L = ctypes.CDLL(path)
        self.L = L
        L.drop_backend_name.restype = ctypes.c_char_p
        L.drop_tensor_new.restype = _P
        L.drop_tensor_new.argtypes = [ctypes.c_uint32, _P, ctypes.c_int, ctypes.c_int]
        L.drop_tensor3_new.restype = _P
        L.drop_tensor3_new.argtypes = [ctypes.c_uint32, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.drop_moe_ffn.argtypes = [_P, _P, _P, _P, _P] + [ctypes.c_int] * 6 + [_P]
        for f in ("drop_tensor_free", "drop_upload", "drop_resident", "drop_release"):
            getattr(L, f).argtypes = [_P]
        L.drop_bytes_resident.restype = ctypes.c_uint64
        mm = [_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]
        L.drop_matmul_tensor.argtypes = mm
        L.drop_matmul_cpu.argtypes = mm
        L.drop_matmul_tensors.argtypes = [_P, ctypes.c_int, _P, ctypes.c_int, ctypes.c_int, _P, _P]
        self._keep = {}

    def backend_name(self) -> str:
        return self.L.drop_backend_name().decode()

    def tensor(self, t: int, packed: np.ndarray, n_in: int, n_out: int):
        packed = np.ascontiguousarray(packed)
        h = self.L.drop_tensor_new(t, _ptr(packed), n_in, n_out)
        self._keep[h] = (packed, n_in, n_out)
        return h

    def tensor3(self, t: int, packed: np.ndarray, n_in: int, n_out: int, n_expert: int):
        """A 3-D expert TensorInfo [n_expert][n_out][n_in] over the packed bytes."""
        packed = np.ascontiguousarray(packed)
        h = self.L.drop_tensor3_new(t, _ptr(packed), n_in, n_out, n_expert)
        self._keep[h] = (packed, n_in, n_out)
        return h

    def moe_ffn(self, hs, x, logits, n_ff: int, n_expert: int, k: int, norm: bool = True):
        """The expert hook called with FISH's TensorInfo keys (out, or None when refused)."""
        x = np.ascontiguousarray(x, np.float32)
        logits = np.ascontiguousarray(logits, np.float32)
        out = np.zeros_like(x)
        ok = self.L.drop_moe_ffn(hs[0], hs[1], hs[2], _ptr(x), _ptr(logits), x.shape[0], x.shape[1], n_ff, n_expert,
                                 k, int(norm), _ptr(out))
        return out if ok else None

    def free(self, h) -> None:
        self.L.drop_tensor_free(h)
        self._keep.pop(h, None)

    def upload(self, h) -> bool:
        return bool(self.L.drop_upload(h))

    def resident(self, h) -> bool:
        return bool(self.L.drop_resident(h))

    def release(self, h) -> None:
        self.L.drop_release(h)

    def bytes_resident(self) -> int:
        return int(self.L.drop_bytes_resident())

    def _mm(self, fn, h, x):
        _, n_in, n_out = self._keep[h]
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros((x.shape[0], n_out), np.float32)
        fn(h, _ptr(x), x.shape[0], n_in, n_out, _ptr(y))
        return y

    def matmul_tensor(self, h, x):
        return self._mm(self.L.drop_matmul_tensor, h, x)

    def matmul_cpu(self, h, x):
        return self._mm(self.L.drop_matmul_cpu, h, x)

    def matmul_tensors(self, hs, x):
        x = np.ascontiguousarray(x, np.float32)
        n_in = self._keep[hs[0]][1]
        ys = [np.zeros((x.shape[0], self._keep[h][2]), np.float32) for h in hs]
        arr = (_P * len(hs))(*hs)
        outs = (ctypes.c_int * len(hs))(*[self._keep[h][2] for h in hs])
        yp = (_P * len(hs))(*[y.ctypes.data for y in ys])
        self.L.drop_matmul_tensors(arr, len(hs), _ptr(x), x.shape[0], n_in, outs, yp)
        return ys

