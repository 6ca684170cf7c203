"""ctypes binding of liboracle.so, the CPU restatement of model/moe.go.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU baseline,
never as part of the product path.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

F32, BF16, INT8G32, INT4G32 = 0, 1, 2, 3

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")


def build() -> None:
    subprocess.run(["make", "-B", "-C", _HERE, "liboracle.so"], check=True,
                   stdout=subprocess.DEVNULL)


_lib = None


class OrcLinear(ctypes.Structure):
    _fields_ = [("fmt", ctypes.c_int), ("out_dim", ctypes.c_int), ("in_dim", ctypes.c_int),
                ("w", ctypes.c_void_p), ("scale", ctypes.c_void_p)]


class OrcMoe(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("n_experts", ctypes.c_int), ("top_k", ctypes.c_int),
                ("inter", ctypes.c_int), ("shared_inter", ctypes.c_int), ("scope", ctypes.c_int),
                ("router", OrcLinear), ("expert_fmt", ctypes.c_int),
                ("gate_up", ctypes.c_void_p), ("gate_up_scale", ctypes.c_void_p),
                ("down", ctypes.c_void_p), ("down_scale", ctypes.c_void_p),
                ("sh_gate", OrcLinear), ("sh_up", OrcLinear), ("sh_down", OrcLinear),
                ("shared_gate", ctypes.c_void_p), ("threads", ctypes.c_int)]


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i, f, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_bf16_to_f32.restype = f
        L.orc_f32_to_bf16_rne.argtypes = [f]
        L.orc_f32_to_bf16_rne.restype = ctypes.c_uint16
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = f
        L.orc_f32_to_f16_rne.argtypes = [f]
        L.orc_f32_to_f16_rne.restype = ctypes.c_uint16
        for n in ("orc_f32_to_bf16_array", "orc_f16_to_f32_array", "orc_f32_to_f16_array"):
            getattr(L, n).argtypes = [vp, vp, sz]
            getattr(L, n).restype = None
        L.orc_quantize_int8.argtypes = [vp, i, i, vp, vp]
        L.orc_quantize_int4.argtypes = [vp, i, i, vp, vp]
        L.orc_quantize_stack.argtypes = [i, vp, i, i, i, vp, vp]
        L.orc_dequantize.argtypes = [i, vp, vp, i, i, vp]
        L.orc_matvec.argtypes = [ctypes.POINTER(OrcLinear), vp, vp, i]
        L.orc_softmax.argtypes = [vp, i]
        L.orc_silu.argtypes = [vp, i]
        L.orc_sigmoid1.argtypes = [f]
        L.orc_sigmoid1.restype = f
        L.orc_select.argtypes = [vp, i, i, i, vp, vp]
        L.orc_argmax.argtypes = [vp, i]
        L.orc_argmax.restype = i
        L.orc_gemma_rmsnorm.argtypes = [vp, vp, i, f]
        L.orc_moe_forward.argtypes = [ctypes.POINTER(OrcMoe), vp, i, vp, vp, vp]
        L.orc_moe_forward.restype = i
        L.orc_moe_router.argtypes = [ctypes.POINTER(OrcMoe), vp, i, vp, vp, vp]
        L.orc_moe_router.restype = i
        _lib = L
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ------------------------------------------------------------- conversions

def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().orc_f32_to_bf16_array(_p(a), _p(out), a.size)
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def f32_to_f16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(a), _p(out), a.size)
    return out


def bf16_to_f32(b: int) -> float:
    return lib().orc_bf16_to_f32(b)


# --------------------------------------------------------------- quantiser

def quantize(bits: int, w: np.ndarray):
    """(..., rows, cols) f32 -> (codes, f32 scales) per quantizeInt8/4."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape[-2], w.shape[-1]
    n_mat = int(np.prod(w.shape[:-2])) if w.ndim > 2 else 1
    lead = w.shape[:-2]
    if bits == 8:
        codes = np.empty(lead + (rows, cols), np.int8)
    else:
        codes = np.empty(lead + (rows, cols // 2), np.uint8)
    scales = np.empty(lead + (rows, cols // 32), np.float32)
    lib().orc_quantize_stack(bits, _p(w), n_mat, rows, cols, _p(codes), _p(scales))
    return codes, scales


def quantize_f16(bits: int, w: np.ndarray):
    """Codes plus the f32 scales rounded to fp16 (bit patterns): the device format."""
    codes, s = quantize(bits, w)
    return codes, f32_to_f16(s)


def host_quantizer(bits: int, w: np.ndarray, n_mat: int, rows: int, cols: int, f32_scales: bool = False):
    """Drop-in for qmoe.device_quantizer that runs the oracle on the CPU.
    f32_scales: keep the quantiser's f32 scales (what qwen-quant writes)
    instead of rounding them to fp16."""
    a = np.asarray(w, np.float32).reshape(n_mat, rows, cols) if n_mat > 1 else np.asarray(w, np.float32).reshape(rows, cols)
    return quantize(bits, a) if f32_scales else quantize_f16(bits, a)


def dequantize(bits: int, codes: np.ndarray, scales_f32: np.ndarray, rows: int, cols: int) -> np.ndarray:
    out = np.empty((rows, cols), np.float32)
    lib().orc_dequantize(bits, _p(np.ascontiguousarray(codes)), _p(np.ascontiguousarray(scales_f32, np.float32)),
                         rows, cols, _p(out))
    return out


# ------------------------------------------------------------ primitives

def _linear(fmt: int, w: np.ndarray, scales_f32, rows: int, cols: int):
    l = OrcLinear(fmt, rows, cols, _p(w), _p(scales_f32) if scales_f32 is not None else None)
    return l


def matvec(fmt: int, w: np.ndarray, scales_f32, x: np.ndarray, rows: int, cols: int, threads: int = 1):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    l = _linear(fmt, np.ascontiguousarray(w), scales_f32, rows, cols)
    lib().orc_matvec(ctypes.byref(l), _p(x), _p(y), threads)
    return y


def softmax(v: np.ndarray) -> np.ndarray:
    v = np.array(v, np.float32, copy=True)
    lib().orc_softmax(_p(v), v.size)
    return v


def silu(v: np.ndarray) -> np.ndarray:
    v = np.array(v, np.float32, copy=True)
    lib().orc_silu(_p(v), v.size)
    return v


def sigmoid1(x: float) -> float:
    return lib().orc_sigmoid1(x)


def select(p: np.ndarray, k: int, scope: int):
    p = np.ascontiguousarray(p, np.float32)
    idx = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    lib().orc_select(_p(p), p.size, k, scope, _p(idx), _p(w))
    return idx, w


def argmax(v: np.ndarray) -> int:
    """model.go:652-660 on one row."""
    v = np.ascontiguousarray(v, np.float32)
    return int(lib().orc_argmax(_p(v), v.size))


def gemma_rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """gemmaRMSNormApply (tensors.go:147-157) on each row of x (T, n) or (n,)."""
    out = np.array(x, np.float32, copy=True, order="C")
    w = np.ascontiguousarray(w, np.float32)
    rows = out.reshape(-1, w.size)
    for r in rows:
        lib().orc_gemma_rmsnorm(_p(r), _p(w), w.size, eps)
    return out


# ------------------------------------------------------------------ layer

def orc_fmt(fmt: int) -> int:
    """The oracle's format for a product format: the group-32 formats with f32
    scales (4, 5) are the reference's quantLinear with its f32 scales, which
    the oracle takes for every INT format."""
    return {4: INT8G32, 5: INT4G32}.get(fmt, fmt)


class OracleLayer:
    """Holds an OrcMoe plus the numpy arrays it points into."""

    def __init__(self, hw, scope: int | None = None, threads: int = 1):
        cfg = hw.cfg
        self.cfg = cfg
        self.keep = []

        def sc(s):
            # fp16 bit patterns are widened exactly; f32 scales are used as they are
            if s is None:
                return None
            a = np.ascontiguousarray(s, np.float32) if s.dtype == np.float32 else f16_to_f32(s)
            self.keep.append(a)
            return a

        def lin(fmt, w, s16, rows, cols):
            self.keep.append(w)
            return _linear(orc_fmt(fmt), np.ascontiguousarray(w), sc(s16), rows, cols)

        H, E, I, Is = cfg.hidden, cfg.n_experts, cfg.moe_inter, cfg.shared_inter
        m = OrcMoe()
        m.hidden, m.n_experts, m.top_k, m.inter, m.shared_inter = H, E, cfg.top_k, I, Is
        m.scope = scope if scope else cfg.scope
        m.router = lin(cfg.router_fmt, hw.router, hw.router_s, E, H)
        m.expert_fmt = orc_fmt(cfg.expert_fmt)
        self.keep += [hw.gate_up, hw.down]
        m.gate_up = _p(hw.gate_up)
        m.gate_up_scale = _p(sc(hw.gate_up_s)) if hw.gate_up_s is not None else None
        m.down = _p(hw.down)
        m.down_scale = _p(sc(hw.down_s)) if hw.down_s is not None else None
        if Is:
            m.sh_gate = lin(cfg.shared_fmt, hw.sh_gate, hw.sh_gate_s, Is, H)
            m.sh_up = lin(cfg.shared_fmt, hw.sh_up, hw.sh_up_s, Is, H)
            m.sh_down = lin(cfg.shared_fmt, hw.sh_down, hw.sh_down_s, H, Is)
            g = np.ascontiguousarray(hw.shared_gate, np.float32)
            self.keep.append(g)
            m.shared_gate = _p(g)
        m.threads = threads
        self.m = m

    def forward(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32)
        T = x.shape[0]
        H, k = self.cfg.hidden, self.cfg.top_k
        out = np.empty((T, H), np.float32)
        ids = np.empty((T, k), np.int32)
        w = np.empty((T, k), np.float32)
        if lib().orc_moe_forward(ctypes.byref(self.m), _p(x), T, _p(out), _p(ids), _p(w)) != 0:
            raise ValueError("oracle rejected the layer description")
        return out, ids, w

    def forward_residual(self, x: np.ndarray, norm_w: np.ndarray, eps: float):
        """decodeLayers' MLP step (model/model.go:506-517): x + forward(gemmaRMSNorm(x)),
        the add in f32."""
        x = np.ascontiguousarray(x, np.float32)
        out, ids, w = self.forward(gemma_rmsnorm(x, norm_w, eps))
        return (x + out).astype(np.float32), ids, w, out

    def router(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32)
        T = x.shape[0]
        E, k = self.cfg.n_experts, self.cfg.top_k
        probs = np.empty((T, E), np.float32)
        ids = np.empty((T, k), np.int32)
        w = np.empty((T, k), np.float32)
        if lib().orc_moe_router(ctypes.byref(self.m), _p(x), T, _p(probs), _p(ids), _p(w)) != 0:
            raise ValueError("oracle rejected the layer description")
        return probs, ids, w
