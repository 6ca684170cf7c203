"""ctypes binding of libqmoe.so (include/qmoe.h) plus synthetic layer builders.

`MoeLayer` mirrors qwen-go's moeMLP (model/moe.go:10-99): construct it with the
layer's dimensions, upload the router, the stacked experts and the optional
shared expert, then call `forward(x)`.  Every compute call goes to the HIP
library; if libqmoe.so is missing the import fails loudly (there is no CPU
fallback).

The synthetic builders make the benchmark layers: weights ~ N(0, 0.02) from a
seed, bf16 by round-to-nearest-even, int8/int4 group-32 by the device
quantiser (quantizeInt8/4 of model/moe.go:165-217 with fp16 scales).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field

import numpy as np

F32, BF16, INT8G32, INT4G32, INT8G32_F32S, INT4G32_F32S = 0, 1, 2, 3, 4, 5
FORMAT_NAMES = {F32: "f32", BF16: "bf16", INT8G32: "int8g32", INT4G32: "int4g32",
                INT8G32_F32S: "int8g32-f32scales", INT4G32_F32S: "int4g32-f32scales"}
# the group-32 formats with the reference's own f32 scales (qwen-quant output)
F32_SCALE_FORMATS = (INT8G32_F32S, INT4G32_F32S)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqmoe.so")

STATUS = {0: "ok", 1: "invalid argument", 2: "invalid state", 3: "out of device memory",
          4: "HIP runtime error", 5: "unsupported configuration"}


class QmoeError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"qmoe status {status} ({STATUS.get(status, '?')}): {msg}")
        self.status = status


class QmoeDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "hidden", "n_experts", "top_k", "moe_inter", "shared_inter", "select_scope",
        "router_fmt", "expert_fmt", "shared_fmt", "device")]


_lib = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads libqmoe.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(path)
    vp, i32, i64, c = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_char_p
    sigs = {
        "qmoe_create": ([ctypes.POINTER(QmoeDesc), ctypes.POINTER(vp)], i32),
        "qmoe_destroy": ([vp], None),
        "qmoe_last_error": ([vp], c),
        "qmoe_status_string": ([i32], c),
        "qmoe_set_router": ([vp, vp, vp], i32),
        "qmoe_set_experts": ([vp, vp, vp, vp, vp], i32),
        "qmoe_set_shared": ([vp, vp, vp, vp, vp, vp, vp, vp], i32),
        "qmoe_quantize_experts": ([vp, vp, vp], i32),
        "qmoe_quantize_device": ([i32, vp, i64, i32, i32, vp, vp, vp], i32),
        "qmoe_forward": ([vp, vp, i32, vp, vp, vp], i32),
        "qmoe_forward_device": ([vp, vp, i32, vp, vp, vp, vp], i32),
        "qmoe_dequant_debug": ([vp, i32, i32, vp], i32),
        "qmoe_device_bytes": ([vp], i64),
        "qmoe_forward_path": ([vp, i32], i32),
        "qmoe_profile_enable": ([vp, ctypes.c_uint32], i32),
        "qmoe_profile_read": ([vp, vp, vp, i32], i32),
        "qmoe_router_fallbacks": ([vp, vp], i32),
        "qmoe_router_rescues": ([vp, vp], i32),
        "qmoe_router_bounds_debug": ([vp, vp, i32, vp], i32),
        "qmoe_debug_exchange_budget": ([vp, i64], i32),
        "qmoe_forward_device_noalloc": ([vp, vp, i32, vp, vp, vp, vp], i32),
        "qmoe_set_post_norm": ([vp, vp, ctypes.c_float], i32),
        "qmoe_reserve": ([vp, i32], i32),
        "qmoe_forward_residual": ([vp, vp, i32, vp, vp], i32),
        "qmoe_forward_residual_device": ([vp, vp, i32, vp, vp, vp, vp], i32),
        "qmoe_norm_recomputes": ([vp, vp], i32),
        "qmoe_debug_norm_sequential": ([vp, i32], i32),
        "qmoe_norm_debug": ([vp, vp, i32, vp], i32),
        "qmoe_linear_create": ([i32, i32, i32, i32, ctypes.POINTER(vp)], i32),
        "qmoe_linear_destroy": ([vp], None),
        "qmoe_linear_last_error": ([vp], c),
        "qmoe_linear_set": ([vp, vp, vp], i32),
        "qmoe_linear_forward": ([vp, vp, i32, vp], i32),
        "qmoe_linear_forward_device": ([vp, vp, i32, vp, vp], i32),
        "qmoe_linear_greedy": ([vp, vp, i32, vp, vp], i32),
        "qmoe_linear_argmax_device": ([vp, vp, i32, i32, vp, vp], i32),
        "qmoe_linear_device_bytes": ([vp], i64),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return ["qmoe_create", "qmoe_destroy", "qmoe_last_error", "qmoe_status_string",
            "qmoe_set_router", "qmoe_set_experts", "qmoe_set_shared", "qmoe_quantize_experts",
            "qmoe_quantize_device", "qmoe_forward", "qmoe_forward_device", "qmoe_dequant_debug",
            "qmoe_device_bytes", "qmoe_profile_enable", "qmoe_profile_read", "qmoe_router_fallbacks",
            "qmoe_router_rescues", "qmoe_router_bounds_debug", "qmoe_debug_exchange_budget",
            "qmoe_forward_device_noalloc", "qmoe_reserve", "qmoe_set_post_norm", "qmoe_forward_residual",
            "qmoe_forward_residual_device", "qmoe_norm_recomputes", "qmoe_debug_norm_sequential", "qmoe_norm_debug",
            "qmoe_linear_create", "qmoe_linear_destroy", "qmoe_linear_last_error", "qmoe_linear_set",
            "qmoe_linear_forward", "qmoe_linear_forward_device", "qmoe_linear_greedy",
            "qmoe_linear_argmax_device", "qmoe_linear_device_bytes"]


(STAGE_ROUTER, STAGE_SELECT, STAGE_GATE_UP, STAGE_SHARED_GATE_UP, STAGE_DOWN, STAGE_FUSED, STAGE_DISPATCH,
 STAGE_COMBINE) = range(8)
STAGE_COUNT = 8
STAGE_NAMES = {STAGE_ROUTER: "router_logits", STAGE_SELECT: "softmax_select",
               STAGE_GATE_UP: "gate_up", STAGE_SHARED_GATE_UP: "shared_gate_up", STAGE_DOWN: "down",
               STAGE_FUSED: "fused_experts", STAGE_DISPATCH: "dispatch", STAGE_COMBINE: "combine"}
PATH_GEMV, PATH_MFMA = 0, 1


def _ptr(a):
    if a is None:
        return None
    if isinstance(a, int):
        return a
    assert isinstance(a, np.ndarray) and a.flags["C_CONTIGUOUS"], "arrays must be C-contiguous"
    return a.ctypes.data


def _last_create_error(lib) -> str:
    return lib.qmoe_last_error(None).decode()


# --------------------------------------------------------------- conversions

def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    if nan.any():
        r[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def weight_bytes(fmt: int, rows: int, cols: int) -> int:
    """Device bytes of a (rows, cols) matrix in fmt (the f32-scale formats are
    stored as their f32 dequantisation)."""
    per2 = {F32: 8, BF16: 4, INT8G32: 2, INT4G32: 1, INT8G32_F32S: 8, INT4G32_F32S: 8}[fmt]
    b = rows * cols * per2 // 2
    if fmt in (INT8G32, INT4G32):
        b += rows * (cols // 32) * 2
    return b


# --------------------------------------------------------------------- layer

@dataclass
class LayerConfig:
    hidden: int
    n_experts: int
    top_k: int
    moe_inter: int
    shared_inter: int = 0
    select_scope: int = 0
    router_fmt: int = BF16
    expert_fmt: int = BF16
    shared_fmt: int = BF16
    name: str = ""
    tokens: tuple = field(default_factory=tuple)

    @property
    def scope(self) -> int:
        return self.select_scope or self.top_k

    def with_(self, **kw) -> "LayerConfig":
        d = dict(self.__dict__)
        d.update(kw)
        return LayerConfig(**d)


class MoeLayer:
    """One MoE layer resident on a gfx950 device (a qmoe_layer handle)."""

    def __init__(self, cfg: LayerConfig, device: int = 0):
        self.lib = load_library()
        self.cfg = cfg
        d = QmoeDesc(cfg.hidden, cfg.n_experts, cfg.top_k, cfg.moe_inter, cfg.shared_inter,
                     cfg.select_scope, cfg.router_fmt, cfg.expert_fmt, cfg.shared_fmt, device)
        h = ctypes.c_void_p()
        st = self.lib.qmoe_create(ctypes.byref(d), ctypes.byref(h))
        if st != 0:
            raise QmoeError(st, _last_create_error(self.lib))
        self.h = h

    def _check(self, st: int):
        if st != 0:
            raise QmoeError(st, self.lib.qmoe_last_error(self.h).decode())

    def set_router(self, w, scales=None):
        self._check(self.lib.qmoe_set_router(self.h, _ptr(w), _ptr(scales)))

    def set_experts(self, gate_up, gate_up_scales, down, down_scales):
        self._check(self.lib.qmoe_set_experts(self.h, _ptr(gate_up), _ptr(gate_up_scales),
                                              _ptr(down), _ptr(down_scales)))

    def set_shared(self, gate, gate_s, up, up_s, down, down_s, shared_gate):
        self._check(self.lib.qmoe_set_shared(self.h, _ptr(gate), _ptr(gate_s), _ptr(up), _ptr(up_s),
                                             _ptr(down), _ptr(down_s), _ptr(shared_gate)))

    def quantize_experts(self, gate_up_f32, down_f32):
        self._check(self.lib.qmoe_quantize_experts(self.h, _ptr(gate_up_f32), _ptr(down_f32)))

    def forward(self, x: np.ndarray):
        """x (T, H) float32 -> (out (T, H), ids (T, k), weights (T, k))."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        out = np.empty((T, self.cfg.hidden), np.float32)
        ids = np.empty((T, self.cfg.top_k), np.int32)
        w = np.empty((T, self.cfg.top_k), np.float32)
        self._check(self.lib.qmoe_forward(self.h, _ptr(x), T, _ptr(out), _ptr(ids), _ptr(w)))
        return out, ids, w

    def forward_device(self, d_x: int, T: int, d_out: int, d_ids: int | None = None,
                       d_w: int | None = None, stream: int | None = None):
        self._check(self.lib.qmoe_forward_device(self.h, d_x, T, d_out, d_ids, d_w, stream))

    def forward_device_noalloc(self, d_x: int, T: int, d_out: int, d_ids: int | None = None,
                               d_w: int | None = None, stream: int | None = None):
        """forward_device for T <= 32 with no device allocation (the kernels'
        scratch is a static device array shared by every call on the device)."""
        self._check(self.lib.qmoe_forward_device_noalloc(self.h, d_x, T, d_out, d_ids, d_w, stream))

    def reserve(self, max_T: int) -> None:
        """Size the workspace for calls of up to max_T tokens now (no allocation later)."""
        self._check(self.lib.qmoe_reserve(self.h, max_T))

    def set_post_norm(self, w, eps: float):
        """postAttentionLayernorm (H) f32 and float32(RmsNormEps)."""
        self._check(self.lib.qmoe_set_post_norm(self.h, _ptr(np.ascontiguousarray(w, np.float32)), eps))

    def forward_residual(self, x: np.ndarray):
        """decodeLayers' MLP step (model/model.go:506-517) for T tokens:
        returns (x + block(gemmaRMSNorm(x)), ids, weights); x is not modified."""
        xo = np.array(x, dtype=np.float32, copy=True, order="C")
        T = xo.shape[0]
        ids = np.empty((T, self.cfg.top_k), np.int32)
        w = np.empty((T, self.cfg.top_k), np.float32)
        self._check(self.lib.qmoe_forward_residual(self.h, _ptr(xo), T, _ptr(ids), _ptr(w)))
        return xo, ids, w

    def forward_residual_device(self, d_x: int, T: int, d_out: int, d_ids: int | None = None,
                                d_w: int | None = None, stream: int | None = None):
        self._check(self.lib.qmoe_forward_residual_device(self.h, d_x, T, d_out, d_ids, d_w, stream))

    def norm_recomputes(self) -> int:
        c = ctypes.c_int64()
        self._check(self.lib.qmoe_norm_recomputes(self.h, ctypes.byref(c)))
        return c.value

    def norm(self, x: np.ndarray) -> np.ndarray:
        """The post-attention norm alone (bit-exact check)."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self._check(self.lib.qmoe_norm_debug(self.h, _ptr(x), x.shape[0], _ptr(out)))
        return out

    def set_norm_sequential(self, on: bool) -> None:
        self._check(self.lib.qmoe_debug_norm_sequential(self.h, int(on)))

    def dequant(self, which: int, expert: int = 0) -> np.ndarray:
        c = self.cfg
        H, I, Is, E = c.hidden, c.moe_inter, c.shared_inter, c.n_experts
        shape = {0: (2 * I, H), 1: (H, I), 2: (E, H), 3: (Is, H), 4: (Is, H), 5: (H, Is)}[which]
        out = np.empty(shape, np.float32)
        self._check(self.lib.qmoe_dequant_debug(self.h, which, expert, _ptr(out)))
        return out

    def profile_enable(self, stages) -> None:
        mask = 0
        for st in stages:
            mask |= 1 << st
        self._check(self.lib.qmoe_profile_enable(self.h, mask))

    def profile_read(self, reset: bool = True):
        """-> (ms per stage, launches per stage), summed since the last reset."""
        ms = np.zeros(STAGE_COUNT, np.float64)
        n = np.zeros(STAGE_COUNT, np.int64)
        self._check(self.lib.qmoe_profile_read(self.h, _ptr(ms), _ptr(n), 1 if reset else 0))
        return ms, n

    def router_fallbacks(self) -> int:
        n = ctypes.c_int64()
        self._check(self.lib.qmoe_router_fallbacks(self.h, ctypes.byref(n)))
        return int(n.value)

    def router_bounds(self, x: np.ndarray) -> np.ndarray:
        """{S, B} per (token, expert) from the certified router forward uses
        for these tokens: (T, E, 2) float64."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        out = np.empty((T, self.cfg.n_experts, 2), dtype=np.float64)
        self._check(self.lib.qmoe_router_bounds_debug(self.h, x.ctypes.data, T, out.ctypes.data))
        return out

    def router_rescues(self) -> int:
        """Tokens whose first certification failed and was rescued by exact
        logits of the candidates in doubt (no full exact routing)."""
        n = ctypes.c_int64()
        self._check(self.lib.qmoe_router_rescues(self.h, ctypes.byref(n)))
        return int(n.value)

    def set_exchange_budget(self, ticks: int) -> None:
        """Wait budget of the T = 1 kernel's router exchange (100 MHz ticks;
        negative: the default; 0: give up at once, making the call fail)."""
        self._check(self.lib.qmoe_debug_exchange_budget(self.h, ticks))

    def device_bytes(self) -> int:
        return int(self.lib.qmoe_device_bytes(self.h))

    def forward_path(self, T: int) -> int:
        """PATH_GEMV (f32 activations) or PATH_MFMA (bf16 MFMA) for T tokens."""
        return int(self.lib.qmoe_forward_path(self.h, T))

    def close(self):
        if getattr(self, "h", None) is not None and self.h.value:
            self.lib.qmoe_destroy(self.h)
            self.h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Linear:
    """One dense projection resident on the device (a qmoe_linear handle):
    qwen-go's linear / quantLinear (model/model.go:106-205, model/moe.go:124-162)
    with outputs bit-identical to its sequential f32 sums.  Used for the dense
    MLP projections and the LM head; `greedy` adds the argmax of
    model/model.go:652-660 on the device."""

    def __init__(self, out_dim: int, in_dim: int, fmt: int, device: int = 0):
        self.lib = load_library()
        self.out_dim, self.in_dim, self.fmt = out_dim, in_dim, fmt
        h = ctypes.c_void_p()
        st = self.lib.qmoe_linear_create(out_dim, in_dim, fmt, device, ctypes.byref(h))
        if st != 0:
            raise QmoeError(st, self.lib.qmoe_linear_last_error(None).decode())
        self.h = h

    def _check(self, st: int):
        if st != 0:
            raise QmoeError(st, self.lib.qmoe_linear_last_error(self.h).decode())

    def set(self, w, scales=None):
        self._check(self.lib.qmoe_linear_set(self.h, _ptr(w), _ptr(scales)))

    def forward(self, x: np.ndarray) -> np.ndarray:
        """x (T, in) or (in,) float32 -> y (T, out) (or (out,))."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        one = x.ndim == 1
        x2 = x.reshape(1, -1) if one else x
        y = np.empty((x2.shape[0], self.out_dim), np.float32)
        self._check(self.lib.qmoe_linear_forward(self.h, _ptr(x2), x2.shape[0], _ptr(y)))
        return y[0] if one else y

    def forward_device(self, d_x: int, T: int, d_y: int, stream: int | None = None):
        self._check(self.lib.qmoe_linear_forward_device(self.h, d_x, T, d_y, stream))

    def greedy(self, x: np.ndarray, logits: bool = False):
        """Next tokens (T,) int32 of x (T, in); with logits=True also (T, out)."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, self.in_dim)
        T = x.shape[0]
        tok = np.empty(T, np.int32)
        lg = np.empty((T, self.out_dim), np.float32) if logits else None
        self._check(self.lib.qmoe_linear_greedy(self.h, _ptr(x), T, _ptr(tok), _ptr(lg)))
        return (tok, lg) if logits else tok

    def argmax_device(self, d_v: int, T: int, n: int, d_tok: int, stream: int | None = None):
        self._check(self.lib.qmoe_linear_argmax_device(self.h, d_v, T, n, d_tok, stream))

    def device_bytes(self) -> int:
        return int(self.lib.qmoe_linear_device_bytes(self.h))

    def close(self):
        if getattr(self, "h", None) is not None and self.h.value:
            self.lib.qmoe_linear_destroy(self.h)
            self.h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def linear_step(fmt: int) -> int:
    """in_dim granularity of Linear: one super-chunk of a row (256 elements for
    every group-32 format, whose 8 scales travel with it)."""
    return {F32: 32, BF16: 64, INT8G32: 256, INT4G32: 256, INT8G32_F32S: 256, INT4G32_F32S: 256}[fmt]


def quantize_device(bits: int, d_w: int, n_mat: int, rows: int, cols: int, d_codes: int,
                    d_scales: int, stream: int | None = None):
    lib = load_library()
    st = lib.qmoe_quantize_device(bits, d_w, n_mat, rows, cols, d_codes, d_scales, stream)
    if st != 0:
        raise QmoeError(st, _last_create_error(lib))


# ---------------------------------------------------------- the five layers

CONFIGS = {
    # toy layer, f32 everywhere, no shared expert; runs on model/moe.go as is
    "toy": LayerConfig(1024, 8, 2, 512, 0, 0, F32, F32, F32, "toy-h1024-e8-k2-i512-f32", (16,)),
    # Qwen3-30B-A3B-shaped layer, bf16
    "qwen3_30b_a3b": LayerConfig(2048, 128, 8, 768, 0, 0, BF16, BF16, BF16,
                                 "qwen3-30b-a3b-h2048-e128-k8-i768-bf16", (1, 8, 2048)),
    # same shape, int8 group-32 experts
    "qwen3_30b_a3b_int8": LayerConfig(2048, 128, 8, 768, 0, 0, BF16, INT8G32, BF16,
                                      "qwen3-30b-a3b-h2048-e128-k8-i768-int8g32", (1, 512)),
    # Qwen3-Next-style sparse layer with a gated shared expert, int4 group-32
    "qwen3_next": LayerConfig(2048, 512, 10, 512, 512, 0, BF16, INT4G32, INT4G32,
                              "qwen3-next-h2048-e512-k10-i512-s512-int4g32", (1, 4096)),
}


def layer_bytes(cfg: LayerConfig) -> dict:
    """Stored bytes of each part of a layer."""
    H, E, I, Is = cfg.hidden, cfg.n_experts, cfg.moe_inter, cfg.shared_inter
    per_expert = weight_bytes(cfg.expert_fmt, 2 * I, H) + weight_bytes(cfg.expert_fmt, H, I)
    shared = 0
    if Is:
        shared = 2 * weight_bytes(cfg.shared_fmt, Is, H) + weight_bytes(cfg.shared_fmt, H, Is) + H * 4
    return {"router": weight_bytes(cfg.router_fmt, E, H), "per_expert": per_expert, "shared": shared}


def algorithmic_bytes(cfg: LayerConfig, ids: np.ndarray, T: int) -> int:
    """HBM bytes one forward must move: the distinct experts routed to, the
    router, the shared expert, x in and out (f32)."""
    b = layer_bytes(cfg)
    touched = len(np.unique(ids))
    return touched * b["per_expert"] + b["router"] + b["shared"] + 2 * T * cfg.hidden * 4


def algorithmic_flops(cfg: LayerConfig, T: int) -> int:
    H, E, k, I, Is = cfg.hidden, cfg.n_experts, cfg.top_k, cfg.moe_inter, cfg.shared_inter
    f = 2 * H * E + k * 2 * 3 * H * I
    if Is:
        f += 2 * 3 * H * Is + 2 * H
    return T * f


_BIG = 1 << 24  # elements; larger arrays come from torch's multi-threaded CPU generator


def _normal(seed: int, shape, std: float) -> np.ndarray:
    """float32 ~ N(0, std^2) from a seed.  Small arrays use numpy's PCG64
    (identical on every machine with the same numpy); large ones use a seeded
    torch CPU generator for speed.  Either way both the device and the oracle
    consume the same host array."""
    n = int(np.prod(shape))
    if n <= _BIG:
        rng = np.random.default_rng(seed)
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)
    import torch
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(tuple(shape), generator=g, dtype=torch.float32)
    t.mul_(std)
    return t.numpy()


def _to_bf16(w: np.ndarray) -> np.ndarray:
    if w.size <= _BIG:
        return f32_to_bf16_bits(w)
    import torch
    return torch.from_numpy(np.ascontiguousarray(w, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


@dataclass
class HostWeights:
    """Host copies of one layer's weights in the device formats, plus the f32
    scales widened from fp16 (what the oracle reads)."""
    cfg: LayerConfig
    router: np.ndarray
    router_s: np.ndarray | None
    gate_up: np.ndarray
    gate_up_s: np.ndarray | None
    down: np.ndarray
    down_s: np.ndarray | None
    sh_gate: np.ndarray | None = None
    sh_gate_s: np.ndarray | None = None
    sh_up: np.ndarray | None = None
    sh_up_s: np.ndarray | None = None
    sh_down: np.ndarray | None = None
    sh_down_s: np.ndarray | None = None
    shared_gate: np.ndarray | None = None

    def upload(self, layer: MoeLayer):
        layer.set_router(self.router, self.router_s)
        layer.set_experts(self.gate_up, self.gate_up_s, self.down, self.down_s)
        if self.cfg.shared_inter:
            layer.set_shared(self.sh_gate, self.sh_gate_s, self.sh_up, self.sh_up_s,
                             self.sh_down, self.sh_down_s, self.shared_gate)


def _store(fmt: int, w: np.ndarray, n_mat: int, rows: int, cols: int, quantizer):
    """f32 (n_mat, rows, cols) -> (stored array, scales or None): fp16 scale
    bits for INT8G32/INT4G32, the quantiser's f32 scales for the f32-scale
    formats (quantizer(..., f32_scales=True))."""
    if fmt == F32:
        return np.ascontiguousarray(w, np.float32), None
    if fmt == BF16:
        return _to_bf16(w), None
    bits = 8 if fmt in (INT8G32, INT8G32_F32S) else 4
    if fmt in F32_SCALE_FORMATS:
        return quantizer(bits, w, n_mat, rows, cols, f32_scales=True)
    return quantizer(bits, w, n_mat, rows, cols)


def device_quantizer(bits: int, w: np.ndarray, n_mat: int, rows: int, cols: int, f32_scales: bool = False):
    """Quantises on the device (qmoe_quantize_device); returns host codes and
    fp16 scale bits."""
    if f32_scales:
        raise ValueError("the device quantiser writes fp16 scales; quantise f32-scale formats on the host")
    import torch
    dw = torch.from_numpy(np.ascontiguousarray(w, np.float32).reshape(-1)).to("cuda")
    ncodes = n_mat * rows * (cols if bits == 8 else cols // 2)
    codes = torch.empty(ncodes, dtype=torch.uint8, device="cuda")
    scales = torch.empty(n_mat * rows * (cols // 32), dtype=torch.int16, device="cuda")
    quantize_device(bits, dw.data_ptr(), n_mat, rows, cols, codes.data_ptr(), scales.data_ptr(),
                    torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    c = codes.cpu().numpy()
    if bits == 8:
        c = c.view(np.int8)
    return c, scales.cpu().numpy().view(np.uint16)


def synthetic_weights(cfg: LayerConfig, seed: int, quantizer=device_quantizer,
                      router_scale: float = 1.0) -> HostWeights:
    """Seeded N(0, 0.02) weights in cfg's formats.  router_scale multiplies the
    router weights before rounding (x4 sharpens the logits)."""
    H, E, I, Is = cfg.hidden, cfg.n_experts, cfg.moe_inter, cfg.shared_inter
    s0 = seed * 1000
    r32 = _normal(s0 + 1, (E, H), 0.02) * np.float32(router_scale)
    router, router_s = _store(cfg.router_fmt, r32, 1, E, H, quantizer)
    gu32 = _normal(s0 + 2, (E, 2 * I, H), 0.02)
    gate_up, gate_up_s = _store(cfg.expert_fmt, gu32, E, 2 * I, H, quantizer)
    del gu32
    dn32 = _normal(s0 + 3, (E, H, I), 0.02)
    down, down_s = _store(cfg.expert_fmt, dn32, E, H, I, quantizer)
    del dn32
    hw = HostWeights(cfg, router, router_s, gate_up, gate_up_s, down, down_s)
    if Is:
        g = _normal(s0 + 4, (Is, H), 0.02)
        u = _normal(s0 + 5, (Is, H), 0.02)
        dd = _normal(s0 + 6, (H, Is), 0.02)
        hw.sh_gate, hw.sh_gate_s = _store(cfg.shared_fmt, g, 1, Is, H, quantizer)
        hw.sh_up, hw.sh_up_s = _store(cfg.shared_fmt, u, 1, Is, H, quantizer)
        hw.sh_down, hw.sh_down_s = _store(cfg.shared_fmt, dd, 1, H, Is, quantizer)
        hw.shared_gate = _normal(s0 + 7, (H,), 0.02)
    return hw


def synthetic_tokens(cfg: LayerConfig, T: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed + 7919)
    return rng.standard_normal((T, cfg.hidden), dtype=np.float32)


def skewed_tokens(cfg, hw, T, seed, target):
    """Prefill tokens with a skewed expert load: x_t = z_t + c u with a fixed
    random unit direction u; c is chosen on the host (router logits in
    float64) so that the busiest expert receives about `target` times the
    median expert's load.  Returns (x, load stats)."""
    rng = np.random.default_rng(seed)
    u = rng.standard_normal(cfg.hidden)
    u /= np.linalg.norm(u)
    z = synthetic_tokens(cfg, T, seed)
    if cfg.router_fmt == BF16:
        r = bf16_bits_to_f32(hw.router).astype(np.float64)
    else:
        r = np.asarray(hw.router, np.float64)
    r = r.reshape(cfg.n_experts, cfg.hidden)
    zl, ul = z.astype(np.float64) @ r.T, r @ u

    def load(c):
        lg = zl + c * ul
        top = np.argsort(-lg, axis=1, kind="stable")[:, :cfg.top_k]
        return np.bincount(top.reshape(-1), minlength=cfg.n_experts)

    def ratio(c):
        n = load(c)
        return n.max() / max(np.median(n), 1.0)

    lo, hi = 0.0, 64.0
    if ratio(lo) < target:
        for _ in range(30):
            mid = 0.5 * (lo + hi)
            lo, hi = (mid, hi) if ratio(mid) < target else (lo, mid)
    c = hi if ratio(lo) < target else lo
    n = load(c)
    x = (z + c * u[None, :]).astype(np.float32)
    stats = {"c": round(float(c), 3), "max_load": int(n.max()), "median_load": float(np.median(n)),
             "min_load": int(n.min()), "experts_used": int((n > 0).sum())}
    return x, stats
