"""The C ABI without a GPU: libqmoe.so loads, exports every function that
include/qmoe.h declares, and rejects malformed layer descriptions before it
touches the device.  Also the host-side helpers of qwen-go_amd/qmoe.py."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
import qmoe

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qmoe.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    return sorted(set(re.findall(r"\b(qmoe_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = qmoe.load_library()
    names = declared_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_status_strings():
    lib = qmoe.load_library()
    seen = set()
    for s in range(6):
        txt = lib.qmoe_status_string(s).decode()
        assert txt and txt != "unknown status"
        seen.add(txt)
    assert len(seen) == 6
    assert lib.qmoe_status_string(99).decode() == "unknown status"


def _desc(**kw):
    d = dict(hidden=256, n_experts=8, top_k=2, moe_inter=64, shared_inter=0, select_scope=0,
             router_fmt=qmoe.BF16, expert_fmt=qmoe.BF16, shared_fmt=qmoe.BF16, device=0)
    d.update(kw)
    return qmoe.QmoeDesc(**d)


@pytest.mark.parametrize("bad, status", [
    (dict(hidden=0), 1),
    (dict(top_k=9), 1),                    # top_k > n_experts (the reference panics, moe.go:56)
    (dict(select_scope=1), 1),             # scope below top_k
    (dict(select_scope=9), 1),             # scope above n_experts
    (dict(expert_fmt=7), 1),
    (dict(shared_inter=-32), 1),
    (dict(hidden=250), 5),                 # the group-32 formats need multiples of 32
    (dict(moe_inter=40), 5),
    (dict(n_experts=2048), 5),
    (dict(top_k=65, n_experts=128), 5),
])
def test_create_rejects_bad_descriptions(bad, status):
    lib = qmoe.load_library()
    h = ctypes.c_void_p()
    st = lib.qmoe_create(ctypes.byref(_desc(**bad)), ctypes.byref(h))
    assert st == status
    assert not h.value
    assert lib.qmoe_last_error(None)  # the thread-local message is set
    assert lib.qmoe_create(None, ctypes.byref(h)) == 1


def test_null_handles_are_rejected():
    lib = qmoe.load_library()
    assert lib.qmoe_forward(None, None, 1, None, None, None) == 1
    assert lib.qmoe_set_router(None, None, None) == 1
    assert lib.qmoe_dequant_debug(None, 0, 0, None) == 1
    lib.qmoe_destroy(None)  # no-op
    assert lib.qmoe_device_bytes(None) == 0


def test_bf16_helper_matches_oracle():
    rng = np.random.default_rng(2)
    v = (rng.standard_normal(10000) * 0.02).astype(np.float32)
    assert np.array_equal(qmoe.f32_to_bf16_bits(v), oracle.f32_to_bf16(v))
    b = qmoe.f32_to_bf16_bits(v)
    assert np.array_equal(qmoe.bf16_bits_to_f32(b).view(np.uint32), (b.astype(np.uint32) << 16))


def test_algorithmic_bytes_of_the_decode_layer():
    """Qwen3-30B-A3B at T=1 with 8 distinct experts: 8 x 3 x 2048 x 768 bf16
    experts + the 128 x 2048 bf16 router + x and out in f32 (about 76.0 MB)."""
    cfg = qmoe.CONFIGS["qwen3_30b_a3b"]
    ids = np.arange(8, dtype=np.int32).reshape(1, 8)
    b = qmoe.algorithmic_bytes(cfg, ids, 1)
    assert b == 8 * 3 * 2048 * 768 * 2 + 128 * 2048 * 2 + 2 * 2048 * 4
    ids2 = np.array([[0, 1, 2, 3, 4, 5, 6, 7], [0, 1, 2, 3, 4, 5, 6, 8]], np.int32)
    assert qmoe.algorithmic_bytes(cfg, ids2, 2) - b == 3 * 2048 * 768 * 2 + 2 * 2048 * 4
    assert qmoe.algorithmic_flops(cfg, 1) == 2 * 2048 * 128 + 8 * 2 * 3 * 2048 * 768


def test_weight_bytes_formats():
    assert qmoe.weight_bytes(qmoe.F32, 4, 64) == 4 * 64 * 4
    assert qmoe.weight_bytes(qmoe.BF16, 4, 64) == 4 * 64 * 2
    assert qmoe.weight_bytes(qmoe.INT8G32, 4, 64) == 4 * 64 + 4 * 2 * 2
    assert qmoe.weight_bytes(qmoe.INT4G32, 4, 64) == 4 * 32 + 4 * 2 * 2


def test_synthetic_weights_are_seeded():
    cfg = qmoe.LayerConfig(64, 4, 2, 32, 32, 0, qmoe.BF16, qmoe.INT8G32, qmoe.INT4G32, "s")
    a = qmoe.synthetic_weights(cfg, 9, quantizer=oracle.host_quantizer)
    b = qmoe.synthetic_weights(cfg, 9, quantizer=oracle.host_quantizer)
    assert np.array_equal(a.gate_up, b.gate_up) and np.array_equal(a.sh_down_s, b.sh_down_s)
    assert a.gate_up.shape == (4, 64, 64) and a.gate_up.dtype == np.int8
    assert a.down.shape == (4, 64, 32) and a.gate_up_s.shape == (4, 64, 2)
    assert a.sh_gate.shape == (32, 32) and a.sh_gate.dtype == np.uint8
    assert a.router.dtype == np.uint16 and a.router.shape == (4, 64)


@pytest.mark.parametrize("out_dim, in_dim, fmt, status", [
    (0, 64, qmoe.BF16, 1),
    (16, -64, qmoe.BF16, 1),
    (16, 64, 9, 1),                      # unknown format
    (16, 100, qmoe.BF16, 5),             # not a multiple of the 64-element bf16 step
    (16, 48, qmoe.INT8G32, 1),           # group-32 formats need in_dim % 32 == 0
    (16, 160, qmoe.INT4G32, 5),          # int4 and int8 super-chunks are 256 elements
    (16, 384, qmoe.INT8G32, 5),
    (16, 48, qmoe.INT8G32_F32S, 1),
    (16, 96, qmoe.INT4G32_F32S, 5),           # f32-scale formats keep their codes: 256-element steps
])
def test_linear_create_rejects_bad_shapes(out_dim, in_dim, fmt, status):
    lib = qmoe.load_library()
    h = ctypes.c_void_p()
    assert lib.qmoe_linear_create(out_dim, in_dim, fmt, 0, ctypes.byref(h)) == status
    assert not h.value
    assert lib.qmoe_linear_last_error(None)
    assert lib.qmoe_linear_create(16, 64, qmoe.BF16, 0, None) == 1


def test_linear_null_handles_are_rejected():
    lib = qmoe.load_library()
    assert lib.qmoe_linear_set(None, None, None) == 1
    assert lib.qmoe_linear_forward(None, None, 1, None) == 1
    assert lib.qmoe_linear_forward_device(None, None, 1, None, None) == 1
    assert lib.qmoe_linear_greedy(None, None, 1, None, None) == 1
    assert lib.qmoe_linear_argmax_device(None, None, 1, 1, None, None) == 1
    lib.qmoe_linear_destroy(None)
    assert lib.qmoe_linear_device_bytes(None) == 0


def test_linear_step_matches_the_library():
    """in_dim = one step passes the shape checks (then needs a device: status 0
    or 1); one step plus 32 elements is refused as unsupported (5)."""
    lib = qmoe.load_library()
    for fmt in (qmoe.F32, qmoe.BF16, qmoe.INT8G32, qmoe.INT4G32, qmoe.INT8G32_F32S, qmoe.INT4G32_F32S):
        step = qmoe.linear_step(fmt)
        h = ctypes.c_void_p()
        st = lib.qmoe_linear_create(4, step, fmt, 0, ctypes.byref(h))
        assert st in (0, 1), (fmt, st)
        if h.value:
            lib.qmoe_linear_destroy(h)
        if step > 32:
            h = ctypes.c_void_p()
            assert lib.qmoe_linear_create(4, step + 32, fmt, 0, ctypes.byref(h)) == 5, fmt
