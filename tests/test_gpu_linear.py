"""GPU parity of the dense projection (qmoe_linear_*) and the greedy token.

Bars: the outputs are the reference's sequential f32 sums (linear.matvec,
matmulVec, quantLinear.forward: model/model.go:131-176, model/tensors.go:77-89,
model/moe.go:159-162), so y must equal the oracle's matvec bit for bit; the
greedy token must equal model.go:652-660's argmax of those logits exactly.
Every test prints the case it runs before touching the GPU.
"""
import numpy as np
import pytest

import oracle
import qmoe

pytestmark = pytest.mark.gpu


def announce(msg):
    print(f"[case] {msg}", flush=True)


def make_weights(fmt, rows, cols, seed):
    """Seeded N(0, 0.02) weights stored in fmt, plus what the oracle takes:
    (stored, scales for the device, oracle format, oracle scales f32)."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))
    if fmt == qmoe.F32:
        return w, None, oracle.F32, None
    if fmt == qmoe.BF16:
        return qmoe.f32_to_bf16_bits(w), None, oracle.BF16, None
    bits = 8 if fmt in (qmoe.INT8G32, qmoe.INT8G32_F32S) else 4
    if fmt in qmoe.F32_SCALE_FORMATS:
        codes, s = oracle.quantize(bits, w)
        return codes, s, oracle.orc_fmt(fmt), s
    codes, s16 = oracle.quantize_f16(bits, w)
    return codes, s16, fmt, oracle.f16_to_f32(s16)


def oracle_rows(ofmt, stored, osc, x, rows, cols):
    return np.stack([oracle.matvec(ofmt, stored, osc, x[t], rows, cols, threads=8) for t in range(x.shape[0])])


CASES = [  # (fmt, rows, cols, T)
    (qmoe.F32, 300, 1024, 1), (qmoe.F32, 64, 32, 5),
    (qmoe.BF16, 1000, 2048, 1), (qmoe.BF16, 257, 512, 8), (qmoe.BF16, 4099, 2048, 13), (qmoe.BF16, 8, 64, 2),
    (qmoe.INT8G32, 777, 2048, 1), (qmoe.INT8G32, 130, 256, 9), (qmoe.INT8G32, 64, 768, 2),
    (qmoe.INT4G32, 1500, 2048, 1), (qmoe.INT4G32, 65, 256, 3), (qmoe.INT4G32, 2048, 512, 1),
    (qmoe.BF16, 100, 4096, 4), (qmoe.BF16, 2048, 768, 1), (qmoe.F32, 129, 96, 8),
    (qmoe.INT8G32_F32S, 512, 2048, 1), (qmoe.INT4G32_F32S, 300, 1024, 4), (qmoe.INT8G32_F32S, 70, 768, 9),
    (qmoe.INT4G32_F32S, 4096, 2048, 1),
]


@pytest.mark.parametrize("fmt, rows, cols, T", CASES)
def test_linear_bit_exact(fmt, rows, cols, T):
    announce(f"linear {qmoe.FORMAT_NAMES[fmt]} ({rows}, {cols}) T={T}")
    stored, sc, ofmt, osc = make_weights(fmt, rows, cols, seed=rows * 7 + cols + T)
    rng = np.random.default_rng(T + 3)
    x = rng.standard_normal((T, cols), dtype=np.float32)
    lin = qmoe.Linear(rows, cols, fmt)
    try:
        lin.set(stored, sc)
        y = lin.forward(x)
    finally:
        lin.close()
    ref = oracle_rows(ofmt, stored, osc, x, rows, cols)
    bad = np.argwhere(y.view(np.uint32) != ref.view(np.uint32))
    assert bad.size == 0, f"{len(bad)} outputs differ, first at {bad[:3]}: {y[tuple(bad[0])]} vs {ref[tuple(bad[0])]}"


def test_linear_device_pointers_and_T0():
    import torch
    announce("linear bf16 (512, 2048) T=3 device pointers, T=0")
    rows, cols, T = 512, 2048, 3
    stored, _, ofmt, _ = make_weights(qmoe.BF16, rows, cols, seed=5)
    x = np.random.default_rng(6).standard_normal((T, cols), dtype=np.float32)
    lin = qmoe.Linear(rows, cols, qmoe.BF16)
    try:
        lin.set(stored)
        dx = torch.from_numpy(x).cuda()
        dy = torch.full((T, rows), float("nan"), device="cuda")
        lin.forward_device(dx.data_ptr(), T, dy.data_ptr(), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        y = dy.cpu().numpy()
        lin.forward_device(dx.data_ptr(), 0, dy.data_ptr())  # T = 0: nothing to do
        assert lin.device_bytes() >= rows * cols * 2
    finally:
        lin.close()
    ref = oracle_rows(ofmt, stored, None, x, rows, cols)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_linear_rejects_bad_use():
    announce("linear argument checks")
    with pytest.raises(qmoe.QmoeError) as e:
        qmoe.Linear(10, 100, qmoe.BF16)  # 100 not a multiple of 64
    assert e.value.status == 5
    with pytest.raises(qmoe.QmoeError) as e:
        qmoe.Linear(10, 384, qmoe.INT4G32)  # int4 super-chunks are 256 elements
    assert e.value.status == 5
    with pytest.raises(qmoe.QmoeError) as e:
        qmoe.Linear(0, 64, qmoe.BF16)
    assert e.value.status == 1
    lin = qmoe.Linear(16, 64, qmoe.BF16)
    try:
        with pytest.raises(qmoe.QmoeError) as e:
            lin.forward(np.zeros((1, 64), np.float32))  # weights not uploaded
        assert e.value.status == 2
    finally:
        lin.close()


def test_lm_head_greedy_token():
    """The LM head of a 151936-token vocabulary over H = 2048 (bf16, tied or
    untied: the same matvec) and greedy decode's argmax."""
    rows, cols = 151936, 2048
    announce(f"lm head bf16 ({rows}, {cols}) T=1 and T=2 greedy")
    rng = np.random.default_rng(21)
    w = qmoe.f32_to_bf16_bits(rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))
    x = rng.standard_normal((2, cols), dtype=np.float32)
    lin = qmoe.Linear(rows, cols, qmoe.BF16)
    try:
        lin.set(w)
        tok, logits = lin.greedy(x, logits=True)
        tok1 = lin.greedy(x[:1])
    finally:
        lin.close()
    ref = oracle_rows(oracle.BF16, w, None, x, rows, cols)
    assert np.array_equal(logits.view(np.uint32), ref.view(np.uint32))
    want = [oracle.argmax(ref[t]) for t in range(2)]
    assert list(tok) == want and tok1[0] == want[0]


@pytest.mark.parametrize("n", [1, 7, 1024, 1025, 8193, 151936])
def test_argmax_device_semantics(n):
    import torch
    announce(f"argmax n={n} T=6 with ties and NaNs")
    rng = np.random.default_rng(n)
    v = rng.integers(-50, 50, (6, n)).astype(np.float32)  # ties
    v[1, :] = -np.inf
    v[2, 0] = np.nan                       # v[0] NaN -> 0
    v[3, rng.random(n) < 0.3] = np.nan     # NaNs skipped
    v[4, :] = np.nan
    v[5, -1] = 1e30                        # the last element
    if n > 1:
        v[0, n // 2:] = v[0].max()         # the first of many equal maxima
    lin = qmoe.Linear(16, 64, qmoe.BF16)
    try:
        lin.set(np.zeros((16, 64), np.uint16))
        dv = torch.from_numpy(v).cuda()
        dt = torch.full((6,), -7, dtype=torch.int32, device="cuda")
        lin.argmax_device(dv.data_ptr(), 6, n, dt.data_ptr(), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        got = dt.cpu().numpy()
    finally:
        lin.close()
    want = [oracle.argmax(v[t]) for t in range(6)]
    assert list(got) == want
