"""CPU pins of the oracle (oracle/qmoe_oracle.c) -- no GPU.

Each oracle function is checked against something that does not restate it:
numpy / torch conversions, hand-derived known answers with exact f32
arithmetic (tests/golden/known_answers.json), a float64 evaluation of the
layer written from the reference's definitions (tests/golden/tiny_layer.npz),
brute force, closed forms and invariants.  A plausible slip -- a dropped
term, FMA contraction, pairwise instead of sequential sums, round-half-even
instead of half-away, swapped nibbles, a transposed operand -- fails at least
one of them.
"""
import json
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def known():
    with open(os.path.join(GOLDEN, "known_answers.json")) as fh:
        return json.load(fh)


@pytest.fixture(scope="module")
def tiny():
    with np.load(os.path.join(GOLDEN, "tiny_layer.npz")) as z:
        return {k: z[k] for k in z.files}


def bits32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------ conversions

def test_f16_to_f32_all_patterns():
    """safetensors.go:182-207 widening == IEEE half -> single for all 65536."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits32(got)[~nan], bits32(ref)[~nan])
    # NaNs keep sign and payload, shifted into the top mantissa bits
    # (safetensors.go:201-202); numpy may quiet them, so compare by fields
    hn = h[nan].astype(np.uint32)
    want = ((hn >> 15) << 31) | np.uint32(0x7F800000) | ((hn & 0x3FF) << 13)
    assert np.array_equal(bits32(got)[nan], want)


def test_f32_to_f16_rne():
    rng = np.random.default_rng(3)
    v = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(0.02),
        rng.standard_normal(5000).astype(np.float32) * np.float32(1e-6),   # subnormal halves
        np.float32([0.0, -0.0, 65504.0, 65520.0, 1e9, -1e9, 6.1e-5, 5.96e-8, 2.98e-8, 1.0 + 2 ** -11]),
        (np.arange(1, 2049, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),  # ties
    ])
    got = oracle.f32_to_f16(v)
    with np.errstate(over="ignore"):
        assert np.array_equal(got, v.astype(np.float16).view(np.uint16))


def test_bf16_conversions():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(4)
    v = np.concatenate([rng.standard_normal(50000).astype(np.float32),
                        np.float32([0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3e38, -1e-40])])
    got = oracle.f32_to_bf16(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    for b in (0x3F80, 0xBF80, 0x0001, 0x7F7F, 0x4049):
        want = torch.from_numpy(np.uint16([b]).view(np.int16)).view(torch.bfloat16).float().item()
        assert oracle.bf16_to_f32(b) == want


# --------------------------------------------------------------- quantiser

def test_quantize_known_answers(known):
    for case in known["quantize"]:
        w = np.float32(case["w"]).reshape(1, 32)
        codes, scales = oracle.quantize(case["bits"], w)
        assert scales[0, 0] == np.float32(case["scale"])
        if case["bits"] == 8:
            assert codes.reshape(-1).tolist() == case["codes"]
        else:
            assert codes.reshape(-1).tolist() == case["packed"]


@pytest.mark.parametrize("bits", [8, 4])
def test_quantize_invariants(bits):
    """Round trip within half a step, codes in range, amax element at the
    extreme code (the invariant is stronger than TestQuantRoundTrip's 0.02)."""
    rng = np.random.default_rng(7)
    rows, cols = 16, 128
    w = (rng.standard_normal((rows, cols)) * 0.1).astype(np.float32)
    codes, s = oracle.quantize(bits, w)
    dq = oracle.dequantize(bits, codes, s, rows, cols)
    step = np.repeat(s, 32, axis=1)
    assert np.all(np.abs(w.astype(np.float64) - dq) <= step.astype(np.float64) * (0.5 + 1e-6))
    lim = 127 if bits == 8 else 7
    vals = np.rint(dq / step).astype(np.int64)
    assert vals.min() >= -lim and vals.max() <= lim
    g = np.abs(w).reshape(rows, cols // 32, 32)
    at = g.argmax(axis=2)
    v3 = vals.reshape(rows, cols // 32, 32)
    assert np.all(np.abs(np.take_along_axis(v3, at[..., None], 2)) == lim)
    if bits == 4:
        nib = np.stack([codes >> 4, codes & 0xF], axis=-1).reshape(rows, cols)
        assert nib.min() >= 1 and nib.max() <= 15
    if bits == 8:  # TestQuantRoundTrip's bar for int8 (model_test.go:130-149)
        assert np.all(np.abs(w - dq) <= 0.02)


def test_dequantize_known_bytes(known):
    for case in known["dequantize"]:
        bits, b = case["bits"], case["bytes"]
        nbytes = 32 if bits == 8 else 16
        raw = np.zeros(nbytes, np.uint8)
        raw[:len(b)] = b
        codes = raw.view(np.int8) if bits == 8 else raw
        got = oracle.dequantize(bits, codes.reshape(1, -1), np.float32([[case["scale"]]]), 1, 32)
        vals = case["values"]
        assert got[0, :len(vals)].tolist() == vals
        pad_value = 0.0 if bits == 8 else -8.0 * case["scale"]
        assert np.all(got[0, len(vals):] == pad_value)


# ------------------------------------------------------------ primitives

def seq_dot_f32(x, w):
    """Sequential f32 sum of f32 products, each step rounded (no FMA)."""
    acc = np.float32(0.0)
    for a, b in zip(x, w):
        acc = np.float32(acc + np.float32(a * b))
    return acc


@pytest.mark.parametrize("fmt", [oracle.F32, oracle.BF16, oracle.INT8G32, oracle.INT4G32])
def test_matvec_sequential_order(fmt):
    rng = np.random.default_rng(11 + fmt)
    rows, cols = 6, 96
    wf = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    if fmt == oracle.F32:
        w, s, dense = wf, None, wf
    elif fmt == oracle.BF16:
        w = oracle.f32_to_bf16(wf)
        s = None
        dense = (w.astype(np.uint32) << np.uint32(16)).view(np.float32)
    else:
        bits = 8 if fmt == oracle.INT8G32 else 4
        w, s = oracle.quantize(bits, wf)
        dense = oracle.dequantize(bits, w, s, rows, cols)
    y = oracle.matvec(fmt, w, s, x, rows, cols)
    want = np.float32([seq_dot_f32(x, dense[r]) for r in range(rows)])
    assert np.array_equal(bits32(y), bits32(want))
    # and it is the dot product (float64) to within the sequential-sum bound
    exact = dense.astype(np.float64) @ x.astype(np.float64)
    bound = cols * 2.0 ** -24 * (np.abs(dense).astype(np.float64) @ np.abs(x).astype(np.float64)) * 1.01
    assert np.all(np.abs(y - exact) <= bound)


def test_matvec_threads_do_not_change_bits():
    """bf16 linears fan out over goroutines (model.go:136-162), one row per
    worker, so the result is independent of the thread count."""
    rng = np.random.default_rng(12)
    rows, cols = 256, 512  # rows * cols >= 65536: the threaded branch
    w = oracle.f32_to_bf16((rng.standard_normal((rows, cols)) * 0.05).astype(np.float32))
    x = rng.standard_normal(cols).astype(np.float32)
    y1 = oracle.matvec(oracle.BF16, w, None, x, rows, cols, threads=1)
    y8 = oracle.matvec(oracle.BF16, w, None, x, rows, cols, threads=8)
    assert np.array_equal(bits32(y1), bits32(y8))


def test_softmax():
    l = np.float32([3.0, 0.0, 0.0, 0.0])
    p = oracle.softmax(l)
    e3 = np.exp(3.0)
    assert abs(p[0] - e3 / (e3 + 3)) < 1e-7 and abs(p[1] - 1 / (e3 + 3)) < 1e-8
    assert p[1] == p[2] == p[3]
    rng = np.random.default_rng(5)
    for _ in range(20):
        v = (rng.standard_normal(128) * 3).astype(np.float32)
        p = oracle.softmax(v).astype(np.float64)
        q = np.exp(v.astype(np.float64) - v.max())
        q /= q.sum()
        # f32 rounding of (v - max) moves the exponent by up to |v - max| * 2^-24
        bound = (np.abs(v.astype(np.float64) - v.max()) + 4.0) * 2.0 ** -23
        assert np.all(np.abs(p - q) / q <= bound)
        assert abs(p.sum() - 1) < 1e-6
        o = np.argsort(v, kind="stable")
        assert np.all(np.diff(p[o]) >= 0)  # monotone in the logits


def test_silu_sigmoid_closed_forms():
    v = np.float32([0.0, 1.0, -1.0, 20.0, -20.0, 1e-3, -100.0])
    got = oracle.silu(v).astype(np.float64)
    want = v.astype(np.float64) / (1 + np.exp(-v.astype(np.float64)))
    assert got[0] == 0.0
    assert np.all(np.abs(got - want) <= 2e-7 * np.maximum(np.abs(want), 1e-30))
    assert oracle.sigmoid1(0.0) == 0.5
    for g in (0.3, -2.0, 9.0):
        assert abs(oracle.sigmoid1(g) - 1 / (1 + np.exp(-g))) < 1e-7


def brute_select(p, k, scope):
    order = sorted(range(scope), key=lambda e: (-p[e], e))[:k]
    return order


def test_select_known_answers(known):
    for case in known["select"]:
        idx, w = oracle.select(np.float32(case["p"]), case["k"], case["scope"])
        assert idx.tolist() == case["ids"], case


@pytest.mark.parametrize("scope_kind", ["k", "E", "mid"])
def test_select_brute_force(scope_kind):
    rng = np.random.default_rng(21)
    E, k = 64, 8
    scope = {"k": k, "E": E, "mid": 20}[scope_kind]
    for trial in range(200):
        p = rng.random(E).astype(np.float32)
        if trial % 3 == 0:  # many exact ties
            p = np.round(p * 4).astype(np.float32) / np.float32(4)
        idx, w = oracle.select(p, k, scope)
        assert idx.tolist() == brute_select(p, k, scope)
        if scope == k:
            assert sorted(idx.tolist()) == list(range(k))  # the first-k quirk: set {0..k-1}
        ws = np.float64(p[idx]).sum()
        assert np.allclose(w, p[idx] / (ws + 1e-9), rtol=1e-6)
        assert abs(np.float64(w).sum() - ws / (ws + 1e-9)) < 1e-6


# ------------------------------------------------------------------ layer

class _HW:
    """Minimal host-weights holder in the shape OracleLayer reads."""

    def __init__(self, cfg, **kw):
        self.cfg = cfg
        for k_, v in kw.items():
            setattr(self, k_, v)


def _cfg(H, E, k, I, Is, scope):
    import qmoe
    return qmoe.LayerConfig(H, E, k, I, Is, scope, qmoe.F32, qmoe.F32, qmoe.F32, "t")


def test_moe_routing_known_answer(known):
    """TestMoERouting (model_test.go:182-201): router row 0 = [1,2,3,4,0..],
    logits ~[3,0,0,0], first-k selection [0,1]; with zero experts and a zero
    shared expert the output is exactly zero.  Then with non-zero experts the
    output is the closed form w0 * down0(act0) + w1 * down1(act1)."""
    c = known["routing"]
    H, E, k, I, Is = 8, 4, 2, 16, 4
    router = np.zeros((E, H), np.float32)
    router[0] = c["router_row0"]
    x = np.float32(c["x"]).reshape(1, H)
    zeros = dict(router=router, router_s=None, gate_up=np.zeros((E, 2 * I, H), np.float32), gate_up_s=None,
                 down=np.zeros((E, H, I), np.float32), down_s=None,
                 sh_gate=np.zeros((Is, H), np.float32), sh_gate_s=None, sh_up=np.zeros((Is, H), np.float32),
                 sh_up_s=None, sh_down=np.zeros((H, Is), np.float32), sh_down_s=None,
                 shared_gate=np.zeros(H, np.float32))
    cfg = _cfg(H, E, k, I, Is, k)
    L = oracle.OracleLayer(_HW(cfg, **zeros))
    out, ids, w = L.forward(x)
    assert ids[0].tolist() == c["ids_first_k"]
    assert np.all(out == 0.0)
    probs, _, _ = L.router(x)
    assert abs(probs[0, 0] - c["p0"]) < 1e-6 and abs(probs[0, 1] - c["p1"]) < 1e-7
    assert abs(w[0, 0] - c["w0"]) < 1e-6 and abs(w[0, 1] - c["w1"]) < 1e-6
    # non-zero experts 0 and 1: closed form
    rng = np.random.default_rng(1)
    gu = (rng.standard_normal((E, 2 * I, H)) * 0.2).astype(np.float32)
    dn = (rng.standard_normal((E, H, I)) * 0.2).astype(np.float32)
    L2 = oracle.OracleLayer(_HW(cfg, **{**zeros, "gate_up": gu, "down": dn}))
    out2, ids2, w2 = L2.forward(x)
    xd = x[0].astype(np.float64)
    want = np.zeros(H)
    for r, e in enumerate(ids2[0]):
        h = gu[e].astype(np.float64) @ xd
        a = h[:I] / (1 + np.exp(-h[:I])) * h[I:]
        want += w2[0, r] * (dn[e].astype(np.float64) @ a)
    assert np.max(np.abs(out2[0] - want)) <= 1e-5 * np.max(np.abs(want))


@pytest.mark.parametrize("scope_tag", ["E", "k"])
def test_layer_vs_float64_golden(tiny, scope_tag):
    """Whole layer against the committed float64 evaluation (f32 weights)."""
    t = tiny
    E, H = t["router"].shape
    I = t["gate_up"].shape[1] // 2
    Is = t["sh_gate"].shape[0]
    k = t["ids_E"].shape[1]
    scope = E if scope_tag == "E" else k
    cfg = _cfg(H, E, k, I, Is, scope)
    hw = _HW(cfg, router=t["router"], router_s=None, gate_up=t["gate_up"], gate_up_s=None, down=t["down"],
             down_s=None, sh_gate=t["sh_gate"], sh_gate_s=None, sh_up=t["sh_up"], sh_up_s=None,
             sh_down=t["sh_down"], sh_down_s=None, shared_gate=t["shared_gate"])
    out, ids, w = oracle.OracleLayer(hw).forward(t["x"])
    assert np.array_equal(ids, t[f"ids_{scope_tag}"])
    np.testing.assert_allclose(w, t[f"w_{scope_tag}"], rtol=1e-5)
    ref = t[f"out_{scope_tag}"]
    err = np.max(np.abs(out - ref), axis=1) / np.max(np.abs(ref), axis=1)
    assert err.max() < 1e-5


def test_layer_linearity_and_threads(tiny):
    """Zero routed experts leave sg * shared(x); a zero shared expert leaves
    the routed sum; thread count never changes a bit."""
    t = tiny
    E, H = t["router"].shape
    I = t["gate_up"].shape[1] // 2
    Is = t["sh_gate"].shape[0]
    k = t["ids_E"].shape[1]
    cfg = _cfg(H, E, k, I, Is, E)
    base = dict(router=t["router"], router_s=None, gate_up=t["gate_up"], gate_up_s=None, down=t["down"],
                down_s=None, sh_gate=t["sh_gate"], sh_gate_s=None, sh_up=t["sh_up"], sh_up_s=None,
                sh_down=t["sh_down"], sh_down_s=None, shared_gate=t["shared_gate"])
    x = t["x"]
    full, _, _ = oracle.OracleLayer(_HW(cfg, **base)).forward(x)
    no_routed, _, _ = oracle.OracleLayer(_HW(cfg, **{**base, "down": np.zeros_like(t["down"])})).forward(x)
    no_shared, _, _ = oracle.OracleLayer(_HW(cfg, **{**base, "sh_down": np.zeros_like(t["sh_down"])})).forward(x)
    xd = x.astype(np.float64)
    silu = lambda v: v / (1 + np.exp(-v))
    sh = (silu(xd @ t["sh_gate"].T.astype(np.float64)) * (xd @ t["sh_up"].T.astype(np.float64))) \
        @ t["sh_down"].T.astype(np.float64)
    sg = 1 / (1 + np.exp(-(xd @ t["shared_gate"].astype(np.float64))))
    assert np.max(np.abs(no_routed - sg[:, None] * sh)) < 1e-5 * np.max(np.abs(sh))
    assert np.max(np.abs(no_routed + no_shared - full)) < 1e-5 * np.max(np.abs(full))
    f8, _, _ = oracle.OracleLayer(_HW(cfg, **base), threads=8).forward(x)
    assert np.array_equal(bits32(f8), bits32(full))


# ------------------------------------------------- argmax and the norm

def go_argmax_brute(v):
    """The first index of the maximum over the non-NaN entries; 0 if v[0] is
    NaN or every entry is NaN (no comparison against a NaN best succeeds)."""
    if np.isnan(v[0]):
        return 0
    ok = ~np.isnan(v)
    m = v[ok].max()
    return int(np.flatnonzero(ok & (v == m))[0])


def test_argmax_known_answers_and_brute_force():
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    cases = [([1, 3, 3, 2], 1), ([nan, 5, 7], 0), ([1, nan, 2], 2), ([-0.0, 0.0], 0), ([0.0, -0.0], 0),
             ([-inf, -inf], 0), ([nan, nan], 0), ([2, nan, nan], 0), ([-1, -inf, inf, inf], 2), ([7], 0)]
    for v, want in cases:
        assert oracle.argmax(np.float32(v)) == want, v
    rng = np.random.default_rng(11)
    for _ in range(200):
        n = int(rng.integers(1, 300))
        v = rng.integers(-4, 5, n).astype(np.float32)  # many ties
        v[rng.random(n) < 0.1] = np.nan
        assert oracle.argmax(v) == go_argmax_brute(v)
        w = v[~np.isnan(v)]
        if w.size and not np.isnan(v[0]):
            assert oracle.argmax(v) == int(np.flatnonzero(~np.isnan(v))[np.argmax(w)])


def test_gemma_rmsnorm_exact_cases():
    # s = 16, s/n = 4, 1/sqrt(4) = 0.5: every step exact
    w = np.float32([0.0, 1.0, -0.5, 0.25])
    out = oracle.gemma_rmsnorm(np.float32([2, 2, 2, 2]), w, 0.0)
    assert np.array_equal(out, np.float32([1.0, 2.0, 0.5, 1.25]))
    # eps inside the mean: 4/4 + 3 = 4 -> inv 0.5 (eps added before the /n would give 1/sqrt(1.75))
    out = oracle.gemma_rmsnorm(np.float32([1, 1, 1, 1]), w, 3.0)
    assert np.array_equal(out, np.float32([0.5, 1.0, 0.25, 0.625]))
    # the sum of squares is f64: in f32, 1 + 2^-26 rounds back to 1 every time
    # and inv would be exactly 64; in f64 the 4095 small squares count
    x = np.full(4096, 2.0 ** -13, np.float32)
    x[0] = 1.0
    out = oracle.gemma_rmsnorm(x, np.zeros(4096, np.float32), 0.0)
    want = 64.0 / np.sqrt(1.0 + 4095 * 2.0 ** -26)
    assert out[0] < 64.0 and abs(out[0] - want) <= 2 * np.spacing(np.float32(want))


def test_gemma_rmsnorm_vs_float64():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(12)
    for n, eps, scale in [(2048, 1e-6, 1.0), (2048, 1e-6, 1e-3), (1024, 1e-5, 30.0), (64, 1e-2, 0.1)]:
        x = (rng.standard_normal((3, n)) * scale).astype(np.float32)
        w = (rng.standard_normal(n) * 0.3).astype(np.float32)
        got = oracle.gemma_rmsnorm(x, w, eps).astype(np.float64)
        t = torch.from_numpy(x.astype(np.float64))
        ref = torch.nn.functional.rms_norm(t, (n,), torch.from_numpy(1.0 + w.astype(np.float64)),
                                           eps=float(np.float32(eps))).numpy()
        # three f32 roundings (inv, x*inv, *(1+w)) plus the f32 rounding of 1+w
        tol = 4 * np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
        assert np.all(np.abs(got - ref) <= tol)
    # rows are independent
    x = rng.standard_normal((2, 256)).astype(np.float32)
    w = rng.standard_normal(256).astype(np.float32)
    both = oracle.gemma_rmsnorm(x, w, 1e-6)
    assert np.array_equal(both[1], oracle.gemma_rmsnorm(x[1], w, 1e-6))
