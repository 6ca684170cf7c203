"""GPU parity: libqmoe.so (HIP, gfx950) against the CPU oracle.

Bars (written into each assertion):
  * expert ids: exact, in rank order (the router sums each logit sequentially
    in f32 exactly as model/moe.go does);
  * routing weights: 1e-4 relative (decode-sized T uses the certified router,
    whose weights come from f64 logits within its rounding bound of the
    reference's f32 logits; the exact path matches to the last bit of exp);
  * dequantised weights and device-quantised codes/scales: bit-exact;
  * layer output, normwise relative error max_j|y-y_ref| / max_j|y_ref| per
    token: <= 1e-3 on the decode (GEMV) path, f32 activations; <= 2e-2 on the
    batched MFMA path (x and the SwiGLU output in bf16, f32 accumulation).
Every test prints the case it runs before touching the GPU.
"""
import numpy as np
import pytest

import oracle
import qmoe

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3


def rel_err(out, ref):
    return (np.abs(out - ref).max(axis=1) / np.maximum(np.abs(ref).max(axis=1), 1e-30)).max()


def announce(msg):
    print(f"[case] {msg}", flush=True)


TOL_MFMA = 2e-2  # batched path: x and the SwiGLU output rounded to bf16, f32 accumulation


def path_tol(layer, T):
    """The parity bar of the kernels the library runs for T tokens."""
    return TOL_MFMA if layer.forward_path(T) == qmoe.PATH_MFMA else TOL_F32


def check_layer(cfg, hw, x, tol=None, scope=None):
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        out, ids, w = layer.forward(x)
        tol = tol or path_tol(layer, x.shape[0])
    finally:
        layer.close()
    ref, rids, rw = oracle.OracleLayer(hw, scope=scope).forward(x)
    assert np.array_equal(ids, rids), f"ids differ at {np.argwhere(ids != rids)[:5]}"
    np.testing.assert_allclose(w, rw, rtol=1e-4, atol=0)
    err = rel_err(out, ref)
    assert err <= tol, f"normwise relative error {err:.3e} > {tol}"
    return err


# ------------------------------------------------------------ quantiser

@pytest.mark.parametrize("bits", [8, 4])
def test_device_quantizer_bitexact(bits):
    import torch
    announce(f"device quantiser int{bits}")
    rng = np.random.default_rng(11 + bits)
    n_mat, rows, cols = 3, 40, 256
    w = (rng.standard_normal((n_mat, rows, cols), dtype=np.float32) * np.float32(0.02))
    w[0, 0, :32] = 0.0                      # amax 0 -> scale floored at 1e-8
    w[0, 1, :32] = np.float32(1e-12)        # tiny group
    # exact half-way points: w/s = k + 0.5 must round away from zero
    s = np.float32(1.0) / np.float32(127.0) if bits == 8 else np.float32(1.0) / np.float32(7.0)
    w[1, 2, :32] = 0.0
    w[1, 2, 0] = 1.0
    w[1, 2, 1] = np.float32(2.5) * s
    w[1, 2, 2] = -np.float32(2.5) * s
    codes_ref, scales_ref = oracle.quantize_f16(bits, w)
    dw = torch.from_numpy(w.reshape(-1).copy()).cuda()
    codes = torch.empty(codes_ref.size, dtype=torch.uint8, device="cuda")
    scales = torch.empty(scales_ref.size, dtype=torch.int16, device="cuda")
    qmoe.quantize_device(bits, dw.data_ptr(), n_mat, rows, cols, codes.data_ptr(), scales.data_ptr(),
                         torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    c = codes.cpu().numpy()
    assert np.array_equal(c, codes_ref.reshape(-1).view(np.uint8))
    assert np.array_equal(scales.cpu().numpy().view(np.uint16), scales_ref.reshape(-1))


@pytest.mark.parametrize("fmt", [qmoe.INT8G32, qmoe.INT4G32, qmoe.BF16, qmoe.F32])
def test_dequant_debug_bitexact(fmt):
    announce(f"dequant_debug fmt={qmoe.FORMAT_NAMES[fmt]}")
    cfg = qmoe.LayerConfig(256, 6, 2, 96, 64, 0, fmt, fmt, fmt, "dq")
    hw = qmoe.synthetic_weights(cfg, 5, quantizer=oracle.host_quantizer)
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        bits = 8 if fmt == qmoe.INT8G32 else 4

        def ref(w, s16, rows, cols):
            if fmt == qmoe.F32:
                return w.reshape(rows, cols)
            if fmt == qmoe.BF16:
                return qmoe.bf16_bits_to_f32(w).reshape(rows, cols)
            return oracle.dequantize(bits, w, oracle.f16_to_f32(s16), rows, cols)

        H, I, E, Is = cfg.hidden, cfg.moe_inter, cfg.n_experts, cfg.shared_inter
        for e in (0, E - 1):
            gu_s = hw.gate_up_s[e] if hw.gate_up_s is not None else None
            dn_s = hw.down_s[e] if hw.down_s is not None else None
            for which, w, s, rows, cols in ((0, hw.gate_up[e], gu_s, 2 * I, H), (1, hw.down[e], dn_s, H, I)):
                got = layer.dequant(which, e)
                assert np.array_equal(got.view(np.uint32), ref(w, s, rows, cols).view(np.uint32))
        cases = ((2, hw.router, hw.router_s, E, H), (3, hw.sh_gate, hw.sh_gate_s, Is, H),
                 (4, hw.sh_up, hw.sh_up_s, Is, H), (5, hw.sh_down, hw.sh_down_s, H, Is))
        for which, w, s, rows, cols in cases:
            got = layer.dequant(which)
            assert np.array_equal(got.view(np.uint32), ref(w, s, rows, cols).view(np.uint32))
    finally:
        layer.close()


@pytest.mark.parametrize("fmt", [qmoe.INT8G32_F32S, qmoe.INT4G32_F32S])
def test_dequant_debug_f32_scales_bitexact(fmt):
    """The reference's own quantised projections (qwen-quant writes F32
    scales, cmd/qwen-quant/main.go:207-210): router and shared expert with f32
    group scales.  Every stored matrix must equal quantLinear.dequantize with
    the unrounded f32 scales (the oracle's dequantize), bit for bit."""
    announce(f"dequant_debug f32 scales fmt={qmoe.FORMAT_NAMES[fmt]}")
    cfg = qmoe.LayerConfig(256, 6, 2, 96, 64, 0, fmt, fmt, fmt, "dq-f32s")
    hw = qmoe.synthetic_weights(cfg, 6, quantizer=oracle.host_quantizer)
    assert hw.router_s.dtype == np.float32 and hw.sh_gate_s.dtype == np.float32
    # the case that needs f32: scales that fp16 cannot hold exactly
    assert np.any(oracle.f16_to_f32(oracle.f32_to_f16(hw.router_s)) != hw.router_s)
    bits = 8 if fmt == qmoe.INT8G32_F32S else 4
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        H, I, E, Is = cfg.hidden, cfg.moe_inter, cfg.n_experts, cfg.shared_inter
        cases = [(0, e, hw.gate_up[e], hw.gate_up_s[e], 2 * I, H) for e in (0, E - 1)]
        cases += [(1, e, hw.down[e], hw.down_s[e], H, I) for e in (0, E - 1)]
        cases += [(2, 0, hw.router, hw.router_s, E, H), (3, 0, hw.sh_gate, hw.sh_gate_s, Is, H),
                  (4, 0, hw.sh_up, hw.sh_up_s, Is, H), (5, 0, hw.sh_down, hw.sh_down_s, H, Is)]
        for which, e, w, sc, rows, cols in cases:
            got = layer.dequant(which, e)
            ref = oracle.dequantize(bits, w, sc, rows, cols)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (which, e)
    finally:
        layer.close()


MIXED = [
    # (router, experts, shared): the reference's quantised checkpoints keep
    # bf16 experts and quantise the router / shared expert with f32 scales
    (qmoe.INT8G32_F32S, qmoe.BF16, qmoe.INT4G32_F32S),
    (qmoe.BF16, qmoe.BF16, qmoe.INT8G32_F32S),
    (qmoe.INT4G32_F32S, qmoe.INT4G32, qmoe.INT8G32_F32S),
    # fp16-scale shared expert in another format than the experts
    (qmoe.BF16, qmoe.BF16, qmoe.INT8G32),
    (qmoe.BF16, qmoe.INT4G32, qmoe.BF16),
    (qmoe.BF16, qmoe.INT8G32, qmoe.F32),
]


@pytest.mark.parametrize("fmts", MIXED, ids=lambda f: "-".join(map(str, f)))
@pytest.mark.parametrize("T", [1, 5, 100])
def test_f32_scale_and_mixed_formats(fmts, T):
    """Layers whose router, experts and shared expert use different formats,
    including the f32-scale group-32 formats: decode (T = 1, 5) and the
    batched path (T = 100), where the shared expert's GEMMs run in their own
    format and tile size (an f32 shared expert as a bf16 copy).  ids exact,
    weights 1e-4, output at the bar of the path."""
    rf, ef, sf = fmts
    cfg = qmoe.LayerConfig(256, 16, 4, 128, 128, 16, rf, ef, sf, "mixed")
    announce(f"mixed formats {fmts} T={T}")
    hw = qmoe.synthetic_weights(cfg, 700 + T, quantizer=oracle.host_quantizer)
    x = qmoe.synthetic_tokens(cfg, T, 700 + T)
    if T > 32:
        layer = qmoe.MoeLayer(cfg)
        try:
            assert layer.forward_path(T) == qmoe.PATH_MFMA
        finally:
            layer.close()
    check_layer(cfg, hw, x)


# --------------------------------------------------------------- layers

@pytest.mark.parametrize("scope", ["k", "E"])
def test_toy_layer(scope):
    cfg = qmoe.CONFIGS["toy"]
    if scope == "E":
        cfg = cfg.with_(select_scope=cfg.n_experts)
    announce(f"toy layer T=16 scope={scope}")
    hw = qmoe.synthetic_weights(cfg, 1, quantizer=oracle.host_quantizer)
    x = qmoe.synthetic_tokens(cfg, 16, 1)
    check_layer(cfg, hw, x)


SMALL = [
    # (router, experts, shared, shared_inter, scope)
    (qmoe.F32, qmoe.F32, qmoe.F32, 0, 0),
    (qmoe.BF16, qmoe.BF16, qmoe.BF16, 64, 0),
    (qmoe.BF16, qmoe.BF16, qmoe.BF16, 0, 16),
    (qmoe.INT8G32, qmoe.INT8G32, qmoe.INT4G32, 96, 12),
    (qmoe.INT4G32, qmoe.INT4G32, qmoe.INT8G32, 64, 16),
    (qmoe.F32, qmoe.INT4G32, qmoe.F32, 32, 16),
]


@pytest.mark.parametrize("fmts", SMALL, ids=lambda f: "-".join(map(str, f)))
@pytest.mark.parametrize("T", [1, 3, 16, 37])
def test_small_layers(fmts, T):
    """T <= 8: certified router + fused expert kernel (same shared format) or
    the separate kernels; 9..32: certified router + select + GEMVs; > 32:
    exact tiled router + GEMVs."""
    rf, ef, sf, Is, scope = fmts
    cfg = qmoe.LayerConfig(320, 16, 4, 160, Is, scope, rf, ef, sf, "small")
    announce(f"small layer fmts={fmts} T={T}")
    hw = qmoe.synthetic_weights(cfg, 100 + T, quantizer=oracle.host_quantizer)
    x = qmoe.synthetic_tokens(cfg, T, 100 + T)
    check_layer(cfg, hw, x)


@pytest.fixture(scope="module")
def qwen3_bf16():
    cfg = qmoe.CONFIGS["qwen3_30b_a3b"]
    return cfg, qmoe.synthetic_weights(cfg, 2026, quantizer=oracle.host_quantizer)


@pytest.mark.parametrize("T", [1, 8])
@pytest.mark.parametrize("scope", ["k", "E"])
def test_qwen3_30b_a3b_decode(qwen3_bf16, T, scope):
    cfg, hw = qwen3_bf16
    if scope == "E":
        cfg = cfg.with_(select_scope=cfg.n_experts)
        hw.cfg = cfg
    announce(f"qwen3-30b-a3b bf16 T={T} scope={scope}")
    x = qmoe.synthetic_tokens(cfg, T, 2026 + T)
    try:
        check_layer(cfg, hw, x)
    finally:
        hw.cfg = qmoe.CONFIGS["qwen3_30b_a3b"]


def test_qwen3_30b_a3b_int8_decode():
    cfg = qmoe.CONFIGS["qwen3_30b_a3b_int8"].with_(select_scope=128)
    announce("qwen3-30b-a3b int8g32 T=1 scope=E")
    hw = qmoe.synthetic_weights(cfg, 77, quantizer=qmoe.device_quantizer)
    x = qmoe.synthetic_tokens(cfg, 1, 77)
    check_layer(cfg, hw, x)


def test_qwen3_next_int4_decode():
    cfg = qmoe.CONFIGS["qwen3_next"].with_(select_scope=512)
    announce("qwen3-next int4g32 + shared T=1 scope=E")
    hw = qmoe.synthetic_weights(cfg, 99, quantizer=qmoe.device_quantizer)
    x = qmoe.synthetic_tokens(cfg, 2, 99)
    check_layer(cfg, hw, x)


def test_qwen3_next_int4_decode_T1():
    """T = 1: the expert kernel computes the router partials itself; 512
    experts put two router rows on some workgroups."""
    cfg = qmoe.CONFIGS["qwen3_next"].with_(select_scope=512)
    announce("qwen3-next int4g32 + shared T=1 scope=E, in-kernel router")
    hw = qmoe.synthetic_weights(cfg, 98, quantizer=qmoe.device_quantizer)
    x = qmoe.synthetic_tokens(cfg, 1, 98)
    check_layer(cfg, hw, x)


@pytest.mark.parametrize("fmts", [(qmoe.BF16, 512, 0), (qmoe.INT8G32, 1024, 64)], ids=["bf16-H512", "int8-H1024-shared"])
def test_decode_router_exchange_many_calls(fmts):
    """600 T = 1 calls on one handle: the tag of the exchanged router words
    wraps around (1..255) twice; every call's ids must equal the oracle's and
    its output stay within the decode bar."""
    ef, H, Is = fmts
    cfg = qmoe.LayerConfig(H, 16, 4, 128, Is, 16, qmoe.BF16, ef, ef, "exchange")
    announce(f"decode router exchange, 600 calls, fmts={fmts}")
    hw = qmoe.synthetic_weights(cfg, 600 + H, quantizer=oracle.host_quantizer)
    x = qmoe.synthetic_tokens(cfg, 600, 600 + H)
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        outs, idss = [], []
        for i in range(600):
            o, ids, _ = layer.forward(x[i:i + 1])
            outs.append(o)
            idss.append(ids)
    finally:
        layer.close()
    ref, rids, _ = oracle.OracleLayer(hw, scope=16).forward(x)
    ids = np.concatenate(idss)
    assert np.array_equal(ids, rids), f"ids differ at {np.argwhere(ids != rids)[:5]}"
    err = rel_err(np.concatenate(outs), ref)
    assert err <= TOL_F32, f"normwise relative error {err:.3e} > {TOL_F32}"


@pytest.mark.parametrize("rf,H,T,E", [(qmoe.F32, 288, 40, 128), (qmoe.INT8G32, 288, 40, 128),
                                       (qmoe.INT4G32, 288, 2100, 128), (qmoe.BF16, 320, 2100, 128),
                                       (qmoe.BF16, 288, 2100, 128), (qmoe.F32, 256, 70, 40),
                                       (qmoe.INT8G32, 512, 300, 72), (qmoe.BF16, 2048, 33, 128),
                                       (qmoe.INT4G32, 1024, 129, 24), (qmoe.INT8G32, 256, 8200, 128),
                                       (qmoe.INT4G32, 288, 8200, 128)])
def test_router_tile_shapes(rf, H, T, E):
    """The exact router for T > 32 in each of its tilings: 64-wide k slices
    (H a multiple of 64) with one output per lane below 32 experts (E=24), two
    below T x E = 2^20 (tails in T and E: T=70, E=40; T=300, E=72) and four
    from there (T=8200 x 128 experts, an int8 router: a bf16 one takes the
    certified path there); 32-wide slices (H=288) with one output per lane
    (T=40, 2100) or four (T=8200).  ids must equal the reference's exactly."""
    cfg = qmoe.LayerConfig(H, E, 8, 64, 0, E, rf, qmoe.BF16, qmoe.BF16, "router-tiles")
    announce(f"router tiles fmt={rf} H={H} T={T} E={E}")
    hw = qmoe.synthetic_weights(cfg, 7 + T, quantizer=oracle.host_quantizer)
    x = qmoe.synthetic_tokens(cfg, T, 7 + T)
    check_layer(cfg, hw, x)


BOUND_CASES = [
    # (hidden, experts, router fmt, T, router scale)
    (2048, 128, qmoe.BF16, 5, 1.0),
    (2048, 128, qmoe.BF16, 9, 4.0),
    (2048, 512, qmoe.BF16, 6, 4.0),
    (1024, 64, qmoe.INT8G32, 7, 1.0),
    (1024, 64, qmoe.INT4G32, 5, 1.0),
    (512, 32, qmoe.F32, 8, 1.0),
    # matrix-core partials (T > 32, bf16 router)
    (2048, 128, qmoe.BF16, 300, 4.0),
    (2048, 512, qmoe.BF16, 70, 4.0),
    (256, 64, qmoe.BF16, 40, 1.0),
    (4096, 96, qmoe.BF16, 33, 1.0),
]


@pytest.mark.parametrize("H,E,rf,T,rs", BOUND_CASES, ids=lambda v: str(v))
def test_router_bounds_contain_reference_logits(H, E, rf, T, rs):
    """Every reference logit (the sequential f32 matvec of model/tensors.go,
    computed by the oracle) lies in [S - B, S + B] of the certified decode
    router,
    for ordinary rows and for rows of zeros, huge, tiny and mixed magnitudes;
    and the bound is tight enough to be useful (median B below 1e-4 of the
    logits' spread for the f64 partials, 1e-3 for the matrix-core ones:
    closer pairs get exact logits)."""
    cfg = qmoe.LayerConfig(H, E, 8, 64, 0, E, rf, qmoe.BF16, qmoe.BF16, "bounds")
    announce(f"router bounds H={H} E={E} fmt={rf} T={T}")
    hw = qmoe.synthetic_weights(cfg, H + T, quantizer=oracle.host_quantizer, router_scale=rs)
    x = qmoe.synthetic_tokens(cfg, T, H + T)
    x[0] = 0.0
    x[1] *= 1e4
    x[2] *= 1e-20
    x[3, : H // 2] *= 1e3
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        sb = layer.router_bounds(x)
    finally:
        layer.close()
    scales = oracle.f16_to_f32(hw.router_s) if hw.router_s is not None else None
    L = np.stack([oracle.matvec(rf, hw.router, scales, x[t], E, H) for t in range(T)]).astype(np.float64)
    S, B = sb[..., 0], sb[..., 1]
    assert np.all(np.isfinite(S)) and np.all(B >= 0)
    dev = np.abs(L - S)
    assert np.all(dev <= B), f"bound violated at {np.argwhere(dev > B)[:5]}, worst {np.max(dev - B):.3e}"
    spread = np.median(np.std(L[4:], axis=1))
    print(f"median B {np.median(B[4:]):.3e}, median |L - S| {np.median(dev[4:]):.3e}, logit spread {spread:.3f}")
    # f64 partials (T <= 32) are within 1e-4 of the spread, the matrix-core ones within 1e-3
    assert np.median(B[4:]) < (1e-4 if T <= 32 else 1e-3) * spread, (np.median(B[4:]), spread)


@pytest.mark.parametrize("T", [1, 5, 12])
def test_router_near_tie_rescue(T):
    """Two router rows one bf16 ulp apart at their largest weight, where x is
    +-1: their logits differ by ~1e-4, inside the certified bound at H=2048
    (~2e-3) but far above the tie margin.  The first certification fails; exact logits of the
    candidates in doubt settle it without the full exact path, and the order
    must be the reference's."""
    cfg = qmoe.LayerConfig(2048, 128, 8, 64, 0, 128, qmoe.BF16, qmoe.BF16, qmoe.BF16, "near-tie")
    announce(f"router near-tie rescue T={T}")
    hw = qmoe.synthetic_weights(cfg, 77, quantizer=oracle.host_quantizer)
    r = hw.router.copy()
    h0 = int(np.argmax(np.abs(qmoe.bf16_bits_to_f32(r[3]))))  # the largest weight: the widest ulp
    r[5] = r[3]
    r[5, h0] = r[3, h0] + 1  # one ulp further from zero
    hw.router = r
    x = qmoe.synthetic_tokens(cfg, T, 77)
    w3 = qmoe.bf16_bits_to_f32(r[3]).astype(np.float32)
    w2 = qmoe.bf16_bits_to_f32(r[2]).astype(np.float32)
    x = (x + 40.0 * w3 + 38.0 * w2).astype(np.float32)
    x[:, h0] = np.sign(w3[h0]) or 1.0
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        out, ids, w = layer.forward(x)
        fb, rescued = layer.router_fallbacks(), layer.router_rescues()
    finally:
        layer.close()
    ref, rids, rw = oracle.OracleLayer(hw).forward(x)
    assert np.array_equal(ids, rids), (ids, rids)
    assert set(ids[0][:2]) == {3, 5}, ids[0]
    np.testing.assert_allclose(w, rw, rtol=1e-4, atol=0)
    assert rel_err(out, ref) <= TOL_F32
    assert rescued == T and fb == 0, (rescued, fb)


@pytest.mark.parametrize("T", [1, 5, 40])
def test_router_exact_ties(T):
    """Identical router rows give exactly equal logits; the reference breaks the
    tie by the lower expert index.  The certified path cannot certify such a
    gap and must fall back to the exact sequential path in-kernel."""
    cfg = qmoe.LayerConfig(256, 16, 4, 64, 0, 16, qmoe.BF16, qmoe.BF16, qmoe.BF16, "ties")
    announce(f"router exact ties T={T}")
    hw = qmoe.synthetic_weights(cfg, 31, quantizer=oracle.host_quantizer)
    r = hw.router.copy()
    r[5] = r[3]           # 3 and 5 tie, 3 must rank first
    r[9] = r[12] = r[2]   # three-way tie 2 < 9 < 12
    hw.router = r
    x = qmoe.synthetic_tokens(cfg, T, 31)
    # make the tied experts win: align x with their rows
    w3 = qmoe.bf16_bits_to_f32(r[3]).astype(np.float32)
    w2 = qmoe.bf16_bits_to_f32(r[2]).astype(np.float32)
    x = (x + 40.0 * w3 + 38.0 * w2).astype(np.float32)
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        out, ids, w = layer.forward(x)
        fb = layer.router_fallbacks()
        tol = path_tol(layer, T)
    finally:
        layer.close()
    ref, rids, rw = oracle.OracleLayer(hw).forward(x)
    assert np.array_equal(ids, rids), (ids, rids)
    # the leading ranks are a tied group, listed in ascending index order
    assert list(ids[0][:2]) in ([3, 5], [2, 9]), ids[0]
    assert rel_err(out, ref) <= tol
    if T <= 32:
        assert fb >= T  # every token hit a tie, which only the exact path settles


@pytest.mark.parametrize("scope_tag", ["E", "k"])
def test_golden_tiny_layer(scope_tag):
    """The committed float64 evaluation (tests/golden/tiny_layer.npz, f32
    weights, shared expert): ids exact, output within 1e-3 normwise."""
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny_layer.npz")
    with np.load(path) as z:
        t = {k: z[k] for k in z.files}
    E, H = t["router"].shape
    I, Is, k = t["gate_up"].shape[1] // 2, t["sh_gate"].shape[0], t["ids_E"].shape[1]
    scope = E if scope_tag == "E" else k
    announce(f"golden tiny layer scope={scope_tag}")
    cfg = qmoe.LayerConfig(H, E, k, I, Is, scope, qmoe.F32, qmoe.F32, qmoe.F32, "golden")
    hw = qmoe.HostWeights(cfg, t["router"], None, t["gate_up"], None, t["down"], None, t["sh_gate"], None,
                          t["sh_up"], None, t["sh_down"], None, t["shared_gate"])
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        out, ids, w = layer.forward(t["x"])
    finally:
        layer.close()
    assert np.array_equal(ids, t[f"ids_{scope_tag}"])
    np.testing.assert_allclose(w, t[f"w_{scope_tag}"], rtol=1e-5)
    assert rel_err(out, t[f"out_{scope_tag}"]) <= TOL_F32


# ------------------------------------------------- batched (MFMA) path


def check_mfma_layer(cfg, hw, x, scope=None):
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        assert layer.forward_path(x.shape[0]) == qmoe.PATH_MFMA
        out, ids, w = layer.forward(x)
    finally:
        layer.close()
    ref, rids, rw = oracle.OracleLayer(hw, scope=scope, threads=8).forward(x)
    assert np.array_equal(ids, rids), f"ids differ at {np.argwhere(ids != rids)[:5]}"
    np.testing.assert_allclose(w, rw, rtol=1e-6, atol=0)
    err = rel_err(out, ref)
    assert err <= TOL_MFMA, f"normwise relative error {err:.3e} > {TOL_MFMA}"
    return out, ids, err


PREFILL = [
    # (router fmt, expert and shared fmt, shared_inter, scope)
    (qmoe.BF16, qmoe.BF16, 0, 0),
    (qmoe.BF16, qmoe.BF16, 128, 16),
    (qmoe.F32, qmoe.BF16, 128, 0),
    (qmoe.BF16, qmoe.INT8G32, 0, 0),
    (qmoe.BF16, qmoe.INT8G32, 128, 16),
    (qmoe.F32, qmoe.INT4G32, 128, 0),
    (qmoe.BF16, qmoe.INT4G32, 128, 16),
]


@pytest.mark.parametrize("fmts", PREFILL, ids=lambda f: "-".join(map(str, f)))
@pytest.mark.parametrize("T", [33, 100, 300])
def test_prefill_layers(fmts, T):
    """Batched path for bf16, int8 and int4 experts (the INT formats are
    dequantised to bf16 inside the GEMMs)."""
    rf, ef, Is, scope = fmts
    cfg = qmoe.LayerConfig(256, 16, 4, 128, Is, scope, rf, ef, ef, "prefill")
    announce(f"prefill layer fmts={fmts} T={T}")
    hw = qmoe.synthetic_weights(cfg, 300 + T, quantizer=oracle.host_quantizer)
    x = qmoe.synthetic_tokens(cfg, T, 300 + T)
    check_mfma_layer(cfg, hw, x)


def test_prefill_skewed_routing():
    """One expert takes most tokens (several tiles), most take none."""
    cfg = qmoe.LayerConfig(256, 16, 2, 128, 128, 16, qmoe.BF16, qmoe.BF16, qmoe.BF16, "skew")
    announce("prefill skewed routing T=400")
    hw = qmoe.synthetic_weights(cfg, 41, quantizer=oracle.host_quantizer, router_scale=4.0)
    x = qmoe.synthetic_tokens(cfg, 400, 41)
    r = qmoe.bf16_bits_to_f32(hw.router).reshape(16, 256).astype(np.float32)
    x = (x + 3.0 * r[5] / np.linalg.norm(r[5]) * np.sqrt(256)).astype(np.float32)
    out, ids, _ = check_mfma_layer(cfg, hw, x)
    counts = np.bincount(ids.reshape(-1), minlength=16)
    assert counts.max() > 256, counts  # the hot expert spans several tiles


def test_prefill_qwen3_shape_rows_are_independent():
    """Qwen3-30B-A3B shape: T=64 against the oracle, then T=2048 (sharpened
    router) whose first 64 rows must equal the T=64 result bit for bit -- each
    token's output depends on its own row only, whatever the dispatch order."""
    cfg = qmoe.CONFIGS["qwen3_30b_a3b"].with_(select_scope=128)
    announce("prefill qwen3-30b-a3b bf16 T=64 vs oracle, T=2048 row independence")
    hw = qmoe.synthetic_weights(cfg, 2048, quantizer=oracle.host_quantizer, router_scale=4.0)
    x = qmoe.synthetic_tokens(cfg, 2048, 2048)
    out64, ids64, _ = check_mfma_layer(cfg, hw, x[:64])
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        out, ids, w = layer.forward(x)
        perm = np.random.default_rng(1).permutation(2048)
        outp, idsp, _ = layer.forward(np.ascontiguousarray(x[perm]))
    finally:
        layer.close()
    assert np.array_equal(ids[:64], ids64)
    assert np.array_equal(out[:64].view(np.uint32), out64.view(np.uint32))
    assert np.array_equal(idsp, ids[perm])
    assert np.array_equal(outp.view(np.uint32), out[perm].view(np.uint32))
    assert np.all(np.isfinite(out))


def test_prefill_qwen3_bench_input_full_size():
    """The input that bench.py --workload prefill times: the Qwen3-30B-A3B
    layer (bf16, seed 2026) with the router x4 and tokens skewed so that the
    busiest expert takes about 10x the median load, T=2048, top-8 of 128.
    Every token's ids (exact) and weights (1e-6) against the oracle's router,
    and 64 rows strided across the whole batch against the full oracle at the
    MFMA bar."""
    cfg = qmoe.CONFIGS["qwen3_30b_a3b"].with_(select_scope=128)
    announce("prefill qwen3-30b-a3b bf16 T=2048, the bench's skewed input, all ids + strided rows vs oracle")
    hw = qmoe.synthetic_weights(cfg, 2026, quantizer=oracle.host_quantizer, router_scale=4.0)
    x, stats = qmoe.skewed_tokens(cfg, hw, 2048, 2026 + 1000, 10.0)
    assert stats["max_load"] >= 5 * stats["median_load"], stats
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        assert layer.forward_path(2048) == qmoe.PATH_MFMA
        out, ids, w = layer.forward(x)
    finally:
        layer.close()
    ol = oracle.OracleLayer(hw, threads=8)
    _, rids, rw = ol.router(x)
    assert np.array_equal(ids, rids), f"ids differ at {np.argwhere(ids != rids)[:5]}"
    np.testing.assert_allclose(w, rw, rtol=1e-6, atol=0)
    rows = np.arange(0, 2048, 32)
    ref, _, _ = ol.forward(x[rows])
    err = rel_err(out[rows], ref)
    assert err <= TOL_MFMA, f"normwise relative error {err:.3e} > {TOL_MFMA}"
    assert np.all(np.isfinite(out))


def test_prefill_qwen3_first_k_full_size():
    """The input that bench.py --workload prefill_firstk times: the
    Qwen3-30B-A3B layer with the reference's own selection (scope = k = 8),
    so every token goes to experts 0..7 in its own order, T=2048.  These
    tile counts are known on the host, which runs the gate_up GEMM on half
    tiles (768 items instead of 384 on 256 CUs).  Every token's ids (exact)
    and weights (1e-6) against the oracle's router, and 64 rows strided
    across the batch against the full oracle at the MFMA bar."""
    cfg = qmoe.CONFIGS["qwen3_30b_a3b"].with_(select_scope=8)
    announce("prefill qwen3-30b-a3b bf16 T=2048 scope=k, all ids + strided rows vs oracle")
    hw = qmoe.synthetic_weights(cfg, 2026, quantizer=oracle.host_quantizer)
    x = qmoe.synthetic_tokens(cfg, 2048, 2026 + 1000)
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        out, ids, w = layer.forward(x)
    finally:
        layer.close()
    ol = oracle.OracleLayer(hw, scope=8, threads=8)
    _, rids, rw = ol.router(x)
    assert np.array_equal(ids, rids), f"ids differ at {np.argwhere(ids != rids)[:5]}"
    assert np.array_equal(np.sort(ids, axis=1), np.tile(np.arange(8), (2048, 1)))
    np.testing.assert_allclose(w, rw, rtol=1e-6, atol=0)
    rows = np.arange(5, 2048, 32)
    ref, _, _ = ol.forward(x[rows])
    err = rel_err(out[rows], ref)
    assert err <= TOL_MFMA, f"normwise relative error {err:.3e} > {TOL_MFMA}"
    assert np.all(np.isfinite(out))


def test_prefill_long_prompt_chunked():
    """An 8192-token prompt at k=8: 65536 (token, rank) pairs, more than the
    batched path's slot tables hold, so the forward runs in chunks.  Every
    token's ids (exact) and weights (1e-6) against the oracle's router, 64
    rows strided across all chunks against the full oracle at the MFMA bar,
    and the rows of the last chunk equal to a separate forward of those
    tokens bit for bit."""
    cfg = qmoe.CONFIGS["qwen3_30b_a3b"].with_(select_scope=128)
    announce("prefill qwen3-30b-a3b bf16 T=8192 k=8 (chunked), all ids + strided rows vs oracle")
    hw = qmoe.synthetic_weights(cfg, 8192, quantizer=oracle.host_quantizer)
    x = qmoe.synthetic_tokens(cfg, 8192, 8192)
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        out, ids, w = layer.forward(x)
        tail, tail_ids, _ = layer.forward(np.ascontiguousarray(x[8000:]))
    finally:
        layer.close()
    ol = oracle.OracleLayer(hw, threads=8)
    _, rids, rw = ol.router(x)
    assert np.array_equal(ids, rids), f"ids differ at {np.argwhere(ids != rids)[:5]}"
    np.testing.assert_allclose(w, rw, rtol=1e-6, atol=0)
    rows = np.arange(0, 8192, 128)
    ref, _, _ = ol.forward(x[rows])
    assert rel_err(out[rows], ref) <= TOL_MFMA
    assert np.array_equal(tail_ids, ids[8000:])
    assert np.array_equal(tail.view(np.uint32), out[8000:].view(np.uint32))


def test_batched_certified_router_reference_scope():
    """T x E = 2^20 with the reference's own selection (scope = k = 10 of 512)
    and a sharpened router (x4): the matrix-core router's candidates must size
    their roundings from the maximum over all 512 logits, which lies outside
    the scope for most tokens.  ids exact and weights within 1e-6 of the
    oracle's router for every token; strided rows of the output at the MFMA
    bar."""
    cfg = qmoe.LayerConfig(2048, 512, 10, 128, 0, 10, qmoe.BF16, qmoe.BF16, qmoe.BF16, "cert-scope-k")
    announce("batched certified router, scope=k=10 of 512, router x4, T=2048")
    hw = qmoe.synthetic_weights(cfg, 4242, quantizer=oracle.host_quantizer, router_scale=4.0)
    x = qmoe.synthetic_tokens(cfg, 2048, 4242)
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        assert layer.forward_path(2048) == qmoe.PATH_MFMA
        out, ids, w = layer.forward(x)
    finally:
        layer.close()
    ol = oracle.OracleLayer(hw, threads=8)
    probs, rids, rw = ol.router(x)
    assert np.array_equal(ids, rids), f"ids differ at {np.argwhere(ids != rids)[:5]}"
    np.testing.assert_allclose(w, rw, rtol=1e-6, atol=0)
    # the case this covers: the largest probability lies outside the scope
    assert np.mean(np.argmax(probs, axis=1) >= 10) > 0.9
    rows = np.arange(0, 2048, 64)
    ref, _, _ = ol.forward(x[rows])
    assert rel_err(out[rows], ref) <= TOL_MFMA


@pytest.mark.parametrize("key,T_small,T_full", [("qwen3_30b_a3b_int8", 64, 512), ("qwen3_next", 48, 4096)])
def test_prefill_quantized_shapes(key, T_small, T_full):
    """Qwen3-30B-A3B int8 experts (T=512) and the Qwen3-Next int4 layer with its
    int4 shared expert (T=4096): T_small tokens against the oracle, then the
    full batch, whose routing must equal the oracle's (ids exact, weights
    1e-6) and whose first T_small rows must equal the small batch's -- bit
    for bit when both batches route the same way; T=4096 x 512 experts takes
    the matrix-core partials and exact candidate logits, whose weights may
    differ from the exact softmax's in the last bits -- and a permuted full
    batch, whose rows must follow the permutation bit for bit."""
    cfg = qmoe.CONFIGS[key]
    cfg = cfg.with_(select_scope=cfg.n_experts)
    announce(f"prefill {key} T={T_small} vs oracle, T={T_full} row independence")
    hw = qmoe.synthetic_weights(cfg, T_full, quantizer=qmoe.device_quantizer)
    x = qmoe.synthetic_tokens(cfg, T_full, T_full)
    out_s, ids_s, _ = check_mfma_layer(cfg, hw, x[:T_small])
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        out, ids, w = layer.forward(x)
        perm = np.random.default_rng(2).permutation(T_full)
        outp, idsp, _ = layer.forward(np.ascontiguousarray(x[perm]))
    finally:
        layer.close()
    assert np.array_equal(ids[:T_small], ids_s)
    _, rids, rw = oracle.OracleLayer(hw).router(x)
    assert np.array_equal(ids, rids), f"ids differ at {np.argwhere(ids != rids)[:5]}"
    np.testing.assert_allclose(w, rw, rtol=1e-6, atol=0)
    if T_full * cfg.n_experts < (1 << 20):
        assert np.array_equal(out[:T_small].view(np.uint32), out_s.view(np.uint32))
    else:
        # the weighted expert rows are rounded to bf16: a last-bit weight
        # difference can move an element by one bf16 ulp (2^-8 relative)
        assert rel_err(out[:T_small], out_s) <= 2.0 ** -8
    assert np.array_equal(idsp, ids[perm])
    assert np.array_equal(outp.view(np.uint32), out[perm].view(np.uint32))
    assert np.all(np.isfinite(out))


def test_batched_router_candidates_ties():
    """2048 tokens x 512 experts (the size from which the batched path routes
    with the matrix-core partials): rows one bf16 ulp apart (near tie, settled
    by the exact candidate logits) and identical rows (exact tie, lower index
    first; ties between ranks are ordered by index without the exact path).
    ids and weights against the oracle's router for every token."""
    cfg = qmoe.LayerConfig(2048, 512, 8, 64, 0, 512, qmoe.BF16, qmoe.BF16, qmoe.BF16, "cand-ties")
    announce("batched router candidates, ties, T=2048 E=512")
    # unsharpened router: the tied experts' logits (~33) stay within 80 of the
    # others, so no probability underflows (that case takes the exact path)
    hw = qmoe.synthetic_weights(cfg, 91, quantizer=oracle.host_quantizer)
    r = hw.router.copy()
    h0 = int(np.argmax(np.abs(qmoe.bf16_bits_to_f32(r[3]))))
    r[5] = r[3]
    r[5, h0] = r[3, h0] + 1
    r[9] = r[2]
    hw.router = r
    x = qmoe.synthetic_tokens(cfg, 2048, 91)
    w3 = qmoe.bf16_bits_to_f32(r[3]).astype(np.float32)
    w2 = qmoe.bf16_bits_to_f32(r[2]).astype(np.float32)
    x[::2] = (x[::2] + 40.0 * w3 + 38.0 * w2).astype(np.float32)  # half the tokens pick the tied rows
    x[::2, h0] = np.sign(w3[h0]) or 1.0
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        out, ids, w = layer.forward(x)
        fb = layer.router_fallbacks()
    finally:
        layer.close()
    _, rids, rw = oracle.OracleLayer(hw).router(x)
    assert np.array_equal(ids, rids), f"ids differ at {np.argwhere(ids != rids)[:5]}"
    np.testing.assert_allclose(w, rw, rtol=1e-6, atol=0)
    assert list(ids[0][:4]) == [5, 3, 2, 9], ids[0]
    assert fb == 0, fb


def test_batched_router_exact_queue():
    """2048 tokens x 512 experts with one router row scaled by 100: for many
    tokens that expert's logit lies more than 80 above the other selected
    ones, whose probabilities then underflow, which only the exact path
    settles.  Those tokens are queued; the first 64 are routed by workgroups
    that each take a share of the experts, the rest whole by one workgroup.
    ids and weights against the oracle's router for every token."""
    cfg = qmoe.LayerConfig(2048, 512, 8, 64, 0, 512, qmoe.BF16, qmoe.BF16, qmoe.BF16, "exact-queue")
    announce("batched router exact queue, T=2048 E=512, one row x100")
    hw = qmoe.synthetic_weights(cfg, 93, quantizer=oracle.host_quantizer)
    r = qmoe.bf16_bits_to_f32(hw.router).reshape(512, 2048)
    r[7] *= 100.0
    hw.router = qmoe.f32_to_bf16_bits(r.reshape(-1)).reshape(hw.router.shape)
    x = qmoe.synthetic_tokens(cfg, 2048, 93)
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        out, ids, w = layer.forward(x)
        fb = layer.router_fallbacks()
    finally:
        layer.close()
    _, rids, rw = oracle.OracleLayer(hw, threads=8).router(x)
    assert np.array_equal(ids, rids), f"ids differ at {np.argwhere(ids != rids)[:5]}"
    np.testing.assert_allclose(w, rw, rtol=1e-6, atol=0)
    assert fb > 64, fb
    assert np.all(np.isfinite(out))


def test_decode_exchange_timeout_fails_that_call():
    """The T = 1 kernel's workgroups exchange router partials with a bounded
    wait.  With the wait budget set to zero from the host, every wait gives up
    at once (each workgroup still finishes, on exact routing): the synchronous
    call that hit it must fail, and the handle must work again afterwards.  An
    asynchronous call's timeout is reported by the next call, once."""
    import torch
    cfg = qmoe.LayerConfig(512, 16, 4, 128, 0, 16, qmoe.BF16, qmoe.BF16, qmoe.BF16, "timeout")
    announce("decode exchange timeout forced from the host (zero wait budget)")
    hw = qmoe.synthetic_weights(cfg, 515, quantizer=oracle.host_quantizer)
    x = qmoe.synthetic_tokens(cfg, 4, 515)
    ref, rids, _ = oracle.OracleLayer(hw).forward(x)
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        out, ids, _ = layer.forward(x[0:1])
        assert np.array_equal(ids, rids[0:1])
        layer.set_exchange_budget(0)
        with pytest.raises(qmoe.QmoeError) as ei:
            layer.forward(x[1:2])
        assert ei.value.status == 4
        layer.set_exchange_budget(-1)
        out, ids, _ = layer.forward(x[2:3])
        assert np.array_equal(ids, rids[2:3])
        assert rel_err(out, ref[2:3]) <= TOL_F32
        # asynchronous entry
        st = torch.cuda.current_stream().cuda_stream
        dx = torch.from_numpy(np.ascontiguousarray(x[3:4])).cuda()
        dout = torch.empty_like(dx)
        layer.set_exchange_budget(0)
        layer.forward_device(dx.data_ptr(), 1, dout.data_ptr(), None, None, st)
        torch.cuda.synchronize()
        layer.set_exchange_budget(-1)
        with pytest.raises(qmoe.QmoeError) as ei:
            layer.forward_device(dx.data_ptr(), 1, dout.data_ptr(), None, None, st)
        assert ei.value.status == 4
        layer.forward_device(dx.data_ptr(), 1, dout.data_ptr(), None, None, st)
        torch.cuda.synchronize()
        assert rel_err(dout.cpu().numpy(), ref[3:4]) <= TOL_F32
    finally:
        layer.close()


# ----------------------------------------------------------- contract

def test_contract_errors():
    announce("C ABI error paths")
    cfg = qmoe.LayerConfig(256, 8, 2, 64, 0, 0, qmoe.BF16, qmoe.BF16, qmoe.BF16, "errs")
    layer = qmoe.MoeLayer(cfg)
    try:
        x = np.zeros((1, 256), np.float32)
        with pytest.raises(qmoe.QmoeError) as ei:
            layer.forward(x)  # no weights yet
        assert ei.value.status == 2
        hw = qmoe.synthetic_weights(cfg, 1, quantizer=oracle.host_quantizer)
        hw.upload(layer)
        out, ids, w = layer.forward(np.zeros((0, 256), np.float32))
        assert out.shape == (0, 256)
        st = layer.lib.qmoe_forward(layer.h, None, 1, None, None, None)
        assert st == 1
        with pytest.raises(qmoe.QmoeError):
            layer.set_shared(None, None, None, None, None, None, None)
        with pytest.raises(qmoe.QmoeError):
            layer.dequant(0, 99)
    finally:
        layer.close()
    layer.close()  # idempotent


def test_reserve_sizes_the_workspace_up_front():
    """qmoe_reserve(max_T): later calls of up to max_T tokens allocate nothing
    (the handle's device bytes stay put) and still match the oracle."""
    cfg = qmoe.LayerConfig(256, 16, 4, 128, 64, 16, qmoe.BF16, qmoe.BF16, qmoe.BF16, "reserve")
    announce("reserve T=300 then forwards of T=1, 40, 300")
    hw = qmoe.synthetic_weights(cfg, 61, quantizer=oracle.host_quantizer)
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        before = layer.device_bytes()
        layer.reserve(300)
        reserved = layer.device_bytes()
        assert reserved > before
        for T in (1, 40, 300):
            x = qmoe.synthetic_tokens(cfg, T, 61 + T)
            out, ids, _ = layer.forward(x)
            assert layer.device_bytes() == reserved
            ref, rids, _ = oracle.OracleLayer(hw).forward(x)
            assert np.array_equal(ids, rids)
            assert rel_err(out, ref) <= path_tol(layer, T)
    finally:
        layer.close()
