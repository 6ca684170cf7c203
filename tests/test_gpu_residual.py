"""GPU parity of the block with its neighbours: the post-attention
GemmaRMSNorm and the residual add of decodeLayers (model/model.go:506-517,
model/tensors.go:147-157) around the MoE block.

Bars:
  * the norm: bit for bit against the oracle's gemmaRMSNormApply, on the
    certified path and on the forced index-order path, including zero rows,
    huge and tiny magnitudes and a row with an infinity;
  * the residual step x + block(norm(x)): expert ids exact (they follow from
    the bit-exact norm), routing weights 1e-4 relative, and per token
    max_j (|x'_j - x'_ref_j| - 2^-23 |x'_ref_j|) / max_j |block_ref_j| within
    the block's own bar (1e-3 on the decode path, 2e-2 on the batched MFMA
    path) -- the 2^-23 |x'| is the f32 rounding of the final add, ours and the
    oracle's, which the block's bar does not cover;
  * the device entry in place (out = x) equals the host entry.
Every test prints the case it runs before touching the GPU.
"""
import numpy as np
import pytest

import oracle
import qmoe

pytestmark = pytest.mark.gpu

TOL_F32, TOL_MFMA = 1e-3, 2e-2


def announce(msg):
    print(f"[case] {msg}", flush=True)


def norm_weight(H, seed):
    return (np.random.default_rng(seed).standard_normal(H) * 0.2).astype(np.float32)


def residual_stream(cfg, T, seed):
    """Tokens with a realistic spread of row norms (the stream is not unit-scale)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, cfg.hidden), dtype=np.float32)
    return (x * rng.uniform(0.05, 20.0, (T, 1)).astype(np.float32)).astype(np.float32)


def check_residual(cfg, hw, x, eps=1e-6, seed=1):
    w = norm_weight(cfg.hidden, seed)
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        layer.set_post_norm(w, eps)
        got, ids, wts = layer.forward_residual(x)
        tol = TOL_MFMA if layer.forward_path(x.shape[0]) == qmoe.PATH_MFMA else TOL_F32
    finally:
        layer.close()
    ref, rids, rw, rout = oracle.OracleLayer(hw).forward_residual(x, w, eps)
    assert np.array_equal(ids, rids), f"ids differ at {np.argwhere(ids != rids)[:5]}"
    np.testing.assert_allclose(wts, rw, rtol=1e-4, atol=0)
    err = residual_err(got, ref, rout)
    assert err <= tol, f"relative error {err:.3e} > {tol}"
    return got


def residual_err(got, ref, rout):
    """The block's normwise error in x' = x + block, past the final f32 rounding."""
    d = np.abs(got.astype(np.float64) - ref) - 2.0 ** -23 * np.abs(ref.astype(np.float64))
    return (np.maximum(d, 0).max(axis=1) / np.maximum(np.abs(rout).max(axis=1), 1e-30)).max()


@pytest.mark.parametrize("seq", [False, True])
def test_norm_bit_exact(seq):
    cfg = qmoe.LayerConfig(2048, 8, 2, 64, 0, 0, qmoe.BF16, qmoe.BF16, qmoe.BF16, "norm")
    announce(f"norm bit-exact H=2048 index-order={seq}")
    hw = qmoe.synthetic_weights(cfg, 3, quantizer=oracle.host_quantizer)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((40, 2048), dtype=np.float32)
    x[1] = 0.0                                # s = 0: inv = 1/sqrt(eps)
    x[2] *= np.float32(1e18)                  # huge
    x[3] *= np.float32(1e-20)                 # tiny: eps dominates
    x[4, 7] = np.float32(np.inf)              # inf: inv = 0, inf * 0 = NaN
    x[5, :] = np.float32(3.0)                 # constant row
    x[6, 0] = np.float32(1.0)
    x[6, 1:] = np.float32(2.0 ** -13)         # the f64 sum matters (an f32 sum would stay at 1)
    w = norm_weight(2048, 5)
    for eps in (1e-6, 1e-5):
        layer = qmoe.MoeLayer(cfg)
        try:
            hw.upload(layer)
            layer.set_post_norm(w, eps)
            layer.set_norm_sequential(seq)
            got = layer.norm(x)
            redo = layer.norm_recomputes()
        finally:
            layer.close()
        ref = oracle.gemma_rmsnorm(x, w, eps)
        gb, rb = got.view(np.uint32), ref.view(np.uint32)
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(got), nan)
        bad = np.argwhere((gb != rb) & ~nan)
        assert bad.size == 0, f"{len(bad)} elements differ, first at {bad[:3]}"
        if seq:
            assert redo == x.shape[0]
        else:
            assert redo <= 2  # the inf row; the rest settle on the certified path


@pytest.mark.parametrize("T", [1, 8])
def test_residual_qwen3_bf16_decode(T):
    cfg = qmoe.CONFIGS["qwen3_30b_a3b"].with_(select_scope=128)
    announce(f"residual qwen3-30b-a3b bf16 T={T} scope=E")
    hw = qmoe.synthetic_weights(cfg, 310 + T, quantizer=oracle.host_quantizer)
    check_residual(cfg, hw, residual_stream(cfg, T, 310 + T))


def test_residual_qwen3_next_int4_decode():
    cfg = qmoe.CONFIGS["qwen3_next"].with_(select_scope=512)
    announce("residual qwen3-next int4g32 + shared T=1 and T=3")
    hw = qmoe.synthetic_weights(cfg, 320, quantizer=qmoe.device_quantizer)
    for T in (1, 3):
        check_residual(cfg, hw, residual_stream(cfg, T, 321 + T))


@pytest.mark.parametrize("fmts, T", [
    ((qmoe.F32, qmoe.F32, qmoe.F32, 0), 40),       # exact router, copy-initialised out
    ((qmoe.BF16, qmoe.BF16, qmoe.BF16, 64), 100),  # batched MFMA path: residual in the combine
    ((qmoe.BF16, qmoe.INT8G32, qmoe.BF16, 64), 5),
])
def test_residual_small_layers(fmts, T):
    rf, ef, sf, Is = fmts
    cfg = qmoe.LayerConfig(256, 16, 4, 128, Is, 16, rf, ef, sf, "res-small")
    announce(f"residual small layer fmts={fmts} T={T}")
    hw = qmoe.synthetic_weights(cfg, 330 + T, quantizer=oracle.host_quantizer)
    check_residual(cfg, hw, residual_stream(cfg, T, 330 + T))


@pytest.mark.parametrize("T", [1, 6, 70])
def test_residual_device_in_place(T):
    import torch
    cfg = qmoe.LayerConfig(512, 32, 4, 128, 128, 32, qmoe.BF16, qmoe.BF16, qmoe.BF16, "res-dev")
    announce(f"residual device entry in place T={T}")
    hw = qmoe.synthetic_weights(cfg, 340 + T, quantizer=oracle.host_quantizer)
    x = residual_stream(cfg, T, 340 + T)
    w = norm_weight(cfg.hidden, 9)
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        layer.set_post_norm(w, 1e-6)
        host, ids_h, _ = layer.forward_residual(x)
        dx = torch.from_numpy(x.copy()).cuda()
        ids = torch.empty((T, cfg.top_k), dtype=torch.int32, device="cuda")
        layer.forward_residual_device(dx.data_ptr(), T, dx.data_ptr(), ids.data_ptr(), None,
                                      torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        dev = dx.cpu().numpy()
        with pytest.raises(qmoe.QmoeError):
            qmoe.MoeLayer(cfg).forward_residual(x)  # no weights, no norm: state error
    finally:
        layer.close()
    assert np.array_equal(ids.cpu().numpy(), ids_h)
    ref, _, _, rout = oracle.OracleLayer(hw).forward_residual(x, w, 1e-6)
    tol = TOL_MFMA if T > 32 else TOL_F32
    for got in (host, dev):
        assert residual_err(got, ref, rout) <= tol


@pytest.mark.parametrize("T", [1, 8, 40])
def test_residual_forced_index_order(T):
    """The norm's index-order path in each place it runs: the decode kernel's
    prologue (T = 1), the certified router kernel (T = 8) and the norm kernel
    before the batched path (T = 40).  Same routing as the certified path, the
    same bar against the oracle, and every token counted once as recomputed."""
    cfg = qmoe.LayerConfig(2048, 64, 4, 256, 0, 64, qmoe.BF16, qmoe.BF16, qmoe.BF16, "res-seq")
    announce(f"residual forced index-order norm T={T}")
    hw = qmoe.synthetic_weights(cfg, 350 + T, quantizer=oracle.host_quantizer)
    x = residual_stream(cfg, T, 350 + T)
    w = norm_weight(cfg.hidden, 11)
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        layer.set_post_norm(w, 1e-6)
        cert, ids_c, _ = layer.forward_residual(x)
        before = layer.norm_recomputes()
        layer.set_norm_sequential(True)
        seq, ids_s, _ = layer.forward_residual(x)
        after = layer.norm_recomputes()
        tol = TOL_MFMA if layer.forward_path(T) == qmoe.PATH_MFMA else TOL_F32
    finally:
        layer.close()
    ref, rids, _, rout = oracle.OracleLayer(hw).forward_residual(x, w, 1e-6)
    assert np.array_equal(ids_c, rids) and np.array_equal(ids_s, rids)
    assert after - before == T
    for got in (cert, seq):
        assert residual_err(got, ref, rout) <= tol
