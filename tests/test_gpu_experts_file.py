"""Packed experts end to end on the GPU: a bf16 checkpoint's stacked experts
quantised on the device into .qweight / .scale, read back, uploaded as they
are, and the layer run.  Bars: codes and fp16 scales bit-exact against the
oracle's quantizeInt8 / quantizeInt4 (model/moe.go:165-217) of the same
bf16-widened weights; expert ids exact, weights 1e-4, output 1e-3 (decode) /
2e-2 (batched) against the oracle fed the same codes and scales.
Every test prints the case it runs before touching the GPU."""
import numpy as np
import pytest

import experts_file as ef
import oracle
import qmoe

pytestmark = pytest.mark.gpu


def announce(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("bits, T", [(8, 1), (4, 3), (8, 48)])
def test_packed_experts_end_to_end(tmp_path, bits, T):
    import torch
    from safetensors.torch import save_file
    fmt = qmoe.INT8G32 if bits == 8 else qmoe.INT4G32
    cfg = qmoe.LayerConfig(256, 16, 4, 128, 0, 16, qmoe.BF16, fmt, qmoe.BF16, "packed")
    announce(f"packed experts int{bits} T={T}")
    rng = np.random.default_rng(40 + bits)
    H, E, I = cfg.hidden, cfg.n_experts, cfg.moe_inter
    gu = torch.from_numpy(rng.standard_normal((E, 2 * I, H), dtype=np.float32) * 0.02).to(torch.bfloat16)
    dn = torch.from_numpy(rng.standard_normal((E, H, I), dtype=np.float32) * 0.02).to(torch.bfloat16)
    router = torch.from_numpy(rng.standard_normal((E, H), dtype=np.float32) * 0.05).to(torch.bfloat16)
    src = tmp_path / "src"
    src.mkdir()
    save_file({"model.layers.0.mlp.experts.gate_up_proj.weight": gu,
               "model.layers.0.mlp.experts.down_proj.weight": dn,
               "model.layers.0.mlp.gate.weight": router}, str(src / "model.safetensors"))
    out = tmp_path / "q"
    ef.quantize_checkpoint(str(src), str(out), bits)
    qx = ef.read_layer_experts(str(out), "model.layers.0.")
    # bit-exact against the oracle's quantiser on the same widened weights
    for codes, scales, w in ((qx.gate_up, qx.gate_up_scales, gu), (qx.down, qx.down_scales, dn)):
        rc, rs = oracle.quantize_f16(bits, w.float().numpy())
        assert np.array_equal(codes.view(np.uint8), rc.view(np.uint8))
        assert np.array_equal(scales, rs)
    # the layer from the file: router bf16 as stored, experts as stored
    hw = qmoe.HostWeights(cfg, router.view(torch.int16).numpy().view(np.uint16), None,
                          np.ascontiguousarray(qx.gate_up), np.ascontiguousarray(qx.gate_up_scales),
                          np.ascontiguousarray(qx.down), np.ascontiguousarray(qx.down_scales))
    x = qmoe.synthetic_tokens(cfg, T, 41)
    layer = qmoe.MoeLayer(cfg)
    try:
        layer.set_router(hw.router)
        qx.upload(layer)
        got, ids, w = layer.forward(x)
        tol = 2e-2 if layer.forward_path(T) == qmoe.PATH_MFMA else 1e-3
    finally:
        layer.close()
    ref, rids, rw = oracle.OracleLayer(hw).forward(x)
    assert np.array_equal(ids, rids)
    np.testing.assert_allclose(w, rw, rtol=1e-4, atol=0)
    err = (np.abs(got - ref).max(axis=1) / np.abs(ref).max(axis=1)).max()
    assert err <= tol, err
