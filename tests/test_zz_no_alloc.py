"""qmoe_forward_device_noalloc against qmoe_forward_device (and the oracle).

Two calls in a row through the C ABI, the second with fewer tokens, each
compared with the allocating entry on the same inputs: ids and weights
bit-exact, outputs within 1e-5 normwise of each other (both run the same
kernels; only the order of the f32 atomics into out may differ) and within
the decode bar 1e-3 of the oracle.  Sizes past the scratch are refused.
"""
import numpy as np
import pytest

import oracle
import qmoe

pytestmark = pytest.mark.gpu


def rel_err(out, ref):
    return (np.abs(out - ref).max(axis=1) / np.maximum(np.abs(ref).max(axis=1), 1e-30)).max()


@pytest.mark.parametrize("key", ["qwen3_30b_a3b", "qwen3_next"])
def test_noalloc_matches_allocating_entry(key):
    import torch
    cfg = qmoe.CONFIGS[key]
    cfg = cfg.with_(select_scope=cfg.n_experts)
    print(f"[case] no-alloc entry vs qmoe_forward_device, {key}, T=12 then T=1", flush=True)
    quant = qmoe.device_quantizer if cfg.expert_fmt != qmoe.BF16 else oracle.host_quantizer
    hw = qmoe.synthetic_weights(cfg, 31337, quantizer=quant)
    x = qmoe.synthetic_tokens(cfg, 13, 31337)
    ref, rids, _ = oracle.OracleLayer(hw).forward(x)
    H, k = cfg.hidden, cfg.top_k
    st = torch.cuda.current_stream().cuda_stream
    layer = qmoe.MoeLayer(cfg)
    try:
        hw.upload(layer)
        for lo, T in ((0, 12), (12, 1)):
            dx = torch.from_numpy(np.ascontiguousarray(x[lo:lo + T])).cuda()
            outs, idss, wss = [], [], []
            for noalloc in (True, False):
                dout = torch.full((T, H), float("nan"), device="cuda")
                dids = torch.full((T, k), -1, dtype=torch.int32, device="cuda")
                dw = torch.full((T, k), float("nan"), device="cuda")
                fn = layer.forward_device_noalloc if noalloc else layer.forward_device
                fn(dx.data_ptr(), T, dout.data_ptr(), dids.data_ptr(), dw.data_ptr(), st)
                torch.cuda.synchronize()
                outs.append(dout.cpu().numpy())
                idss.append(dids.cpu().numpy())
                wss.append(dw.cpu().numpy())
            assert np.array_equal(idss[0], idss[1])
            assert np.array_equal(wss[0].view(np.uint32), wss[1].view(np.uint32))
            assert np.array_equal(idss[0], rids[lo:lo + T])
            assert rel_err(outs[0], outs[1]) <= 1e-5
            assert rel_err(outs[0], ref[lo:lo + T]) <= 1e-3
        dx = torch.zeros((33, H), device="cuda")
        dout = torch.zeros((33, H), device="cuda")
        with pytest.raises(qmoe.QmoeError) as ei:
            layer.forward_device_noalloc(dx.data_ptr(), 33, dout.data_ptr(), None, None, st)
        assert ei.value.status == 5
    finally:
        layer.close()
