"""The packed-experts file format without a GPU: the streaming writer's output
read back by the safetensors library (an independent reader), passthrough
tensors byte-identical, packed tensors with the documented dtypes and shapes,
and the product reader returning exactly what was written.  The codes here are
arbitrary data: the quantiser itself is checked on the GPU."""
import json
import os

import numpy as np
import pytest

import experts_file as ef
import qmoe

torch = pytest.importorskip("torch")
from safetensors import safe_open  # noqa: E402
from safetensors.torch import save_file  # noqa: E402


def fake_quantizer(w, bits):
    """Deterministic stand-in: codes and scale bits derived from the input."""
    e, rows, cols = w.shape
    q = np.clip(np.round(w * 1000), -127, 127).astype(np.int8)
    if bits == 4:
        q = ((q[..., 0::2].astype(np.uint8) & 0xF) << 4 | (q[..., 1::2].astype(np.uint8) & 0xF)).view(np.int8)
    s = (np.abs(w).reshape(e, rows, cols // 32, 32).max(axis=3) * 100).astype(np.float16).view(np.uint16)
    return q, s


@pytest.fixture()
def checkpoint(tmp_path):
    rng = np.random.default_rng(1)
    src = tmp_path / "src"
    src.mkdir()
    t = {
        "model.layers.0.mlp.experts.gate_up_proj.weight": torch.from_numpy(
            rng.standard_normal((4, 64, 96), dtype=np.float32) * 0.02).to(torch.bfloat16),
        "model.layers.0.mlp.experts.down_proj.weight": torch.from_numpy(
            rng.standard_normal((4, 96, 32), dtype=np.float32) * 0.02).to(torch.bfloat16),
        "model.layers.0.mlp.gate.weight": torch.from_numpy(rng.standard_normal((4, 96), dtype=np.float32)).to(
            torch.bfloat16),
        "model.layers.1.mlp.experts.gate_up_proj.weight": torch.from_numpy(
            rng.standard_normal((4, 64, 96), dtype=np.float32) * 0.02),
        "model.layers.1.mlp.experts.down_proj.weight": torch.from_numpy(
            rng.standard_normal((4, 96, 32), dtype=np.float32) * 0.02),
        "model.norm.weight": torch.from_numpy(rng.standard_normal(96, dtype=np.float32)),
        "model.embed_tokens.weight": torch.from_numpy(rng.integers(0, 9, (10, 96)).astype(np.int32)),
    }
    save_file(t, str(src / "model.safetensors"))
    (src / "config.json").write_text('{"hidden_size": 96}')
    return src, t


@pytest.mark.parametrize("bits", [8, 4])
def test_round_trip(checkpoint, tmp_path, bits):
    src, t = checkpoint
    out = tmp_path / f"q{bits}"
    man = ef.quantize_checkpoint(str(src), str(out), bits, quantizer=fake_quantizer)
    assert man["bits"] == bits and man["expert_scale_dtype"] == "F16"
    assert sorted(man["experts"]) == sorted(k for k in t if ".experts." in k)
    assert json.loads((out / "quant.json").read_text()) == man
    assert (out / "config.json").read_text() == '{"hidden_size": 96}'
    with safe_open(str(out / "model.safetensors"), framework="pt") as f:
        keys = set(f.keys())
        for k, v in t.items():
            if ".experts." in k:
                base = k[:-len(".weight")]
                assert k not in keys
                q, s = f.get_tensor(base + ".qweight"), f.get_tensor(base + ".scale")
                e, rows, cols = v.shape
                assert q.dtype == torch.int8 and tuple(q.shape) == (e, rows, cols if bits == 8 else cols // 2)
                assert s.dtype == torch.float16 and tuple(s.shape) == (e, rows, cols // 32)
                wq, ws = fake_quantizer(v.float().numpy(), bits)
                assert np.array_equal(q.numpy(), wq) and np.array_equal(s.numpy().view(np.uint16), ws)
            else:
                got = f.get_tensor(k)
                assert got.dtype == v.dtype and torch.equal(got, v)  # passthrough, byte for byte
    for layer in (0, 1):
        qx = ef.read_layer_experts(str(out), f"model.layers.{layer}.")
        gu = t[f"model.layers.{layer}.mlp.experts.gate_up_proj.weight"].float().numpy()
        dn = t[f"model.layers.{layer}.mlp.experts.down_proj.weight"].float().numpy()
        for (codes, scales), w in (((qx.gate_up, qx.gate_up_scales), gu), ((qx.down, qx.down_scales), dn)):
            wq, ws = fake_quantizer(w, bits)
            assert np.array_equal(codes.view(np.int8), wq) and np.array_equal(scales, ws)
        assert qx.fmt == (qmoe.INT8G32 if bits == 8 else qmoe.INT4G32)


def test_reader_rejects_missing_layer(checkpoint, tmp_path):
    src, _ = checkpoint
    out = tmp_path / "q"
    ef.quantize_checkpoint(str(src), str(out), 8, quantizer=fake_quantizer)
    with pytest.raises(KeyError):
        ef.read_layer_experts(str(out), "model.layers.7.")


def test_writer_checks_plan(tmp_path):
    p = str(tmp_path / "x.safetensors")
    w = ef.StreamingWriter(p, [("a", "F32", (2,)), ("b", "I8", (3,))])
    with pytest.raises(ValueError):
        w.write("b", np.zeros(3, np.int8))  # out of order
    with pytest.raises(ValueError):
        w.write("a", np.zeros(3, np.float32))  # wrong size
    w.write("a", np.float32([1.5, -2.0]))
    with pytest.raises(ValueError):
        w.close()  # b missing
    w = ef.StreamingWriter(p, [("a", "F32", (2,)), ("b", "I8", (3,))], {"k": "v"})
    w.write("a", np.float32([1.5, -2.0]))
    w.write("b", np.int8([1, -2, 3]))
    w.close()
    with safe_open(p, framework="numpy") as f:
        assert f.metadata() == {"k": "v"}
        assert np.array_equal(f.get_tensor("a"), np.float32([1.5, -2.0]))
        assert np.array_equal(f.get_tensor("b"), np.int8([1, -2, 3]))
    assert ef.read_header(p)["a"]["data_offsets"] == [0, 8]


def test_quantize_rejects_bad_stacks(tmp_path):
    src = tmp_path / "bad"
    src.mkdir()
    save_file({"model.layers.0.mlp.experts.down_proj.weight": torch.zeros(2, 8, 40)}, str(src / "m.safetensors"))
    with pytest.raises(ValueError):
        ef.quantize_checkpoint(str(src), str(tmp_path / "o"), 8, quantizer=fake_quantizer)  # K = 40
    with pytest.raises(ValueError):
        ef.quantize_checkpoint(str(src), str(tmp_path / "o"), 3, quantizer=fake_quantizer)
