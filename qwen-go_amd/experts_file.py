"""Quantised routed experts on disk: the 3D counterpart of qwen-quant's packed
linears, and its loader.

qwen-quant (cmd/qwen-quant/main.go:47-74, 181, 198-210) packs only 2D linears
into `<base>.qweight` (I8) + `<base>.scale` (F32, (out, in/32)) and lists their
`.weight` names in quant.json ({"bits", "quantized"}); the loader reads them
back as quantLinear (model/load.go:50-53, 474-582) and refuses anything that is
not 2D (main.go:181), so the stacked experts `layers.N.mlp.experts.gate_up_proj
.weight` (E, 2I, H) and `.down_proj.weight` (E, H, I) (load.go:415-449) stay
bf16.  This module adds them:

  <base>.qweight  I8  (E, rows, K)      int8 codes, or
                  I8  (E, rows, K/2)    int4 pairs: high nibble = even element,
                                        stored value = code + 8 (moe.go:190-217)
  <base>.scale    F16 (E, rows, K/32)   one scale per 32-element group

Each (rows, K) matrix is quantised as quantizeInt8 / quantizeInt4 do
(moe.go:165-217: per-group amax / 127 or / 7, floor 1e-8, round half away from
zero, clamp); the codes come from the f32 scale and the scale is then stored
rounded to fp16 (nearest even) -- the format the device kernels read.  The
reference's F16 widening (safetensors.go:182-207) reads it back exactly.
quant.json gains two keys the reference's manifest parser ignores:
"experts" (the `.weight` names packed this way) and "expert_scale_dtype".

The quantiser runs on the GPU (qmoe_quantize_device); writing is streamed one
tensor at a time (at most one stacked tensor in host memory); reading is
memory-mapped.
"""
from __future__ import annotations

import json
import os
import shutil
import struct

import numpy as np

import qmoe

GROUP = 32
EXPERT_SUFFIXES = ("mlp.experts.gate_up_proj.weight", "mlp.experts.down_proj.weight")
_ELEM = {"BOOL": 1, "U8": 1, "I8": 1, "F8_E4M3": 1, "F8_E5M2": 1, "I16": 2, "U16": 2, "F16": 2, "BF16": 2,
         "I32": 4, "U32": 4, "F32": 4, "I64": 8, "U64": 8, "F64": 8}


def is_expert_key(key: str) -> bool:
    return key.endswith(EXPERT_SUFFIXES)


# ------------------------------------------------------------ safetensors I/O

class StreamingWriter:
    """A safetensors file written tensor by tensor: the header (names, dtypes,
    shapes, offsets) is fixed up front from a plan, then each payload is
    appended in plan order."""

    def __init__(self, path: str, plan: list[tuple[str, str, tuple[int, ...]]], metadata: dict | None = None):
        header = {}
        off = 0
        self.sizes = []
        for name, dt, shape in plan:
            n = int(np.prod(shape, dtype=np.int64)) * _ELEM[dt]
            header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + n]}
            self.sizes.append((name, n))
            off += n
        if metadata:
            header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
        hb = json.dumps(header, separators=(",", ":")).encode()
        hb += b" " * (-len(hb) % 8)  # payload 8-byte aligned
        self.f = open(path, "wb")
        self.f.write(struct.pack("<Q", len(hb)))
        self.f.write(hb)
        self.next = 0

    def write(self, name: str, data: bytes | memoryview | np.ndarray):
        want, n = self.sizes[self.next]
        if name != want:
            raise ValueError(f"tensor {name} written out of plan order (expected {want})")
        b = memoryview(np.ascontiguousarray(data)).cast("B") if isinstance(data, np.ndarray) else memoryview(data)
        if b.nbytes != n:
            raise ValueError(f"tensor {name}: {b.nbytes} bytes, the plan says {n}")
        self.f.write(b)
        self.next += 1

    def close(self):
        if self.next != len(self.sizes):
            raise ValueError(f"{len(self.sizes) - self.next} planned tensors were not written")
        self.f.close()


def read_header(path: str) -> dict:
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        return json.loads(f.read(n))


class TensorFile:
    """Memory-mapped read access to one safetensors file (raw bytes per tensor)."""

    def __init__(self, path: str):
        self.path = path
        self.header = read_header(path)
        with open(path, "rb") as f:
            self.base = 8 + struct.unpack("<Q", f.read(8))[0]
        self.mm = np.memmap(path, dtype=np.uint8, mode="r")

    def keys(self):
        return [k for k in self.header if k != "__metadata__"]

    def info(self, key):
        h = self.header[key]
        return h["dtype"], tuple(h["shape"])

    def raw(self, key) -> np.ndarray:
        a, b = self.header[key]["data_offsets"]
        return self.mm[self.base + a:self.base + b]

    def array(self, key, dtype) -> np.ndarray:
        return self.raw(key).view(dtype).reshape(self.info(key)[1])


# ----------------------------------------------------------------- writing

def _bf16_raw_to_f32(raw: np.ndarray) -> np.ndarray:
    return (raw.view(np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def quantize_stack_device(w: np.ndarray, bits: int):
    """(n_mat, rows, K) f32 -> (codes I8 (n_mat, rows, K or K/2), scales fp16
    bits (n_mat, rows, K/32)) on the GPU, quantizeInt8 / quantizeInt4
    (model/moe.go:165-217) then the scale rounded to fp16."""
    n_mat, rows, cols = w.shape
    if cols % GROUP:
        raise ValueError(f"K = {cols} is not a multiple of {GROUP}")
    codes, scales = qmoe.device_quantizer(bits, w, n_mat, rows, cols)
    codes = codes.reshape(n_mat, rows, cols if bits == 8 else cols // 2).view(np.int8)
    return codes, scales.reshape(n_mat, rows, cols // GROUP)


def quantize_checkpoint(src: str, out: str, bits: int, quantizer=quantize_stack_device) -> dict:
    """Copies the checkpoint directory src into out with every stacked expert
    tensor (layers.N.mlp.experts.{gate_up,down}_proj.weight, BF16 or F32)
    replaced by its .qweight / .scale pair; every other tensor passes through
    unchanged into out/model.safetensors, and config.json / tokenizer.json are
    copied.  Returns the manifest written to out/quant.json."""
    if bits not in (8, 4):
        raise ValueError("bits must be 8 or 4")
    shards = sorted(os.path.join(src, f) for f in os.listdir(src) if f.endswith(".safetensors"))
    if not shards:
        raise FileNotFoundError(f"no .safetensors shards in {src}")
    os.makedirs(out, exist_ok=True)
    files = [TensorFile(p) for p in shards]
    plan, jobs, experts = [], [], []
    for tf in files:
        for key in sorted(tf.keys()):
            dt, shape = tf.info(key)
            if is_expert_key(key):
                if len(shape) != 3 or dt not in ("BF16", "F32"):
                    raise ValueError(f"{key}: expected a 3D BF16/F32 stack, got {dt} {shape}")
                e, rows, cols = shape
                if cols % GROUP:
                    raise ValueError(f"{key}: K = {cols} is not a multiple of {GROUP}")
                base = key[:-len(".weight")]
                plan.append((base + ".qweight", "I8", (e, rows, cols if bits == 8 else cols // 2)))
                plan.append((base + ".scale", "F16", (e, rows, cols // GROUP)))
                jobs.append(("quant", tf, key, base))
                experts.append(key)
            else:
                plan.append((key, dt, shape))
                jobs.append(("copy", tf, key, key))
    w = StreamingWriter(os.path.join(out, "model.safetensors"), plan, {"format": "pt"})
    try:
        for kind, tf, key, base in jobs:
            if kind == "copy":
                w.write(key, tf.raw(key))
                continue
            dt, shape = tf.info(key)
            raw = tf.raw(key)
            f32 = _bf16_raw_to_f32(raw) if dt == "BF16" else raw.view(np.float32)
            codes, scales = quantizer(np.ascontiguousarray(f32.reshape(shape)), bits)
            w.write(base + ".qweight", codes)
            w.write(base + ".scale", scales)
    finally:
        w.f.close()
    w.close()
    manifest = {"bits": bits, "quantized": [], "experts": experts, "expert_scale_dtype": "F16"}
    with open(os.path.join(out, "quant.json"), "w") as fh:
        json.dump(manifest, fh, indent=2)
    for aux in ("config.json", "tokenizer.json"):
        if os.path.exists(os.path.join(src, aux)):
            shutil.copyfile(os.path.join(src, aux), os.path.join(out, aux))
    return manifest


# ----------------------------------------------------------------- reading

class QuantExperts:
    """One layer's packed experts as stored: int8 codes (or int4 pairs) and
    fp16 scale bit patterns."""

    def __init__(self, bits, gate_up, gate_up_scales, down, down_scales):
        self.bits = bits
        self.gate_up, self.gate_up_scales = gate_up, gate_up_scales
        self.down, self.down_scales = down, down_scales

    @property
    def fmt(self) -> int:
        return qmoe.INT8G32 if self.bits == 8 else qmoe.INT4G32

    def upload(self, layer: qmoe.MoeLayer):
        """qmoe_set_experts with the stored codes and scales (no re-quantisation)."""
        if layer.cfg.expert_fmt != self.fmt:
            raise ValueError(f"layer expert format {layer.cfg.expert_fmt}, file holds {self.fmt}")
        layer.set_experts(np.ascontiguousarray(self.gate_up), np.ascontiguousarray(self.gate_up_scales),
                          np.ascontiguousarray(self.down), np.ascontiguousarray(self.down_scales))


def load_manifest(path: str) -> dict:
    with open(os.path.join(path, "quant.json")) as fh:
        return json.load(fh)


def read_layer_experts(path: str, prefix: str) -> QuantExperts:
    """The packed experts under key prefix (e.g. "model.layers.3.") of the
    directory path, memory-mapped."""
    man = load_manifest(path)
    bits = int(man["bits"])
    if man.get("expert_scale_dtype", "F16") != "F16":
        raise ValueError("only F16 expert scales are defined")
    found = {}
    for f in sorted(os.listdir(path)):
        if not f.endswith(".safetensors"):
            continue
        tf = TensorFile(os.path.join(path, f))
        for which in ("gate_up_proj", "down_proj"):
            base = f"{prefix}mlp.experts.{which}"
            if base + ".qweight" in tf.header:
                qd, qs = tf.info(base + ".qweight")
                sd, ss = tf.info(base + ".scale")
                if qd != "I8" or sd != "F16" or len(qs) != 3 or len(ss) != 3:
                    raise ValueError(f"{base}: unexpected dtypes/shapes {qd}{qs} {sd}{ss}")
                k = qs[2] * (2 if bits == 4 else 1)
                if ss[:2] != qs[:2] or ss[2] * GROUP != k:
                    raise ValueError(f"{base}: scale shape {ss} does not match codes {qs} at {bits} bits")
                codes = tf.array(base + ".qweight", np.int8)
                found[which] = (codes if bits == 8 else codes.view(np.uint8), tf.array(base + ".scale", np.uint16))
    if set(found) != {"gate_up_proj", "down_proj"}:
        raise KeyError(f"packed experts under {prefix!r} not found in {path}")
    return QuantExperts(bits, *found["gate_up_proj"], *found["down_proj"])


def main(argv=None):
    import argparse
    ap = argparse.ArgumentParser(description="pack the stacked routed experts of a checkpoint into "
                                             ".qweight / .scale (quantised on the GPU)")
    ap.add_argument("--src", required=True, help="checkpoint directory (*.safetensors, config.json)")
    ap.add_argument("--out", required=True, help="output directory")
    ap.add_argument("--bits", type=int, default=8, choices=(8, 4))
    a = ap.parse_args(argv)
    import torch
    torch.cuda.init()  # the HIP runtime torch brings, before the library loads
    man = quantize_checkpoint(a.src, a.out, a.bits)
    print(f"packed {len(man['experts'])} expert stacks to int{a.bits} -> {a.out}")


if __name__ == "__main__":
    main()
