"""Writes the committed golden fixtures of the MoE block (run from the repo root:
python tests/golden/make_golden.py).

Every expected value here is derived without the oracle: hand-derived known
answers whose arithmetic is exact in f32, and a float64 numpy evaluation of
the layer written from the reference's definitions (model/moe.go:41-97).

  known_answers.json
    quantizer groups whose scales are powers of two, so w / s is exact and
    the codes follow from round-half-away-from-zero by hand
    (model/moe.go:165-217, 241-258); dequantised bytes (model/moe.go:134-157);
    the routing of TestMoERouting (model/model_test.go:182-201); the first-k
    selection quirk (model/moe.go:44-53).
  tiny_layer.npz
    a small f32 layer (H=64, E=8, k=2, I=32, shared I_s=32 with its sigmoid
    gate) with T=4 tokens, and the float64 layer output, ids and weights for
    select scope C=E and C=k.  The seed is chosen so that adjacent ranks are
    separated by more than 1e-3 in probability, far beyond f32 rounding.
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f32(v):
    return float(np.float32(v))


def quant_cases():
    cases = []
    # int8, s = 2^-7: amax = 127 * 2^-7
    s8 = 2.0 ** -7
    w = [0.0] * 32
    w[0] = 127 * s8            # amax -> +127
    w[1] = 2.5 * s8            # half way -> 3 (half away from zero; RNE would give 2)
    w[2] = -2.5 * s8           # -> -3
    w[3] = 0.5 * s8            # -> 1
    w[4] = -0.5 * s8           # -> -1
    w[5] = 0.49 * s8           # -> 0
    w[6] = -126.5 * s8         # -> -127
    w[7] = 3 * s8              # exact -> 3
    codes = [0] * 32
    codes[0], codes[1], codes[2], codes[3], codes[4], codes[5], codes[6], codes[7] = 127, 3, -3, 1, -1, 0, -127, 3
    cases.append({"bits": 8, "w": [f32(v) for v in w], "codes": codes, "scale": s8})
    # all-zero group: amax 0 -> scale floored at 1e-8, codes 0
    cases.append({"bits": 8, "w": [0.0] * 32, "codes": [0] * 32, "scale": f32(1e-8)})
    # int4, s = 2^-4: amax = 7 * 2^-4; stored value = code + 8, even element in the high nibble
    s4 = 2.0 ** -4
    w = [0.0] * 32
    w[0] = -7 * s4             # amax -> -7 -> stored 1
    w[1] = 2.5 * s4            # -> 3 -> 11
    w[2] = -2.5 * s4           # -> -3 -> 5
    w[3] = 0.5 * s4            # -> 1 -> 9
    w[4] = 6.5 * s4            # -> 7 -> 15
    w[5] = -0.5 * s4           # -> -1 -> 7
    stored = [8] * 32
    stored[0], stored[1], stored[2], stored[3], stored[4], stored[5] = 1, 11, 5, 9, 15, 7
    packed = [(stored[2 * j] << 4) | stored[2 * j + 1] for j in range(16)]
    cases.append({"bits": 4, "w": [f32(v) for v in w], "packed": packed, "scale": s4})
    return cases


def dequant_cases():
    # int8 code 0x81 = -127; int4 byte 0x9F = nibbles 9, 15 -> values +1, +7
    return [
        {"bits": 8, "bytes": [0x81, 0x7F, 0x00, 0x01], "scale": 0.25, "values": [-31.75, 31.75, 0.0, 0.25]},
        {"bits": 4, "bytes": [0x9F, 0x08, 0x80], "scale": 0.5, "values": [0.5, 3.5, -4.0, 0.0, 0.0, -4.0]},
    ]


def routing_case():
    # TestMoERouting: router row 0 = [1, 2, 3, 4, 0...], other rows 0; x = 0.1..0.8
    x = [0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8]
    l0 = sum(np.float64(np.float32(a)) * b for a, b in zip(x, [1, 2, 3, 4]))
    p0 = np.exp(l0) / (np.exp(l0) + 3.0)
    p1 = 1.0 / (np.exp(l0) + 3.0)
    return {"x": x, "router_row0": [1.0, 2.0, 3.0, 4.0, 0.0, 0.0, 0.0, 0.0], "E": 4, "H": 8, "k": 2,
            "ids_first_k": [0, 1], "p0": float(p0), "p1": float(p1),
            "w0": float(p0 / (p0 + p1)), "w1": float(p1 / (p0 + p1))}


def select_cases():
    return [
        {"p": [0.1, 0.2, 0.6, 0.1], "k": 2, "scope": 2, "ids": [1, 0]},   # first-k: set {0, 1}
        {"p": [0.1, 0.2, 0.6, 0.1], "k": 2, "scope": 4, "ids": [2, 1]},   # true top-k
        {"p": [0.25, 0.25, 0.25, 0.25], "k": 3, "scope": 4, "ids": [0, 1, 2]},  # ties: lowest index
        {"p": [0.1, 0.3, 0.3, 0.3], "k": 2, "scope": 4, "ids": [1, 2]},
    ]


def layer_f64(x, router, gu, dn, sg, su, sd, sgate, k, scope):
    """float64 evaluation of moeMLP.forward (model/moe.go:41-97)."""
    E = router.shape[0]
    I = gu.shape[1] // 2
    T = x.shape[0]
    out = np.zeros((T, x.shape[1]))
    ids = np.zeros((T, k), np.int64)
    ws = np.zeros((T, k))
    silu = lambda v: v / (1.0 + np.exp(-v))
    for t in range(T):
        lg = router @ x[t]
        p = np.exp(lg - lg.max())
        p /= p.sum()
        cand = sorted(range(scope), key=lambda e: (-p[e], e))[:k]
        w = p[cand] / (p[cand].sum() + 1e-9)
        ids[t], ws[t] = cand, w
        for r, e in enumerate(cand):
            h = gu[e] @ x[t]
            a = silu(h[:I]) * h[I:]
            out[t] += w[r] * (dn[e] @ a)
        a = silu(sg @ x[t]) * (su @ x[t])
        gate = 1.0 / (1.0 + np.exp(-(sgate @ x[t])))
        out[t] += gate * (sd @ a)
    return out, ids, ws


def tiny_layer():
    H, E, k, I, Is, T = 64, 8, 2, 32, 32, 4
    for seed in range(1000):
        rng = np.random.default_rng(seed)
        router = (rng.standard_normal((E, H)) * 0.3).astype(np.float32)
        gu = (rng.standard_normal((E, 2 * I, H)) * 0.1).astype(np.float32)
        dn = (rng.standard_normal((E, H, I)) * 0.1).astype(np.float32)
        sg = (rng.standard_normal((Is, H)) * 0.1).astype(np.float32)
        su = (rng.standard_normal((Is, H)) * 0.1).astype(np.float32)
        sd = (rng.standard_normal((H, Is)) * 0.1).astype(np.float32)
        sgate = (rng.standard_normal(H) * 0.1).astype(np.float32)
        x = rng.standard_normal((T, H)).astype(np.float32)
        f = lambda a: a.astype(np.float64)
        ok = True
        for scope in (E, k):
            lg = f(x) @ f(router).T
            for t in range(T):
                p = np.exp(lg[t] - lg[t].max())
                p /= p.sum()
                q = np.sort(p[:scope])[::-1]
                if np.min(np.abs(np.diff(q[:k + 1 if scope > k else k]))) < 1e-3:
                    ok = False
        if ok:
            break
    res = {}
    for tag, scope in (("E", E), ("k", k)):
        out, ids, ws = layer_f64(f(x), f(router), f(gu), f(dn), f(sg), f(su), f(sd), f(sgate), k, scope)
        res[f"out_{tag}"], res[f"ids_{tag}"], res[f"w_{tag}"] = out, ids.astype(np.int32), ws
    np.savez(os.path.join(HERE, "tiny_layer.npz"), seed=np.int64(seed), router=router, gate_up=gu, down=dn,
             sh_gate=sg, sh_up=su, sh_down=sd, shared_gate=sgate, x=x, **res)
    return seed


def main():
    ka = {"quantize": quant_cases(), "dequantize": dequant_cases(), "routing": routing_case(),
          "select": select_cases()}
    with open(os.path.join(HERE, "known_answers.json"), "w") as fh:
        json.dump(ka, fh, indent=1)
    seed = tiny_layer()
    print("wrote known_answers.json and tiny_layer.npz (seed %d)" % seed)


if __name__ == "__main__":
    main()
