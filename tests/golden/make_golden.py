"""Writes tests/golden/tiny_moe.npz: real-weight MoE layers with their inputs
and expected outputs, for the quantized expert path.

Weights are layer 0's MoE block of the two checkpoints the reference's own
integration tests load (tests/fixtures/tiny-qwen3-moe/model.safetensors,
tests/fixtures/tiny-mixtral/model.safetensors, read by tests/tiered_cache.rs
and tests/fixtures/*/config.json):
  qwen3moe: 8 experts, H 64, I 32, top-3, norm_topk_prob true  (f32 weights)
  mixtral:  4 experts, H 64, I 32, top-2, always renormalised (bf16 weights,
            widened to f32 by a 16-bit shift as src/tensor/quant.rs:48-52 does)
(normalize_topk per architecture: src/config.rs:205-208.)

Expected values come from the oracle: the codes of every matrix in q8_0 and
q4_0 (src/tensor/quant.rs:274-321) and, for 12 seeded N(0,1) input rows, the
routes, route weights and MoE outputs (src/model/moe.rs:36-70).  The file
carries the inputs with the outputs, so the tests need neither the reference
tree nor this script.

Run from the repository root:  python tests/golden/make_golden.py
The safetensors files are parsed as JSON header + raw little-endian arrays;
nothing in them is executed.
"""
import json
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402

FIXTURES = "/root/reference/tests/fixtures"
TOKENS = 12
SEED_X = 2024

MODELS = {
    # name: (directory, tensor prefix, router, expert (gate, up, down) names, top_k, normalize)
    "qwen3moe": ("tiny-qwen3-moe", "model.layers.0.mlp.", "gate.weight",
                 ("experts.{e}.gate_proj.weight", "experts.{e}.up_proj.weight",
                  "experts.{e}.down_proj.weight"), "num_experts", 3, True),
    "mixtral": ("tiny-mixtral", "model.layers.0.block_sparse_moe.", "gate.weight",
                ("experts.{e}.w1.weight", "experts.{e}.w3.weight", "experts.{e}.w2.weight"),
                "num_local_experts", 2, True),
}


def read_safetensors(path):
    with open(path, "rb") as f:
        raw = f.read()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    body = raw[8 + n:]
    out = {}
    for name, t in header.items():
        if name == "__metadata__":
            continue
        a, b = t["data_offsets"]
        buf = body[a:b]
        if t["dtype"] == "F32":
            v = np.frombuffer(buf, dtype="<f4").astype(np.float32)
        elif t["dtype"] == "BF16":
            v = (np.frombuffer(buf, dtype="<u2").astype(np.uint32) << 16).view(np.float32)
        else:
            continue
        out[name] = v.reshape(t["shape"])
    return out


def main():
    data = {}
    for m, (d, pre, rname, enames, ekey, k, norm) in MODELS.items():
        cfg = json.load(open(os.path.join(FIXTURES, d, "config.json")))
        assert cfg["num_experts_per_tok"] == k
        E = cfg[ekey]
        t = read_safetensors(os.path.join(FIXTURES, d, "model.safetensors"))
        router = t[pre + rname]
        gate = np.stack([t[pre + enames[0].format(e=e)] for e in range(E)])
        up = np.stack([t[pre + enames[1].format(e=e)] for e in range(E)])
        down = np.stack([t[pre + enames[2].format(e=e)] for e in range(E)])
        Hd, I = gate.shape[2], gate.shape[1]
        x = O.normal(SEED_X, TOKENS * Hd).reshape(TOKENS, Hd)
        data.update({f"{m}_router": router, f"{m}_gate": gate, f"{m}_up": up, f"{m}_down": down,
                     f"{m}_x": x, f"{m}_meta": np.array([E, Hd, I, k, int(norm)], np.int32)})
        for dt, dname in ((O.Q8_0, "q8_0"), (O.Q4_0, "q4_0")):
            codes = [np.stack([O.encode_matrix(dt, w[e]) for e in range(E)]).reshape(E, -1)
                     for w in (gate, up, down)]
            L = O.OracleMoe(dt, Hd, I, E, k, norm, router, *codes)
            out, idx, w = L.prefill(x)
            for name, c in zip(("gate", "up", "down"), codes):
                data[f"{m}_{dname}_{name}_codes"] = c
            data[f"{m}_{dname}_idx"] = idx.astype(np.int32)
            data[f"{m}_{dname}_w"] = w
            data[f"{m}_{dname}_out"] = out
    dst = os.path.join(HERE, "tiny_moe.npz")
    np.savez_compressed(dst, **data)
    print(f"wrote {dst}: {len(data)} arrays, {os.path.getsize(dst)} bytes")


if __name__ == "__main__":
    main()
