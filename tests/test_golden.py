"""Real-weight fixtures: layer 0's MoE block of the two tiny checkpoints the
reference's integration tests load (tests/fixtures/tiny-qwen3-moe and
tests/fixtures/tiny-mixtral), with 12 seeded input rows, the q8_0 / q4_0
codes of every matrix and the expected routes, route weights and outputs.
tests/golden/make_golden.py wrote them with the oracle.

CPU: the oracle still reproduces every committed array bit for bit, and its
outputs stay within activation-quantization error of a float64 SwiGLU MoE
evaluated with the decoded weights on the same routes.
GPU: quantizing the real weights on the device gives the committed codes, and
the grouped multi-token path and the one-token decode path both give the
committed routes, weights and outputs bit for bit (rel-L2 <= 1e-5 asserted
as well).
"""
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny_moe.npz")
MODELS = ("qwen3moe", "mixtral")
DTYPES = (("q8_0", O.Q8_0), ("q4_0", O.Q4_0))
REL_L2 = 1e-5


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def same_bits(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and bool((a.view(np.uint32) == b.view(np.uint32)).all())


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def meta(g, m):
    E, Hd, I, k, norm = (int(v) for v in g[f"{m}_meta"])
    return E, Hd, I, k, bool(norm)


@pytest.mark.parametrize("m", MODELS)
@pytest.mark.parametrize("dname,dt", DTYPES)
def test_oracle_reproduces_fixture(g, m, dname, dt):
    E, Hd, I, k, norm = meta(g, m)
    codes = []
    for name in ("gate", "up", "down"):
        w = g[f"{m}_{name}"]
        c = np.stack([O.encode_matrix(dt, w[e]) for e in range(E)]).reshape(E, -1)
        assert (c == g[f"{m}_{dname}_{name}_codes"]).all(), name
        codes.append(c)
    L = O.OracleMoe(dt, Hd, I, E, k, norm, g[f"{m}_router"], *codes)
    out, idx, w = L.prefill(g[f"{m}_x"])
    assert (idx == g[f"{m}_{dname}_idx"]).all()
    assert same_bits(w, g[f"{m}_{dname}_w"])
    assert same_bits(out, g[f"{m}_{dname}_out"])


@pytest.mark.parametrize("m", MODELS)
@pytest.mark.parametrize("dname,dt", DTYPES)
def test_fixture_outputs_near_float64_moe_on_decoded_weights(g, m, dname, dt):
    """On the committed routes, sum_r w_r * down(silu(gate x) * up x) in
    float64 with the weights decoded from the committed codes: only the q8
    rounding of x and of h separates it from the quantized path (1.1 % rel-L2
    measured for all four cases; bound 2 %).  A wrong nibble pairing, scale
    or dropped block in the quantized dot is far outside that."""
    E, Hd, I, k, norm = meta(g, m)
    x = g[f"{m}_x"].astype(np.float64)
    dec = {}
    for n, (rows, cols) in (("gate", (I, Hd)), ("up", (I, Hd)), ("down", (Hd, I))):
        codes, rb = g[f"{m}_{dname}_{n}_codes"], O.row_bytes(dt, cols)
        dec[n] = np.stack([np.stack([O.decode_row(dt, codes[e][r * rb:(r + 1) * rb], cols)
                                     for r in range(rows)]) for e in range(E)]).astype(np.float64)
    idx, w = g[f"{m}_{dname}_idx"], g[f"{m}_{dname}_w"].astype(np.float64)
    ref = np.zeros_like(x)
    for t in range(x.shape[0]):
        for s in range(idx.shape[1]):
            e = idx[t, s]
            a = dec["gate"][e] @ x[t]
            h = a / (1.0 + np.exp(-a)) * (dec["up"][e] @ x[t])
            ref[t] += w[t, s] * (dec["down"][e] @ h)
    assert rel_l2(g[f"{m}_{dname}_out"], ref) < 0.02


@pytest.mark.gpu
@pytest.mark.parametrize("m", MODELS)
@pytest.mark.parametrize("dname,dt", DTYPES)
def test_gpu_matches_fixture(ctx, g, m, dname, dt):
    import hale_moe as H

    E, Hd, I, k, norm = meta(g, m)
    for name in ("gate", "up", "down"):
        w = g[f"{m}_{name}"].reshape(-1, g[f"{m}_{name}"].shape[2])
        got = H.encode_rows(ctx, dt, w).reshape(E, -1)
        assert (got == g[f"{m}_{dname}_{name}_codes"]).all(), name
    router = H.WeightMatrix.new(ctx, E, Hd, "f32", np.ascontiguousarray(g[f"{m}_router"]).view(np.uint8))
    moe = H.MoeLayer(ctx, 0, E, Hd, I, dt, k, norm, router)
    for e in range(E):
        moe.set_expert(e, *(g[f"{m}_{dname}_{n}_codes"][e] for n in ("gate", "up", "down")))
    x = g[f"{m}_x"]
    want_out, want_idx, want_w = (g[f"{m}_{dname}_{s}"] for s in ("out", "idx", "w"))
    # all 12 rows at once: the expert-grouped path
    out, idx, w = moe.forward(x, return_routes=True)
    assert (np.asarray(idx) == want_idx).all()
    assert same_bits(w, want_w)
    assert rel_l2(out, want_out) <= REL_L2
    assert same_bits(out, want_out)
    # all 12 rows in one decode pass (threshold above 12)
    moe.set_grouped_min_tokens(13)
    out, idx, w = moe.forward(x, return_routes=True)
    assert (np.asarray(idx) == want_idx).all()
    assert same_bits(w, want_w)
    assert same_bits(out, want_out)
    # one row at a time: the decode path
    for t in range(x.shape[0]):
        o, i, ww = moe.forward(x[t], return_routes=True)
        assert list(i) == list(want_idx[t]), t
        assert same_bits(ww, want_w[t]), t
        assert same_bits(o, want_out[t]), t
    moe.close()
