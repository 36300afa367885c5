"""The expert pack (src/expert/pack.rs) as the file tier under the HBM tier.

CPU tests mirror the reference's own pack tests (src/expert/pack.rs:300-356):
records written in any order read back unchanged, a key outside the pack
is rejected, garbage and truncated files are rejected.  Their packs are
written by tests/packs.py in PackWriter's layout.  GPU tests load whole
layers from a pack (synchronously and by prefetch) and check that the
layer's outputs are bit-identical to the same layer filled by set_expert,
and to the oracle.
"""
import struct

import numpy as np
import pytest

import hale_moe as H
import oracle as O
import packs as P


def tiny_header(dtype):
    # the reference test's model: hidden 64, intermediate 32, 3 experts,
    # both of its 2 layers MoE
    return P.header_for(dtype, 64, 32, 3, [0, 1])


def sin_matrix(rows, cols, seed):
    """The reference test's weights: ((i + seed) * 0.37).sin() in f32."""
    i = np.arange(rows * cols, dtype=np.float32)
    return np.sin((i + np.float32(seed)) * np.float32(0.37)).astype(np.float32).reshape(rows, cols)


def f32_record(seed):
    g, u, d = sin_matrix(32, 64, seed), sin_matrix(32, 64, seed + 1.0), sin_matrix(64, 32, seed + 2.0)
    return np.concatenate([g.ravel(), u.ravel(), d.ravel()]).view(np.uint8)


# ---------------------------------------------------------------------------
# file format (no GPU)
# ---------------------------------------------------------------------------

def test_header_geometry():
    f32, q4 = tiny_header(O.F32), tiny_header(O.Q4_0)
    for h in (f32, q4):
        assert h["record_stride"] % P.ALIGN == 0
        assert h["data_offset"] % P.ALIGN == 0
    assert q4["record_bytes"] * 7 < f32["record_bytes"]


def test_write_then_read_every_expert_in_any_order(tmp_path):
    h = tiny_header(O.F32)
    path = tmp_path / "experts.hpk"
    keys = [(1, 2), (0, 0), (1, 0)]
    P.write_pack(path, h, {k: f32_record(k[0] * 10.0 + k[1]) for k in keys})
    pack = H.PackExpertSource.open(path)
    try:
        hd = pack.header
        assert (hd.dtype, hd.hidden_size, hd.intermediate_size, hd.num_experts) == (O.F32, 64, 32, 3)
        assert hd.moe_layers == (0, 1)
        assert (hd.record_bytes, hd.record_stride, hd.data_offset) == \
            (h["record_bytes"], h["record_stride"], h["data_offset"])
        assert hd.file_size() == P.file_size(h)
        g, u, d = pack.read_record(H.ExpertKey(1, 2))
        assert (d.view(np.float32).reshape(64, 32) == sin_matrix(64, 32, 14.0)).all()
        assert (g.view(np.float32).reshape(32, 64) == sin_matrix(32, 64, 12.0)).all()
        assert pack.expert_bytes() == g.size + u.size + d.size
        for k in keys:
            assert pack.offset_of(H.ExpertKey(*k)) == P.offset_of(h, *k)
        with pytest.raises(H.InvalidArgument, match="out of range"):
            pack.read_record(H.ExpertKey(0, 3))
        with pytest.raises(H.InvalidArgument, match="no experts"):
            pack.offset_of(H.ExpertKey(2, 0))
        assert "SSD pack" in pack.describe() and "f32" in pack.describe()
    finally:
        pack.close()


@pytest.mark.parametrize("dtype", [O.Q8_0, O.Q4_0])
def test_quantized_records_round_trip(tmp_path, dtype):
    h = P.header_for(dtype, 64, 32, 3, [4, 7])
    L = O.OracleMoe.synthetic(dtype, 64, 32, 3, 2, seed=5, with_router=False)
    recs = {(7, e): np.concatenate([L.gate[e], L.up[e], L.down[e]]) for e in range(3)}
    P.write_pack(tmp_path / "q.hpk", h, recs)
    pack = H.PackExpertSource.open(tmp_path / "q.hpk")
    for e in range(3):
        g, u, d = pack.read_record(H.ExpertKey(7, e))
        assert (g == L.gate[e]).all() and (u == L.up[e]).all() and (d == L.down[e]).all()
    g, u, d = pack.read_record(H.ExpertKey(4, 1))  # never written: zeros
    assert not g.any() and not d.any()
    pack.close()


def test_rejects_garbage(tmp_path):
    p = tmp_path / "junk.hpk"
    p.write_bytes(b"definitely not a pack")
    with pytest.raises(H.InvalidArgument, match="not a Hale expert pack"):
        H.PackExpertSource.open(p)
    with pytest.raises(OSError):
        H.PackExpertSource.open(tmp_path / "missing.hpk")


def test_rejects_truncated_and_wrong_version(tmp_path):
    h = tiny_header(O.Q8_0)
    p = tmp_path / "t.hpk"
    P.write_pack(p, h, {})
    with open(p, "r+b") as f:
        f.truncate(P.file_size(h) - 1)
    with pytest.raises(H.InvalidArgument, match="truncated"):
        H.PackExpertSource.open(p)
    h2 = dict(h, version=2)
    P.write_pack(p, h2, {})
    with pytest.raises(H.InvalidArgument, match="version 2"):
        H.PackExpertSource.open(p)


def test_rejects_oversized_and_malformed_headers(tmp_path):
    p = tmp_path / "h.hpk"
    with open(p, "wb") as f:
        f.write(P.MAGIC + struct.pack("<Q", 64 * P.ALIGN + 1))
    with pytest.raises(H.InvalidArgument, match="too large"):
        H.PackExpertSource.open(p)
    h = tiny_header(O.Q4_0)
    for bad in (b'{"version":1', b'{"version":1,"dtype":"q5_1"}', b"[1,2]",
                P.to_json({k: v for k, v in h.items() if k != "record_stride"})):
        P.write_pack(p, h, {}, header_bytes=bad)
        with pytest.raises(H.InvalidArgument):
            H.PackExpertSource.open(p)


def test_header_fields_in_any_order_unknown_fields_ignored(tmp_path):
    h = tiny_header(O.Q4_0)
    keys = list(h)[::-1]
    js = "{ " + ", ".join(f'"{k}" : {P.json.dumps(h[k])}' for k in keys) + \
         ', "note": {"a": [1, 2.5, "x"], "b": null, "c": true} }'
    p = tmp_path / "o.hpk"
    P.write_pack(p, h, {}, header_bytes=js.encode())
    pack = H.PackExpertSource.open(p)
    assert pack.header.record_stride == h["record_stride"]
    assert pack.header.moe_layers == (0, 1)
    pack.close()


# ---------------------------------------------------------------------------
# HBM tier from the pack (GPU)
# ---------------------------------------------------------------------------

def same_bits(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and bool((a.view(np.uint32) == b.view(np.uint32)).all())


def layer_from(ctx, L, layer_id, fill):
    router = H.WeightMatrix.new(ctx, L.num_experts, L.hidden, "f32", L.router.view(np.uint8))
    moe = H.MoeLayer(ctx, layer_id, L.num_experts, L.hidden, L.inter, L.dtype, L.top_k,
                     L.normalize, router)
    fill(moe)
    return moe


def set_all(L):
    def fill(moe):
        for e in range(L.num_experts):
            moe.set_expert(e, L.gate[e], L.up[e], L.down[e])
    return fill


def write_layers(path, layers: dict):
    """layers {model layer index: OracleMoe}, all of one shape and dtype."""
    L0 = next(iter(layers.values()))
    h = P.header_for(L0.dtype, L0.hidden, L0.inter, L0.num_experts, sorted(layers))
    recs = {(lid, e): np.concatenate([L.gate[e], L.up[e], L.down[e]])
            for lid, L in layers.items() for e in range(L.num_experts)}
    P.write_pack(path, h, recs)
    return h


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [O.Q8_0, O.Q4_0])
def test_load_pack_equals_set_expert(ctx, tmp_path, dtype):
    layers = {1: O.OracleMoe.synthetic(dtype, 64, 32, 3, 2, seed=11),
              3: O.OracleMoe.synthetic(dtype, 64, 32, 3, 2, seed=12)}
    write_layers(tmp_path / "e.hpk", layers)
    pack = H.PackExpertSource.open(tmp_path / "e.hpk")
    for lid, L in layers.items():
        a = layer_from(ctx, L, lid, lambda m: m.load_pack(pack))
        b = layer_from(ctx, L, lid, set_all(L))
        for s in range(4):
            x = O.normal(300 + s, L.hidden)
            ya, ia, wa = a.forward(x, return_routes=True)
            yb, ib, wb = b.forward(x, return_routes=True)
            yo, io, wo = L.forward(x)
            assert same_bits(ya, yb) and same_bits(ya, yo)
            assert (ia == io).all() and same_bits(wa, wo)
        a.close()
        b.close()
    pack.close()


@pytest.mark.gpu
def test_prefetch_two_layers_in_batches(ctx, tmp_path):
    # 7 experts of 20 MB: three records per 64 MiB batch, so each load runs
    # three batches through the two staging slots
    layers = {0: O.OracleMoe.synthetic(O.Q8_0, 2048, 3072, 7, 2, seed=21),
              2: O.OracleMoe.synthetic(O.Q8_0, 2048, 3072, 7, 2, seed=22)}
    h = write_layers(tmp_path / "big.hpk", layers)
    assert (64 << 20) // h["record_stride"] == 3
    pack = H.PackExpertSource.open(tmp_path / "big.hpk")
    a0 = layer_from(ctx, layers[0], 0, lambda m: m.prefetch_pack(pack))
    a2 = layer_from(ctx, layers[2], 2, lambda m: m.prefetch_pack(pack))  # waits for layer 0's reads
    for lid, a in ((0, a0), (2, a2)):
        L = layers[lid]
        x = O.normal(400 + lid, L.hidden)
        T = 9  # the grouped multi-token path reads every expert
        xs = O.normal(500 + lid, T * L.hidden).reshape(T, L.hidden)
        y = a.forward(x)
        ys = a.forward(xs)
        assert same_bits(y, L.forward(x)[0])
        assert same_bits(ys, L.prefill(xs)[0])
    a0.close()
    a2.close()
    pack.close()


@pytest.mark.gpu
def test_load_pack_errors(ctx, tmp_path):
    L = O.OracleMoe.synthetic(O.Q4_0, 64, 32, 3, 2, seed=13)
    write_layers(tmp_path / "e.hpk", {1: L})
    pack = H.PackExpertSource.open(tmp_path / "e.hpk")
    with pytest.raises(H.InvalidArgument, match="no experts"):
        layer_from(ctx, L, 5, lambda m: m.load_pack(pack))      # layer not in the pack
    L8 = O.OracleMoe.synthetic(O.Q8_0, 64, 32, 3, 2, seed=13)
    with pytest.raises(ValueError, match="does not match"):
        layer_from(ctx, L8, 1, lambda m: m.load_pack(pack))     # q4_0 pack, q8_0 layer
    pack.close()
