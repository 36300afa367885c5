"""The ExpertProvider surface of the HBM MoE layer through the C ABI
(src/expert/mod.rs:128-137, ExpertCache::fetch src/expert/cache.rs:124-194,
CacheStats :15-54): fetch in request order with one routing record per key,
misses loaded from the layer's source pack, CacheStats counters including
bytes_loaded and load_seconds.  Fetched experts are views into the layer's
HBM planes and compute Expert::forward bit-exact against the oracle."""
import numpy as np
import pytest

import hale_moe as H
import oracle as O
import packs as P

pytestmark = pytest.mark.gpu

E, HID, INTER, K, LAYER = 8, 256, 64, 2, 5


def same_bits(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and bool((a.view(np.uint32) == b.view(np.uint32)).all())


@pytest.fixture(params=[O.Q8_0, O.Q4_0])
def oracle_layer(request):
    return O.OracleMoe.synthetic(request.param, HID, INTER, E, K, normalize_topk=True,
                                 seed=40 + request.param)


def new_layer(ctx, L, experts=()):
    router = H.WeightMatrix.new(ctx, E, HID, "f32", L.router.view(np.uint8))
    moe = H.MoeLayer(ctx, LAYER, E, HID, INTER, L.dtype, K, True, router)
    for e in experts:
        moe.set_expert(e, L.gate[e], L.up[e], L.down[e])
    return moe


def write_pack(path, L, layers=(LAYER,)):
    h = P.header_for(L.dtype, HID, INTER, E, layers)
    recs = {(lid, e): np.concatenate([L.gate[e], L.up[e], L.down[e]])
            for lid in layers for e in range(E)}
    P.write_pack(path, h, recs)
    return h


def expert_out(L, e, x):
    return O.expert_forward(L.dtype, HID, INTER, L.gate[e], L.up[e], L.down[e], x)


def test_fetch_serves_resident_experts_in_request_order(ctx, oracle_layer):
    """Keys come back in request order (the reference's tiers_are_consulted_
    in_order); each expert computes Expert::forward and matvec bit-exact,
    holds the registered bytes, and every key is one routing record and
    one pinned hit."""
    L = oracle_layer
    moe = new_layer(ctx, L, range(E))
    keys = [H.ExpertKey(LAYER, e) for e in (3, 1, 3, 0)]
    got = moe.experts.fetch(keys)
    assert len(got) == 4
    x = O.normal(11, HID)
    for k, ex in zip(keys, got):
        assert (ex.gate.rows(), ex.gate.cols(), ex.down.rows(), ex.down.cols()) == (INTER, HID, HID, INTER)
        assert (ex.gate.bytes() == L.gate[k.expert]).all()
        assert (ex.down.bytes() == L.down[k.expert]).all()
        assert same_bits(ex.forward(x), expert_out(L, k.expert, x))
        assert same_bits(ex.up.matvec(x), O.matvec(L.dtype, INTER, HID, L.up[k.expert], x))
    counts = moe.experts.routing_counts()
    assert list(counts) == [1, 1, 0, 2, 0, 0, 0, 0]
    s = moe.experts.stats()
    assert (s.pinned_hits, s.lru_hits, s.misses, s.bytes_loaded) == (4, 0, 0, 0)
    assert (s.pinned_experts, s.pinned_bytes) == (E, E * moe.expert_bytes())
    assert (s.lru_experts, s.lru_bytes, s.lru_capacity_bytes, s.passthrough) == (0, 0, 0, False)
    assert s.hit_rate() == 1.0 and s.load_gbps() == 0.0
    moe.close()


def test_forward_selections_are_pinned_hits(ctx, oracle_layer):
    """A forward serves every selected expert from HBM: k pinned hits per
    token, on the decode and the grouped path, on top of fetch requests."""
    L = oracle_layer
    moe = new_layer(ctx, L, range(E))
    moe.forward(O.normal(12, HID))                              # decode: 1 token
    moe.forward(O.normal(13, 12 * HID).reshape(12, HID))        # grouped: 12 tokens
    moe.experts.fetch([H.ExpertKey(LAYER, 2)])
    s = moe.experts.stats()
    assert s.pinned_hits == 13 * K + 1 and s.misses == 0
    assert int(moe.experts.routing_counts().sum()) == 13 * K + 1
    moe.close()


def test_fetch_of_a_missing_expert_without_source(ctx, oracle_layer):
    """Without a source a missing expert is KeyError; the key is still
    recorded (routing is recorded before any load) and no counter moves."""
    L = oracle_layer
    moe = new_layer(ctx, L, range(4))
    assert not moe.experts.present(5) and moe.experts.present(3)
    with pytest.raises(KeyError, match="L5E5"):
        moe.experts.fetch([H.ExpertKey(LAYER, 3), H.ExpertKey(LAYER, 5)])
    assert moe.experts.routing_counts()[5] == 1
    s = moe.experts.stats()
    assert (s.pinned_hits, s.misses, s.pinned_experts) == (0, 0, 4)
    with pytest.raises(ValueError):
        moe.experts.fetch([H.ExpertKey(LAYER, E)])       # past the layer's experts
    with pytest.raises(ValueError):
        moe.experts.fetch([H.ExpertKey(LAYER + 1, 0)])   # another layer's key
    moe.close()


def test_fetch_misses_load_from_the_source(ctx, oracle_layer, tmp_path):
    """An empty layer with its pack as source: misses load the records into
    HBM (a key missing twice in one request is two misses and its bytes
    count twice, as the reference counts them), later requests hit, a
    whole-layer load adds its bytes and time, and the forward then equals
    the oracle's."""
    L = oracle_layer
    h = write_pack(tmp_path / "e.hpk", L)
    pack = H.PackExpertSource.open(tmp_path / "e.hpk")
    moe = new_layer(ctx, L)
    moe.set_source(pack)
    rb = h["record_bytes"]
    got = moe.experts.fetch([H.ExpertKey(LAYER, e) for e in (2, 5, 2)])
    s = moe.experts.stats()
    assert (s.pinned_hits, s.misses, s.bytes_loaded, s.pinned_experts) == (0, 3, 3 * rb, 2)
    assert s.load_seconds > 0 and s.load_gbps() > 0
    x = O.normal(14, HID)
    for e, ex in zip((2, 5, 2), got):
        assert same_bits(ex.forward(x), expert_out(L, e, x))
    assert moe.experts.present(2) and moe.experts.present(5) and not moe.experts.present(0)
    moe.experts.fetch([H.ExpertKey(LAYER, 5)])
    s2 = moe.experts.stats()
    assert (s2.pinned_hits, s2.misses) == (1, 3)
    assert s2.hit_rate() == 0.25
    moe.load_pack(pack)  # the rest of the layer
    s3 = moe.experts.stats()
    assert s3.pinned_experts == E and s3.bytes_loaded == (3 + E) * rb
    assert s3.load_seconds > s2.load_seconds
    out, idx, w = moe.forward(x, return_routes=True)
    o_out, o_idx, o_w = L.forward(x)
    assert list(idx) == list(o_idx) and same_bits(w, o_w) and same_bits(out, o_out)
    assert list(moe.experts.routing_counts()) == list(
        np.bincount([2, 5, 2, 5] + list(o_idx), minlength=E))
    moe.close()
    pack.close()


def test_source_binding(ctx, oracle_layer, tmp_path):
    """set_source checks the pack like a load does; None unbinds, and closing
    the pack unbinds it from its layers, so misses are KeyError again."""
    L = oracle_layer
    write_pack(tmp_path / "e.hpk", L)
    other = O.OracleMoe.synthetic(L.dtype, HID, 2 * INTER, E, K, seed=3)
    h2 = P.header_for(L.dtype, HID, 2 * INTER, E, [LAYER])
    P.write_pack(tmp_path / "wide.hpk", h2, {})
    wide = H.PackExpertSource.open(tmp_path / "wide.hpk")
    moe = new_layer(ctx, L)
    with pytest.raises(ValueError, match="does not match"):
        moe.set_source(wide)
    pack = H.PackExpertSource.open(tmp_path / "e.hpk")
    moe.set_source(pack)
    moe.set_source(None)
    with pytest.raises(KeyError):
        moe.experts.fetch([H.ExpertKey(LAYER, 1)])
    moe.set_source(pack)
    moe.experts.fetch([H.ExpertKey(LAYER, 1)])
    pack.close()
    with pytest.raises(KeyError):
        moe.experts.fetch([H.ExpertKey(LAYER, 2)])
    assert moe.experts.present(1)
    moe.close()
    wide.close()
    del other


def test_views_belong_to_the_layer(ctx, oracle_layer):
    """Closing a fetched matrix leaves the layer's expert intact: a later
    fetch returns the same weights and the forward is unchanged."""
    L = oracle_layer
    moe = new_layer(ctx, L, range(E))
    x = O.normal(15, HID)
    want, _, _ = L.forward(x)
    ex = moe.experts.fetch([H.ExpertKey(LAYER, 4)])[0]
    for m in (ex.gate, ex.up, ex.down):
        m.close()
    ex2 = moe.experts.fetch([H.ExpertKey(LAYER, 4)])[0]
    assert same_bits(ex2.forward(x), expert_out(L, 4, x))
    assert same_bits(moe.forward(x), want)
    moe.close()


def test_views_outliving_their_layer_free_nothing(ctx, oracle_layer):
    """A fetched expert kept after its layer is closed: closing or dropping
    it must not touch the layer's (freed) memory."""
    L = oracle_layer
    moe = new_layer(ctx, L, range(E))
    ex = moe.experts.fetch([H.ExpertKey(LAYER, 1)])[0]
    moe.close()
    for m in (ex.gate, ex.up, ex.down):
        m.close()
    del ex
    moe2 = new_layer(ctx, L, range(E))  # the context still works
    x = O.normal(16, HID)
    assert same_bits(moe2.experts.fetch([H.ExpertKey(LAYER, 1)])[0].forward(x), expert_out(L, 1, x))
    moe2.close()
