"""GPU parity of the expert-grouped multi-token path (ntok at or above the
layer's grouped threshold: for top-4 and wider 11 tokens (q4_0, hidden
size up to 2048), 9 (q4_0, wider) or 12 (q8_0), 7 below; the
row-chain kernels up to the layer's band threshold, the int8 matrix
products above it) against the oracle's token-at-a-time prefill
(src/model/transformer.rs:231-239).

Bar: bit-exact outputs, routes and weights (rel-L2 <= 1e-5 asserted too).
Both model-shaped workloads (512 tokens of Qwen3-30B-A3B q8_0 and 2048 of
Qwen3-235B-A22B q4_0) are checked on every token against the oracle; the
2048-token one also against the decode path (one token per call).
"""
import numpy as np
import pytest

import hale_moe as H
from hale_moe.synth import zipf_logits
import oracle as O

pytestmark = pytest.mark.gpu

REL_L2 = 1e-5


def same_bits(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and bool((a.view(np.uint32) == b.view(np.uint32)).all())


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def make_layer(ctx, L, layer_id=0):
    router = None
    if L.router is not None:
        router = H.WeightMatrix.new(ctx, L.num_experts, L.hidden, "f32", L.router.view(np.uint8))
    moe = H.MoeLayer(ctx, layer_id, L.num_experts, L.hidden, L.inter, L.dtype, L.top_k,
                     L.normalize, router)
    for e in range(L.num_experts):
        moe.set_expert(e, L.gate[e], L.up[e], L.down[e])
    return moe


def check(moe, L, xs, logits=None, sample=None):
    out, idx, w = moe.forward(xs, logits=logits, return_routes=True)
    toks = range(xs.shape[0]) if sample is None else sample
    for t in toks:
        o, i, ww = L.forward(xs[t], logits=None if logits is None else logits[t], nthreads=8)
        assert list(idx[t]) == list(i), t
        assert same_bits(w[t], ww), t
        assert rel_l2(out[t], o) <= REL_L2, t
        assert same_bits(out[t], o), t
    return out, idx


@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_0])
@pytest.mark.parametrize("with_router", [False, True])
def test_grouped_small(ctx, dtype, with_router):
    E, Hd, I, k, T = 32, 256, 96, 4, 40
    L = O.OracleMoe.synthetic(dtype, Hd, I, E, k, normalize_topk=True, seed=5, with_router=with_router)
    moe = make_layer(ctx, L)
    xs = O.normal(3, T * Hd).reshape(T, Hd)
    logits = None if with_router else zipf_logits(T, E, 1.1, seed=2)
    check(moe, L, xs, logits)


@pytest.mark.parametrize("dtype,Hd,I,E,k,T", [
    (H.Q4_0, 2048, 64, 128, 8, 64),    # 48+ tokens: the router's 8-expert x 8-token tiles (64 of 16 would leave CUs idle)
    (H.Q4_0, 256, 64, 256, 8, 128),    # 16-expert tiles (256 of them)
    (H.Q8_0, 512, 64, 264, 4, 129),    # 16-expert tiles, a partial expert and a partial token tile
    (H.Q8_0, 1024, 64, 32, 6, 49),     # ... from 48 tokens: a partial token tile of one
    (H.Q4_0, 2048, 64, 128, 8, 47),    # one work-group per (expert, token): 6016 of them
    (H.Q8_0, 4160, 64, 16, 4, 40),     # ... rows of 4160 (registers and LDS sized for 8192)
    (H.Q8_0, 2080, 64, 20, 4, 100),    # a partial expert tile, a partial token tile, a partial chunk (260 steps)
    (H.Q4_0, 4096, 64, 128, 8, 72),    # 512 steps: eight chunks
])
def test_grouped_router_many_tokens(ctx, dtype, Hd, I, E, k, T):
    """The router over many tokens (tiles of router rows and tokens in LDS,
    products formed in the chains): routes, weights (the softmax over every
    logit) and outputs have the reference's bits for every token."""
    L = O.OracleMoe.synthetic(dtype, Hd, I, E, k, normalize_topk=True, seed=Hd + E + T,
                              with_router=True)
    moe = make_layer(ctx, L)
    xs = O.normal(T + Hd, T * Hd).reshape(T, Hd)
    check(moe, L, xs)
    moe.close()


@pytest.mark.parametrize("dtype,Hd,I,E,k,T,with_router", [
    (H.Q4_0, 256, 96, 32, 4, 40, True),     # 8-block gate/up rows; down rows of 3 blocks (a partial ring cycle)
    (H.Q8_0, 256, 96, 32, 4, 40, False),
    (H.Q4_0, 2048, 64, 128, 8, 64, True),   # the tiled router feeding the row chains
    (H.Q8_0, 1024, 64, 32, 6, 33, True),
    (H.Q4_0, 2080, 96, 20, 4, 100, True),   # 65-block rows; 65 down tiles (a spare wave per tile)
    (H.Q8_0, 4096, 64, 128, 8, 16, True),   # 128-block rows
    (H.Q4_0, 8192, 64, 8, 2, 5, False),     # 256-block rows: the most activation blocks staged
    (H.Q4_0, 512, 1024, 8, 2, 9, False),    # top-2, 32-block down rows (a ring of 16)
    (H.Q8_0, 256, 160, 4, 4, 30, False),    # 4 experts: every expert in many two-row tiles
    (H.Q8_0, 32, 32, 4, 2, 6, False),       # one block per row, one output tile: spare waves
    (H.Q4_0, 64, 32, 1024, 1, 40, True),    # 1024 experts, top-1
    (H.Q8_0, 256, 9216, 4, 2, 6, False),    # 288-block down rows: the 512-block staging
    # tiles of four (two or more assignments per expert, gate/up rows of 2 KB or more)
    (H.Q8_0, 2048, 96, 16, 4, 8, True),     # exactly two per expert: tiles of four, non-temporal loads
    (H.Q8_0, 2048, 96, 16, 4, 20, False),   # Zipf: tiles of 1-4 rows, ordinary loads
    (H.Q4_0, 4096, 64, 16, 4, 12, True),    # q4_0 (broadcast activation reads)
    (H.Q4_0, 4096, 1056, 8, 2, 13, False),  # q4_0 down rows of 33 blocks (a ring of 16)
    (H.Q4_0, 8192, 64, 8, 2, 9, False),     # 256-block rows: four rows' activations staged
])
def test_band_row_chains(ctx, dtype, Hd, I, E, k, T, with_router):
    """The row-chain grouped kernels (two or four assignments of an expert
    per tile, a lane per weight row, the activations as scalar operands),
    forced for every call: routes, weights and outputs bit-exact per token
    against the oracle, and the same bits as the grouped matrix products."""
    L = O.OracleMoe.synthetic(dtype, Hd, I, E, k, normalize_topk=True, seed=Hd + I + T,
                              with_router=with_router)
    moe = make_layer(ctx, L)
    moe.set_grouped_min_tokens(2)
    moe.set_band_max_tokens(1 << 20)
    xs = O.normal(T + 7, T * Hd).reshape(T, Hd)
    logits = None if with_router else zipf_logits(T, E, 1.1, seed=3)
    out, _ = check(moe, L, xs, logits)
    moe.set_band_max_tokens(0)
    assert same_bits(moe.forward(xs, logits=logits), out)
    moe.close()


@pytest.mark.parametrize("T,bmax", [(16, None), (24, None), (48, None), (64, None), (80, 1 << 20)])
def test_band_qwen30b_q4(ctx, T, bmax):
    """Qwen3-30B-A3B's layer shape (128 q4_0 experts, H 2048, I 768, top-8)
    at 16, 24 (non-temporal weight loads), 48 and 64 tokens (cached loads;
    the default row-chain range is 11 to 76) and at 80 with the row chains
    forced: every token against the oracle."""
    E, Hd, I, k = 128, 2048, 768, 8
    L = O.OracleMoe.synthetic(H.Q4_0, Hd, I, E, k, normalize_topk=True, seed=50 + T, with_router=True)
    moe = make_layer(ctx, L)
    assert moe.grouped_min_tokens == 11 and moe.band_max_tokens == 76
    if bmax is not None:
        moe.set_band_max_tokens(bmax)
    xs = O.normal(60 + T, T * Hd).reshape(T, Hd)
    check(moe, L, xs)
    moe.close()


def test_band_mixtral_8_tokens(ctx):
    """Mixtral-8x7B's layer shape (8 q4_0 experts, H 4096, I 14336, top-2)
    at 8 tokens, its default path (grouped from 7 tokens, row chains up to
    13; 448-block down rows): every token against the oracle."""
    E, Hd, I, k, T = 8, 4096, 14336, 2, 8
    L = O.OracleMoe.synthetic(H.Q4_0, Hd, I, E, k, normalize_topk=True, seed=88, with_router=True)
    moe = make_layer(ctx, L)
    assert moe.grouped_min_tokens == 7 and moe.band_max_tokens == 13
    check(moe, L, O.normal(89, T * Hd).reshape(T, Hd))
    moe.close()


def test_band_crowded_experts(ctx):
    """The row chains with every token on the same two experts (ten two-row
    tiles each) and the others idle."""
    E, Hd, I, k, T = 16, 128, 64, 2, 20
    L = O.OracleMoe.synthetic(O.Q8_0, Hd, I, E, k, normalize_topk=False, seed=19, with_router=False)
    moe = make_layer(ctx, L)
    moe.set_grouped_min_tokens(2)
    moe.set_band_max_tokens(T)
    xs = O.normal(14, T * Hd).reshape(T, Hd)
    logits = np.full((T, E), -5.0, np.float32)
    logits[:, 5] = 2.0
    logits[:, 9] = 1.0
    out, idx = check(moe, L, xs, logits)
    assert (idx[:, 0] == 5).all() and (idx[:, 1] == 9).all()
    moe.close()


def test_grouped_empty_and_crowded_experts(ctx):
    """Every token on the same experts (one group of T rows, many tiles) and
    most experts idle."""
    E, Hd, I, k, T = 16, 128, 64, 2, 100
    L = O.OracleMoe.synthetic(O.Q4_0, Hd, I, E, k, normalize_topk=False, seed=9, with_router=False)
    moe = make_layer(ctx, L)
    xs = O.normal(4, T * Hd).reshape(T, Hd)
    logits = np.full((T, E), -5.0, np.float32)
    logits[:, 3] = 2.0
    logits[:, 11] = 1.0
    out, idx = check(moe, L, xs, logits)
    assert (idx[:, 0] == 3).all() and (idx[:, 1] == 11).all()


def test_grouped_ties_in_routing(ctx):
    """Equal logits: top-k takes the lowest indices."""
    E, Hd, I, k, T = 8, 64, 32, 3, 12
    L = O.OracleMoe.synthetic(O.Q8_0, Hd, I, E, k, normalize_topk=True, seed=1, with_router=False)
    moe = make_layer(ctx, L)
    xs = O.normal(6, T * Hd).reshape(T, Hd)
    logits = np.zeros((T, E), np.float32)
    out, idx = check(moe, L, xs, logits)
    assert (idx == np.array([0, 1, 2])).all()


def test_grouped_qwen30b_prefill_512_q8(ctx):
    """128 q8_0 experts (H 2048, I 768), top-8, 512 tokens, Zipf routing."""
    E, Hd, I, k, T = 128, 2048, 768, 8, 512
    L = O.OracleMoe.synthetic(O.Q8_0, Hd, I, E, k, normalize_topk=True, seed=33, with_router=False)
    moe = make_layer(ctx, L)
    xs = O.normal(7, T * Hd).reshape(T, Hd)
    logits = zipf_logits(T, E, 1.1, seed=3)
    _, idx = check(moe, L, xs, logits)  # every token against the oracle
    # routing counts (added once per expert by the grouping kernel) equal
    # the selections, over two forwards
    moe.forward(xs, logits=logits)
    counts = moe.experts.routing_counts()
    assert (counts == 2 * np.bincount(idx.ravel(), minlength=E)).all()


def test_grouped_qwen235b_prefill_2048_q4(ctx):
    """128 q4_0 experts (H 4096, I 1536), top-8, 2048 tokens, Zipf routing;
    every token against the oracle's token-at-a-time prefill (its tokens
    shared among the host's threads), and every token against the decode
    path (one token per call)."""
    E, Hd, I, k, T = 128, 4096, 1536, 8, 2048
    L = O.OracleMoe.synthetic(O.Q4_0, Hd, I, E, k, normalize_topk=True, seed=44, with_router=False)
    moe = make_layer(ctx, L)
    xs = O.normal(8, T * Hd).reshape(T, Hd)
    logits = zipf_logits(T, E, 1.1, seed=4)
    out, idx, w = moe.forward(xs, logits=logits, return_routes=True)
    o_out, o_idx, o_w = L.prefill(xs, logits=logits, nthreads=O.max_threads())
    assert (idx == o_idx).all()
    assert same_bits(w, o_w)
    assert rel_l2(out, o_out) <= REL_L2
    bad = np.nonzero((out.view(np.uint32) != o_out.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} tokens differ, first {bad[:8].tolist()}"
    for t in range(T):
        o, i, _ = moe.forward(xs[t], logits=logits[t], return_routes=True)
        assert list(i) == list(idx[t]), t
        assert same_bits(o, out[t]), t


@pytest.mark.parametrize("bmax", [None, 0])
def test_grouped_equals_decode_path(ctx, bmax):
    """The grouped path over 24 tokens (this top-6 layer's row-chain kernels,
    up to 50 tokens; with them off, the matrix products) and the decode
    path (one token at a time) give the same bits."""
    E, Hd, I, k, T = 64, 512, 128, 6, 24
    L = O.OracleMoe.synthetic(O.Q4_0, Hd, I, E, k, normalize_topk=True, seed=12, with_router=True)
    moe = make_layer(ctx, L)
    assert moe.band_max_tokens == 50
    if bmax is not None:
        moe.set_band_max_tokens(bmax)
    xs = O.normal(9, T * Hd).reshape(T, Hd)
    batch = moe.forward(xs)
    for t in range(T):
        assert same_bits(moe.forward(xs[t]), batch[t])


@pytest.mark.parametrize("dtype,Hd,I,E,k,T,seed", [
    (O.Q8_0, 2048, 768, 128, 8, 512, 33),    # the Qwen3-30B-A3B prefill shape
    (O.Q4_0, 4096, 1536, 128, 8, 2048, 44),  # the Qwen3-235B-A22B prefill shape
    (O.Q4_0, 256, 64, 16, 4, 40, 5),
])
def test_grouped_fma_down_fold_within_tolerance(ctx, dtype, Hd, I, E, k, T, seed):
    """The opt-in FMA fold of the grouped down projection: routes and
    weights unchanged, every checked token within rel-L2 1e-5 of the
    oracle's MoeLayer::forward (not bit-exact by design), and switching back
    to the exact fold restores the reference's bits."""
    L = O.OracleMoe.synthetic(dtype, Hd, I, E, k, normalize_topk=True, seed=seed, with_router=False)
    moe = make_layer(ctx, L)
    xs = O.normal(seed + 1, T * Hd).reshape(T, Hd)
    logits = zipf_logits(T, E, 1.1, seed=seed)
    moe.set_down_fold("fma")
    out, idx, w = moe.forward(xs, logits=logits, return_routes=True)
    sample = range(T) if T <= 512 else sorted(
        set(np.random.default_rng(2).choice(T, 24, replace=False).tolist()) | {0, T - 1})
    worst = 0.0
    for t in sample:
        o, o_idx, o_w = L.forward(xs[t], logits=logits[t], nthreads=8)
        assert list(idx[t]) == list(o_idx) and same_bits(w[t], o_w)
        worst = max(worst, rel_l2(out[t], o))
    assert worst <= REL_L2, worst
    moe.set_down_fold("exact")
    exact = moe.forward(xs[:16], logits=logits[:16])
    for t in range(16):
        o, _, _ = L.forward(xs[t], logits=logits[t], nthreads=8)
        assert same_bits(exact[t], o)
    with pytest.raises(ValueError):
        moe.set_down_fold("fast")
    moe.close()
