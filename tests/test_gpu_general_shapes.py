"""GPU parity of the general path: MoE layers, matvecs and expert forwards
whose shapes lie beyond the fast kernels' (more than 1024 experts, top_k
above 64, hidden above 8192, rows of more than 512 blocks).  The reference
has no such limits (src/model/moe.rs:25-70, src/ops/topk.rs:44-61,
src/tensor/matrix.rs:115-143); these layers run the general kernels
(router logits by the f32 GEMV, the any-size routing kernel, lane-per-row
chains, the route-order combine) and must give the oracle's bits.

Bar: bit-exact outputs, routes and weights (rel-L2 <= 1e-5 asserted too).
"""
import numpy as np
import pytest

import hale_moe as H
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


def make_layer(ctx, L):
    router = None
    if L.router is not None:
        router = H.WeightMatrix.new(ctx, L.num_experts, L.hidden, "f32", L.router.view(np.uint8))
    moe = H.MoeLayer(ctx, 0, L.num_experts, L.hidden, L.inter, L.dtype, L.top_k, L.normalize, router)
    for e in range(L.num_experts):
        moe.set_expert(e, L.gate[e], L.up[e], L.down[e])
    return moe


def check(moe, L, xs, logits=None):
    out, idx, w = moe.forward(xs, logits=logits, return_routes=True)
    o_out, o_idx, o_w = L.prefill(xs, logits=logits, nthreads=O.max_threads())
    assert (idx == o_idx).all()
    assert same_bits(w, o_w)
    assert rel_l2(out, o_out) <= REL_L2
    assert same_bits(out, o_out)
    return out, idx


@pytest.mark.parametrize("dtype,Hd,I,E,k,T,with_router", [
    (O.Q8_0, 64, 32, 1100, 6, 1, True),     # more than 1024 experts
    (O.Q4_0, 96, 64, 1100, 8, 40, False),   # ... over 40 tokens, logits given
    (O.Q4_0, 64, 64, 96, 70, 3, True),      # top_k above 64
    (O.Q8_0, 64, 32, 80, 80, 2, False),     # top_k equal to the expert count
    (O.Q4_0, 8224, 64, 4, 2, 2, True),      # hidden above 8192 (router [4 x 8224])
    (O.Q8_0, 64, 16416, 3, 2, 2, True),     # down rows of 513 blocks
])
def test_general_layer_bit_exact(ctx, dtype, Hd, I, E, k, T, with_router):
    L = O.OracleMoe.synthetic(dtype, Hd, I, E, k, normalize_topk=bool(E % 2 == 0), seed=Hd + I + E + k,
                              with_router=with_router)
    moe = make_layer(ctx, L)
    xs = O.normal(T + Hd, T * Hd).reshape(T, Hd)
    logits = None if with_router else O.normal(T + E, T * E, 0.0, 2.0).reshape(T, E)
    check(moe, L, xs, logits)
    if with_router:  # MoeLayer::route on its own
        routes = moe.route(xs[0])
        o_idx, o_w = L.route(xs[0])
        assert [r.key.expert for r in routes] == list(o_idx)
        assert same_bits(np.array([r.weight for r in routes], np.float32), o_w)
    moe.close()


def test_general_routing_ties_and_counts(ctx):
    """Equal logits over 1100 experts: top-70 takes the lowest indices, the
    weights are the reference's 1/70 renormalised, and the routing counts
    record every selection."""
    E, Hd, I, k, T = 1100, 64, 32, 70, 3
    L = O.OracleMoe.synthetic(O.Q8_0, Hd, I, E, k, normalize_topk=True, seed=3, with_router=False)
    moe = make_layer(ctx, L)
    xs = O.normal(5, T * Hd).reshape(T, Hd)
    logits = np.zeros((T, E), np.float32)
    logits[1, 500] = 1.0
    _, idx = check(moe, L, xs, logits)
    assert (idx[0] == np.arange(k)).all()
    counts = moe.experts.routing_counts()
    assert (counts == np.bincount(idx.ravel(), minlength=E)).all()
    moe.close()


def test_general_layer_noalloc_equals_forward_device(ctx):
    E, Hd, I, k, T = 1100, 64, 32, 6, 9
    L = O.OracleMoe.synthetic(O.Q4_0, Hd, I, E, k, normalize_topk=True, seed=8)
    moe = make_layer(ctx, L)
    xs = O.normal(9, T * Hd).reshape(T, Hd)
    bx, bo1, bo2 = ctx.malloc(xs.nbytes), ctx.malloc(xs.nbytes), ctx.malloc(xs.nbytes)
    bx.upload(xs)
    moe.forward_device(T, bx.address, bo1.address)
    moe.forward_device_noalloc(T, bx.address, bo2.address)
    ctx.synchronize()
    a = bo1.download(np.float32, xs.size)
    b = bo2.download(np.float32, xs.size)
    assert same_bits(a, b)
    o_out, _, _ = L.prefill(xs)
    assert same_bits(a.reshape(T, Hd), o_out)
    for buf in (bx, bo1, bo2):
        buf.free()
    moe.close()


@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_0])
@pytest.mark.parametrize("rows,cols", [(100, 20000), (3, 16416), (70, 32800)])
def test_matvec_rows_beyond_512_blocks(ctx, dtype, rows, cols):
    w = O.encode_matrix(dtype, O.normal(rows + cols, rows * cols, 0, 0.02).reshape(rows, cols))
    x = O.normal(7, cols)
    m = H.WeightMatrix.new(ctx, rows, cols, dtype, w)
    got = m.matvec(x)
    want = O.matvec(dtype, rows, cols, w, x, nthreads=8)
    assert rel_l2(got, want) <= REL_L2
    assert same_bits(got, want)
    m.close()


@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_0])
@pytest.mark.parametrize("hidden,inter", [(16416, 64), (64, 16416)])
def test_expert_forward_long_rows(ctx, dtype, hidden, inter):
    """Expert::forward with gate/up rows (hidden) or down rows (inter) of
    more than 512 blocks."""
    g = O.encode_matrix(dtype, O.normal(1, inter * hidden, 0, 0.02).reshape(inter, hidden))
    u = O.encode_matrix(dtype, O.normal(2, inter * hidden, 0, 0.02).reshape(inter, hidden))
    d = O.encode_matrix(dtype, O.normal(3, hidden * inter, 0, 0.02).reshape(hidden, inter))
    x = O.normal(4, hidden)
    ex = H.Expert(H.WeightMatrix.new(ctx, inter, hidden, dtype, g),
                  H.WeightMatrix.new(ctx, inter, hidden, dtype, u),
                  H.WeightMatrix.new(ctx, hidden, inter, dtype, d))
    got = ex.forward(x)
    want = O.expert_forward(dtype, hidden, inter, g, u, d, x)
    assert same_bits(got, want)
    for m in (ex.gate, ex.up, ex.down):
        m.close()
