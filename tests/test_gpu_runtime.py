"""Graph capture and scratch lifetime of the MoE layer, through the C ABI.

A captured graph keeps the device addresses of the layer's per-token
scratch.  The runtime must (a) refuse to grow scratch while the stream is
being captured (growing synchronizes and allocates), and (b) keep scratch
that a later, larger call outgrows alive until the graphs that may use it
are destroyed, so that replaying an older graph stays correct.  Every
replay is checked against the eager result, with eager work and
synchronizations between the replays.
"""
import numpy as np
import pytest

import hale_moe as H
import oracle as O

pytestmark = pytest.mark.gpu

E, HID, INTER, K = 16, 256, 64, 4


def make_layer(ctx, L):
    router = H.WeightMatrix.new(ctx, L.num_experts, L.hidden, "f32", L.router.view(np.uint8))
    moe = H.MoeLayer(ctx, 0, L.num_experts, L.hidden, L.inter, L.dtype, L.top_k, L.normalize, router)
    for e in range(L.num_experts):
        moe.set_expert(e, L.gate[e], L.up[e], L.down[e])
    return moe


@pytest.fixture
def layer(ctx):
    L = O.OracleMoe.synthetic(O.Q4_0, HID, INTER, E, K, normalize_topk=True, seed=21)
    moe = make_layer(ctx, L)
    yield L, moe
    moe.close()


def test_capture_refuses_scratch_growth(ctx, layer):
    """A layer that has never run a token has no scratch: capturing its first
    forward would have to allocate, so the call fails with ValueError and the
    capture ends cleanly; after one eager call the same capture works."""
    L, moe = layer
    x, out = ctx.malloc(HID * 4), ctx.malloc(HID * 4)
    x.upload(O.normal(1, HID))
    with pytest.raises(ValueError, match="captured"):
        ctx.capture(lambda: moe.forward_device(1, x.address, out.address))
    moe.forward_device(1, x.address, out.address)  # sizes the scratch eagerly
    ctx.synchronize()
    g = ctx.capture(lambda: moe.forward_device(1, x.address, out.address))
    g.launch()
    ctx.synchronize()
    o_out, _, _ = L.forward(O.normal(1, HID))
    assert (out.download(np.float32, HID).view(np.uint32) == o_out.view(np.uint32)).all()
    g.close()
    for b in (x, out):
        b.free()


@pytest.mark.parametrize("T", [3, 24])
def test_reserve_sizes_scratch_for_capture(ctx, layer, T):
    """hale_moe_reserve sizes the layer's scratch (and from the grouped
    threshold on, 11 tokens for this top-4 q4_0 layer, its grouped workspace) so
    that the first forward can be captured; replays are bit-exact.  A
    reserve that would have to grow scratch during a capture is refused."""
    L, moe = layer
    moe.reserve(T)
    bx, bo = ctx.malloc(T * HID * 4), ctx.malloc(T * HID * 4)
    xs = O.normal(40 + T, T * HID).reshape(T, HID)
    bx.upload(xs)
    g = ctx.capture(lambda: moe.forward_device(T, bx.address, bo.address))
    want, _, _ = L.prefill(xs)
    for rep in range(2):
        g.launch()
        ctx.synchronize()
        got = bo.download(np.float32, T * HID).reshape(T, HID)
        assert (got.view(np.uint32) == want.view(np.uint32)).all(), rep
    g.close()
    with pytest.raises(ValueError, match="captured"):
        ctx.capture(lambda: moe.reserve(64))
    moe.reserve(64)  # outside a capture it grows
    for b in (bx, bo):
        b.free()


@pytest.mark.parametrize("big", [5, 24])
def test_graph_replays_after_scratch_grows(ctx, layer, big):
    """Capture a one-token forward, then grow the layer's scratch with an
    eager forward of `big` tokens (decode path at 5, grouped path at 24):
    the old graph still replays correctly, replay after replay, with eager
    work between the replays."""
    L, moe = layer
    x1 = O.normal(2, HID)
    xs = O.normal(3, big * HID).reshape(big, HID)
    bx, bo = ctx.malloc(HID * 4), ctx.malloc(HID * 4)
    bxs, bos = ctx.malloc(big * HID * 4), ctx.malloc(big * HID * 4)
    bx.upload(x1)
    bxs.upload(xs)
    moe.forward_device(1, bx.address, bo.address)
    ctx.synchronize()
    g = ctx.capture(lambda: moe.forward_device(1, bx.address, bo.address))
    want1, _, _ = L.forward(x1)
    wantn, _, _ = L.prefill(xs)
    for rep in range(4):
        bo.upload(np.zeros(HID, np.float32))
        g.launch()
        ctx.synchronize()
        assert (bo.download(np.float32, HID).view(np.uint32) == want1.view(np.uint32)).all(), rep
        moe.forward_device(big, bxs.address, bos.address)  # grows scratch on the first pass
        ctx.synchronize()
        got = bos.download(np.float32, big * HID).reshape(big, HID)
        assert (got.view(np.uint32) == wantn.view(np.uint32)).all(), rep
    g.close()  # frees the retired scratch
    moe.forward_device(1, bx.address, bo.address)
    ctx.synchronize()
    assert (bo.download(np.float32, HID).view(np.uint32) == want1.view(np.uint32)).all()
    for b in (bx, bo, bxs, bos):
        b.free()


@pytest.mark.parametrize("T", [12, 24])
def test_graph_of_grouped_forward_replays(ctx, layer, T):
    """A captured grouped (multi-token) forward replays bit-exact, several
    times, with different inputs uploaded between the replays: 12 tokens
    on the row-chain kernels (up to 14 tokens for this layer), 24 on the
    matrix products."""
    L, moe = layer
    bx, bo = ctx.malloc(T * HID * 4), ctx.malloc(T * HID * 4)
    bx.upload(O.normal(4, T * HID))
    moe.forward_device(T, bx.address, bo.address)
    ctx.synchronize()
    g = ctx.capture(lambda: moe.forward_device(T, bx.address, bo.address))
    for rep in range(3):
        xs = O.normal(10 + rep, T * HID).reshape(T, HID)
        bx.upload(xs)
        g.launch()
        ctx.synchronize()
        want, _, _ = L.prefill(xs)
        got = bo.download(np.float32, T * HID).reshape(T, HID)
        assert (got.view(np.uint32) == want.view(np.uint32)).all(), rep
    g.close()
    for b in (bx, bo):
        b.free()


def test_graph_of_two_tile_decode_replays(ctx):
    """A decode whose gate/up grid is larger than the GPU holds at once (two
    tiles per work-group) replays bit-exact from a graph, several times, and
    so does an eager call between the replays."""
    L = O.OracleMoe.synthetic(O.Q8_0, 256, 2080, 8, 8, normalize_topk=True, seed=31)
    moe = make_layer(ctx, L)
    bx, bo = ctx.malloc(256 * 4), ctx.malloc(256 * 4)
    bx.upload(O.normal(5, 256))
    moe.forward_device(1, bx.address, bo.address)
    ctx.synchronize()
    g = ctx.capture(lambda: moe.forward_device(1, bx.address, bo.address))
    for rep in range(4):
        x = O.normal(40 + rep, 256)
        bx.upload(x)
        if rep == 2:
            moe.forward_device(1, bx.address, bo.address)
        else:
            g.launch()
        ctx.synchronize()
        want, _, _ = L.forward(x, nthreads=8)
        got = bo.download(np.float32, 256)
        assert (got.view(np.uint32) == want.view(np.uint32)).all(), rep
    g.close()
    moe.close()
    for b in (bx, bo):
        b.free()
