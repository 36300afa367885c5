"""hale_moe_forward_device_noalloc against hale_moe_forward_device, through
the C ABI: the same layer and inputs give the same bits (outputs, routes,
weights) on two calls in a row, the second smaller than the first, and a
call whose scratch would exceed the fixed array is refused before anything
runs."""
import numpy as np
import pytest

import hale_moe as H
import oracle as O

pytestmark = pytest.mark.gpu

E, HID, INTER, K = 16, 256, 64, 4


@pytest.fixture(scope="module")
def layer(ctx):
    L = O.OracleMoe.synthetic(O.Q4_0, HID, INTER, E, K, normalize_topk=True, seed=61)
    router = H.WeightMatrix.new(ctx, E, HID, "f32", L.router.view(np.uint8))
    moe = H.MoeLayer(ctx, 0, E, HID, INTER, L.dtype, K, True, router)
    for e in range(E):
        moe.set_expert(e, L.gate[e], L.up[e], L.down[e])
    yield L, moe
    moe.close()


def run(ctx, moe, fn, xs, logits):
    T = xs.shape[0]
    bx, bl = ctx.malloc(xs.nbytes), ctx.malloc(max(logits.nbytes, 4) if logits is not None else 4)
    bo, bi, bw = ctx.malloc(xs.nbytes), ctx.malloc(T * K * 4), ctx.malloc(T * K * 4)
    bx.upload(xs)
    if logits is not None:
        bl.upload(logits)
    bo.upload(np.full(xs.size, np.nan, np.float32))
    fn(T, bx.address, bo.address, bl.address if logits is not None else 0, bi.address, bw.address)
    ctx.synchronize()
    res = (bo.download(np.float32, xs.size).reshape(xs.shape), bi.download(np.uint32, T * K),
           bw.download(np.float32, T * K))
    for b in (bx, bl, bo, bi, bw):
        b.free()
    return res


@pytest.mark.parametrize("with_logits", [False, True])
def test_noalloc_forward_equals_forward_device(ctx, layer, with_logits):
    L, moe = layer
    # 40 tokens (grouped path), then 3 (decode path) in the same fixed scratch
    for T, seed in ((40, 1), (3, 2)):
        xs = O.normal(seed, T * HID).reshape(T, HID)
        lg = O.normal(seed + 50, T * E).reshape(T, E) if with_logits else None
        got = run(ctx, moe, moe.forward_device_noalloc, xs, lg)
        want = run(ctx, moe, moe.forward_device, xs, lg)
        assert (got[0].view(np.uint32) == want[0].view(np.uint32)).all(), T
        assert (got[1] == want[1]).all() and (got[2].view(np.uint32) == want[2].view(np.uint32)).all()
        o_out, o_idx, o_w = L.prefill(xs, logits=lg)
        assert (got[0].view(np.uint32) == o_out.view(np.uint32)).all(), T
        assert (got[1].reshape(T, K) == o_idx).all()


def test_noalloc_refuses_more_than_the_fixed_scratch(ctx, layer):
    L, moe = layer
    T = 5000  # the grouped workspace alone needs T * K * HID * 4 = 20 MB
    bx, bo = ctx.malloc(T * HID * 4), ctx.malloc(T * HID * 4)
    with pytest.raises(ValueError, match="fixed scratch"):
        moe.forward_device_noalloc(T, bx.address, bo.address)
    for b in (bx, bo):
        b.free()
    # the layer still works afterwards
    xs = O.normal(9, 2 * HID).reshape(2, HID)
    got = run(ctx, moe, moe.forward_device_noalloc, xs, None)
    o_out, _, _ = L.prefill(xs)
    assert (got[0].view(np.uint32) == o_out.view(np.uint32)).all()
