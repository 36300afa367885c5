"""hale_moe_forward_device_noalloc against hale_moe_forward_device, through
the C ABI: the same layer and inputs give the same bits (outputs, routes,
weights) on two calls in a row, the second smaller than the first; calls
larger than the fixed array run in chunks with the same bits, also at the
Qwen3-30B-A3B and Qwen3-235B-A22B layer shapes; and forwards captured into a
graph on a layer that has never run (so nothing can have been sized before)
replay with the oracle's bits."""
import numpy as np
import pytest

import hale_moe as H
import oracle as O

pytestmark = pytest.mark.gpu

E, HID, INTER, K = 16, 256, 64, 4


def make_layer(ctx, L, layer_id=0):
    router = H.WeightMatrix.new(ctx, L.num_experts, L.hidden, "f32", L.router.view(np.uint8))
    moe = H.MoeLayer(ctx, layer_id, L.num_experts, L.hidden, L.inter, L.dtype, L.top_k, True, router)
    for e in range(L.num_experts):
        moe.set_expert(e, L.gate[e], L.up[e], L.down[e])
    return moe


@pytest.fixture(scope="module")
def layer(ctx):
    L = O.OracleMoe.synthetic(O.Q4_0, HID, INTER, E, K, normalize_topk=True, seed=61)
    moe = make_layer(ctx, L)
    yield L, moe
    moe.close()


def run(ctx, moe, fn, xs, logits, k=K):
    T = xs.shape[0]
    bx, bl = ctx.malloc(xs.nbytes), ctx.malloc(max(logits.nbytes, 4) if logits is not None else 4)
    bo, bi, bw = ctx.malloc(xs.nbytes), ctx.malloc(T * k * 4), ctx.malloc(T * k * 4)
    bx.upload(xs)
    if logits is not None:
        bl.upload(logits)
    bo.upload(np.full(xs.size, np.nan, np.float32))
    fn(T, bx.address, bo.address, bl.address if logits is not None else 0, bi.address, bw.address)
    ctx.synchronize()
    res = (bo.download(np.float32, xs.size).reshape(xs.shape), bi.download(np.uint32, T * k),
           bw.download(np.float32, T * k))
    for b in (bx, bl, bo, bi, bw):
        b.free()
    return res


def same(got, want):
    return ((got[0].view(np.uint32) == want[0].view(np.uint32)).all() and (got[1] == want[1]).all()
            and (got[2].view(np.uint32) == want[2].view(np.uint32)).all())


@pytest.mark.parametrize("with_logits", [False, True])
def test_noalloc_forward_equals_forward_device(ctx, layer, with_logits):
    L, moe = layer
    # 40 tokens (grouped path), then 3 (decode path) in the same fixed scratch
    for T, seed in ((40, 1), (3, 2)):
        xs = O.normal(seed, T * HID).reshape(T, HID)
        lg = O.normal(seed + 50, T * E).reshape(T, E) if with_logits else None
        got = run(ctx, moe, moe.forward_device_noalloc, xs, lg)
        want = run(ctx, moe, moe.forward_device, xs, lg)
        assert same(got, want), T
        o_out, o_idx, o_w = L.prefill(xs, logits=lg)
        assert (got[0].view(np.uint32) == o_out.view(np.uint32)).all(), T
        assert (got[1].reshape(T, K) == o_idx).all()


def test_noalloc_runs_calls_beyond_the_fixed_scratch_in_chunks(ctx, layer):
    """12,000 tokens need more than the fixed array (about 6 KB per token
    on the grouped path here): two chunks, the same bits as one call, and
    routing counts that count every token once."""
    L, moe = layer
    T = 12000
    xs = O.normal(9, T * HID).reshape(T, HID)
    before = moe.experts.routing_counts().copy()
    got = run(ctx, moe, moe.forward_device_noalloc, xs, None)
    mid = moe.experts.routing_counts().copy()
    want = run(ctx, moe, moe.forward_device, xs, None)
    assert same(got, want)
    assert ((mid - before) == np.bincount(got[1], minlength=E)).all()
    sample = [0, 1, 5000, 6001, T - 1]
    o_out, o_idx, _ = L.prefill(xs[sample])
    assert (got[0][sample].view(np.uint32) == o_out.view(np.uint32)).all()


def gpu_layer(ctx, dtype, hid, inter, experts, k, seed):
    """A layer with N(0, 0.02^2) weights and router generated and quantized
    on the GPU (the forward_device path it is compared with is checked
    against the oracle at these shapes by the decode and prefill tests)."""
    ng, nd = inter * H.row_bytes(dtype, hid), hid * H.row_bytes(dtype, inter)
    chunk = 16
    vals = ctx.malloc(chunk * inter * hid * 4)
    aos = [ctx.malloc(chunk * ng), ctx.malloc(chunk * ng), ctx.malloc(chunk * nd)]
    rbuf = ctx.malloc(experts * hid * 4)
    rbuf.fill_normal(seed, experts * hid, 0.0, 0.02)
    rmat = H._vp()
    ctx.check(H.lib().hale_matrix_upload_device(ctx.handle, H.F32, experts, hid, H._vp(rbuf.address),
                                                experts * hid * 4, H.C.byref(rmat)), "router")
    moe = H.MoeLayer(ctx, 0, experts, hid, inter, dtype, k, True,
                     H.WeightMatrix(ctx, rmat, experts, hid, H.F32))
    for e0 in range(0, experts, chunk):
        for j, (rows, cols) in enumerate(((inter, hid), (inter, hid), (hid, inter))):
            vals.fill_normal(seed + 101 * (j + 1) + 1000003 * e0, chunk * rows * cols, 0.0, 0.02)
            ctx.check(H.lib().hale_encode_rows_device(ctx.handle, dtype, chunk * rows, cols,
                                                      H._vp(vals.address), H._vp(aos[j].address)),
                      "encode")
        moe.set_experts_device(e0, chunk, aos[0].address, aos[1].address, aos[2].address)
    for b in (vals, rbuf, *aos):
        b.free()
    return moe


@pytest.mark.parametrize("shape,sizes", [
    ((H.Q4_0, 2048, 768, 128, 8), (3, 16, 64, 700)),   # Qwen3-30B-A3B: 700 tokens take two chunks
    ((H.Q4_0, 4096, 1536, 128, 8), (2, 16, 300)),      # Qwen3-235B-A22B: 300 tokens take two chunks
])
def test_noalloc_at_model_shapes(ctx, shape, sizes):
    dtype, hid, inter, experts, k = shape
    moe = gpu_layer(ctx, dtype, hid, inter, experts, k, seed=hid + inter)
    try:
        for T in sizes:
            print(f"noalloc shape H {hid} I {inter}: {T} tokens", flush=True)
            xs = O.normal(T + hid, T * hid).reshape(T, hid)
            got = run(ctx, moe, moe.forward_device_noalloc, xs, None, k)
            want = run(ctx, moe, moe.forward_device, xs, None, k)
            assert same(got, want), T
    finally:
        moe.close()


def test_noalloc_captured_on_a_fresh_layer(ctx):
    """A new layer's first forwards are no-allocation ones captured into a
    graph (a grouped call, the largest that fits one chunk here, and a
    decode call).  The library refuses to grow scratch while the stream is
    captured, so the capture succeeding shows nothing was allocated.  Every
    replay, with eager work between them, gives the oracle's bits."""
    L = O.OracleMoe.synthetic(O.Q8_0, HID, INTER, E, K, normalize_topk=True, seed=62)
    moe = make_layer(ctx, L, layer_id=1)
    sizes = (2000, 5)
    xs = [O.normal(70 + T, T * HID).reshape(T, HID) for T in sizes]
    bx = [ctx.malloc(x.nbytes) for x in xs]
    bo = [ctx.malloc(x.nbytes) for x in xs]
    for b, x in zip(bx, xs):
        b.upload(x)
    want = [L.prefill(x)[0] for x in xs]
    try:
        g = ctx.capture(lambda: [moe.forward_device_noalloc(T, bx[i].address, bo[i].address)
                                 for i, T in enumerate(sizes)])
        other = ctx.malloc(4096)
        for rep in range(3):
            for b, x in zip(bo, xs):
                b.upload(np.full(x.size, np.nan, np.float32))
            g.launch()
            ctx.synchronize()
            for i, T in enumerate(sizes):
                got = bo[i].download(np.float32, xs[i].size).reshape(xs[i].shape)
                assert (got.view(np.uint32) == want[i].view(np.uint32)).all(), (rep, T)
            other.fill_normal(rep, 1024)  # eager work between replays
            ctx.synchronize()
        g.close()
        other.free()
    finally:
        for b in bx + bo:
            b.free()
        moe.close()
