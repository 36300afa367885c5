"""GPU parity of RMSNorm and one-token attention against the oracle, through
the C ABI.

Bar: bit-exact.  RMSNorm sums the squares in order (src/ops/norm.rs:25-28);
attention keeps the reference's in-order score sums, softmax_in_place and
the position-ordered context (src/model/attention.rs:31-86), so every
output of every position equals the oracle's bits.  The accumulation-order
tolerance (rel-L2 <= 1e-5) is asserted as well.
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


@pytest.mark.parametrize("n", [1, 7, 64, 2048, 4096, 8192])
@pytest.mark.parametrize("eps", [1e-6, 0.0])
def test_rms_norm_bit_exact(ctx, n, eps):
    x = O.normal(n + 1, n, 0.0, 3.0)
    w = O.normal(n + 2, n, 1.0, 0.1)
    got = H.rms_norm(ctx, x, w, eps)
    want = O.rms_norm(x, w, eps)
    assert same_bits(got, want)


def test_rms_norm_reference_case_and_zero_row(ctx):
    x = np.array([3.0, -4.0, 0.0, 5.0], np.float32)
    got = H.rms_norm(ctx, x, np.ones(4, np.float32), 0.0)
    assert same_bits(got, O.rms_norm(x, np.ones(4, np.float32), 0.0))
    z = H.rms_norm(ctx, np.zeros(64, np.float32), np.ones(64, np.float32), 1e-6)
    assert same_bits(z, O.rms_norm(np.zeros(64, np.float32), np.ones(64, np.float32), 1e-6))
    with pytest.raises(ValueError):
        H.rms_norm(ctx, np.zeros(8193, np.float32), np.ones(8193, np.float32), 1e-6)


def test_residual_rms_norm_rows_on_device(ctx):
    rows, n = 5, 2048
    x = O.normal(31, rows * n)
    d = O.normal(32, rows * n)
    w = O.normal(33, n, 1.0, 0.1)
    bx, bd, bw, bo = ctx.malloc(x.nbytes), ctx.malloc(d.nbytes), ctx.malloc(w.nbytes), ctx.malloc(x.nbytes)
    bx.upload(x)
    bd.upload(d)
    bw.upload(w)
    ctx.check(H.lib().hale_rms_norm_device(ctx.handle, H._vp(bx.address), H._vp(bd.address),
                                           H._vp(bw.address), rows, n, np.float32(1e-6),
                                           H._vp(bo.address)), "rms_norm")
    xs = bx.download(np.float32, rows * n).reshape(rows, n)
    got = bo.download(np.float32, rows * n).reshape(rows, n)
    want_x = (x + d).reshape(rows, n)  # add_in_place, one rounding per element
    assert same_bits(xs, want_x)
    for r in range(rows):
        assert same_bits(got[r], O.rms_norm(want_x[r], w, 1e-6))
    for b in (bx, bd, bw, bo):
        b.free()


def build(ctx, dtype, Hd, nh, nkv, hd, seed, qk_norm, max_len):
    mats, gm = [], []
    for j, (r, c) in enumerate(((nh * hd, Hd), (nkv * hd, Hd), (nkv * hd, Hd), (Hd, nh * hd))):
        m = O.encode_matrix(dtype, O.normal(seed + j, r * c, 0.0, 0.05).reshape(r, c))
        mats.append(m)
        gm.append(H.WeightMatrix.new(ctx, r, c, dtype, m))
    qn = kn = None
    if qk_norm:
        qn, kn = O.normal(seed + 10, hd, 1.0, 0.1), O.normal(seed + 11, hd, 1.0, 0.1)
    ref = O.OracleAttention(dtype, Hd, nh, nkv, hd, 1e-6, *mats, q_norm=qn, k_norm=kn, max_len=max_len)
    att = H.Attention(ctx, *gm, qn, kn, nh, nkv, hd, 1e-6, max_len=max_len)
    return ref, att


@pytest.mark.parametrize("dtype,Hd,nh,nkv,hd,qk,steps", [
    (O.F32, 64, 4, 2, 16, True, 40),            # small, GQA group 2
    (O.BF16, 2048, 32, 4, 128, True, 24),       # Qwen3-30B-A3B attention shape
    (O.Q8_0, 2048, 32, 4, 128, True, 12),
    (O.Q4_0, 4096, 32, 8, 128, False, 10),      # Mixtral shape, no QK-norm
])
def test_attention_decode_bit_exact(ctx, dtype, Hd, nh, nkv, hd, qk, steps):
    ref, att = build(ctx, dtype, Hd, nh, nkv, hd, seed=Hd + nh, qk_norm=qk, max_len=64)
    for pos in range(steps):
        x = O.normal(1000 + pos, Hd)
        c, s = O.rope_angles(hd, 1e6, pos)
        got = att.forward(x, pos, c, s)
        want = ref.forward(x, c, s)
        assert rel_l2(got, want) <= REL_L2
        assert same_bits(got, want), (dtype, pos)
    assert len(att) == steps
    att.close()


@pytest.mark.parametrize("nh,nkv,hd", [(8, 2, 32), (16, 2, 16), (16, 1, 16), (6, 2, 16), (4, 4, 16)])
def test_attention_long_context(ctx, nh, nkv, hd):
    # 1100 positions with GQA groups of 4, 8, 16, 3 and 1: 35 score blocks of
    # 32 positions, three softmax pipeline steps of 512, and context passes
    # over five 256-position tiles, so a register stage of the value stream
    # is refilled and both LDS buffers alternate; groups 3 and 1 leave a
    # work-group of the softmax + context kernel with one query head
    ref, att = build(ctx, O.BF16, 256, nh, nkv, hd, seed=77, qk_norm=True, max_len=1100)
    for pos in range(1100):
        x = O.normal(5000 + pos, 256)
        c, s = O.rope_angles(hd, 1e6, pos)
        got = att.forward(x, pos, c, s)
        want = ref.forward(x, c, s)
        if pos % 100 == 99 or pos == 1099:
            assert same_bits(got, want), pos
    att.close()


def test_attention_softmax_past_one_lds_chunk(ctx):
    # rows up to 8192 positions run softmax and context in one kernel, longer
    # ones in two; a score row longer than the softmax keeps in LDS (12288)
    # goes through global memory in chunks: positions on both sides of both
    # limits
    ref, att = build(ctx, O.F32, 64, 4, 2, 16, seed=91, qk_norm=False, max_len=12300)
    for pos in range(12300):
        x = O.normal(100 + pos, 64)
        c, s = O.rope_angles(16, 1e6, pos)
        got = att.forward(x, pos, c, s)
        want = ref.forward(x, c, s)
        if pos in (8190, 8191, 8192, 12286, 12287, 12288, 12299):
            assert same_bits(got, want), pos
    att.close()


def test_attention_position_rules(ctx):
    ref, att = build(ctx, O.F32, 64, 4, 2, 16, seed=3, qk_norm=False, max_len=2)
    c, s = O.rope_angles(16, 1e6, 0)
    x = O.normal(1, 64)
    with pytest.raises(ValueError, match="cache holds 0"):
        att.forward(x, 1, c, s)                 # position must equal the cache length
    att.forward(x, 0, c, s)
    att.forward(x, 1, c, s)
    with pytest.raises(ValueError, match="context overflow"):
        att.forward(x, 2, c, s)
    att.reset()
    assert len(att) == 0
    assert same_bits(att.forward(x, 0, c, s), ref.forward(x, c, s))
    att.close()
