"""GPU parity of the decode path against the CPU oracle, through the C ABI.

Bar: bit-exact.  Quantization codes and scales, per-block i32 sums and the
f32 outputs of matvec, Expert::forward and MoeLayer::forward all equal the
oracle's bits (the kernels keep the reference's left-to-right block order).
The accumulation-order tolerance for f32 outputs, rel-L2 <= 1e-5, is asserted as
well, so a failure reports both.
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


def assert_parity(got, want):
    assert rel_l2(got, want) <= REL_L2
    assert same_bits(got, want)


# ---------------------------------------------------------------------------
# quantization
# ---------------------------------------------------------------------------

def test_act_quant_bit_exact(ctx):
    x = O.normal(1, 4096)
    x[32:64] = 0.0                          # zero block
    x[64:96] *= 1e-30                       # subnormal products
    x[96:128] = O.test_values(32, 3) * 127  # scale exactly near 1
    x[128] = np.inf                         # inf block: scale inf, codes 0
    q = H.Q8Activations.quantize(ctx, x)
    s, c = O.q8_quantize(x)
    assert same_bits(q.scales, s)
    assert (q.quants == c).all()
    with pytest.raises(ValueError):
        H.Q8Activations.quantize(ctx, np.zeros(33, np.float32))


@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_0])
def test_encode_rows_bit_exact(ctx, dtype):
    rows, cols = 96, 256
    v = O.normal(4, rows * cols, 0.0, 0.02).reshape(rows, cols)
    v[0, :32] = 0.0
    v[1, :32] = 1e-6 * O.normal(5, 32)       # f16 subnormal scales
    v[2, :32] = [-8.0, 8.0] + [0.0] * 30     # q4 tie: first wins
    v[3, :32] = [2.5, -2.5, 127.0] + [0.0] * 29
    v[4, :32] = 7e4                          # scale overflows f16 for q4 -> inf
    got = H.encode_rows(ctx, dtype, v)
    want = O.encode_matrix(dtype, v)
    assert (got == want).all()


@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_0])
def test_upload_download_round_trip(ctx, dtype):
    rows, cols = 100, 96   # rows not a multiple of the 64-row group
    w = O.encode_matrix(dtype, O.normal(6, rows * cols, 0, 0.02).reshape(rows, cols))
    m = H.WeightMatrix.new(ctx, rows, cols, dtype, w)
    assert (m.bytes() == w).all()
    with pytest.raises(ValueError):
        H.WeightMatrix.new(ctx, rows, cols, dtype, w[:-1])


# ---------------------------------------------------------------------------
# matvec
# ---------------------------------------------------------------------------

# (4096, 4096) is the reference's kernel benchmark shape; (6000, 4000) has a
# partial last block group and a partial last tile; (10000, 2048) takes
# eight rows per wave (8192 rows and more)
SHAPES = [(768, 2048), (2048, 768), (1536, 4096), (4096, 1536), (32, 64), (100, 96), (4096, 14336),
          (4096, 4096), (6000, 4000), (10000, 2048)]


@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_0])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_matvec_bit_exact(ctx, dtype, rows, cols):
    w = O.encode_matrix(dtype, O.normal(rows + cols, rows * cols, 0, 0.02).reshape(rows, cols))
    x = O.normal(7, cols)
    m = H.WeightMatrix.new(ctx, rows, cols, dtype, w)
    got = m.matvec(x)
    want = O.matvec(dtype, rows, cols, w, x, nthreads=8)
    assert_parity(got, want)
    if rows * cols <= 2048 * 768:
        assert (m.block_sums(x) == O.matvec_block_sums(dtype, rows, cols, w, x)).all()


@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_0])
@pytest.mark.parametrize("shift", [0, 4, 8, 12])
def test_matvec_device_any_x_alignment(ctx, dtype, shift):
    # the activation quantizer reads x 16 bytes at a time when x is 16-byte
    # aligned and value by value otherwise; both give the oracle's bits
    rows, cols = 256, 1024
    w = O.encode_matrix(dtype, O.normal(rows, rows * cols, 0, 0.02).reshape(rows, cols))
    x = O.normal(8, cols)
    x[:32] = 0.0
    m = H.WeightMatrix.new(ctx, rows, cols, dtype, w)
    bx, bo = ctx.malloc(cols * 4 + 16), ctx.malloc(rows * 4)
    bx.upload(x, offset=shift)
    ctx.check(H.lib().hale_matvec_device(ctx.handle, m.handle, H._vp(bx.address + shift),
                                         H._vp(bo.address)), "matvec_device")
    got = bo.download(np.float32, rows)
    assert same_bits(got, O.matvec(dtype, rows, cols, w, x))
    bx.free()
    bo.free()


def test_matvec_rejects_wrong_lengths(ctx):
    w = O.encode_matrix(H.Q8_0, O.normal(1, 64 * 64).reshape(64, 64))
    m = H.WeightMatrix.new(ctx, 64, 64, H.Q8_0, w)
    with pytest.raises(ValueError):
        m.matvec(np.zeros(63, np.float32))
    with pytest.raises(ValueError):
        m.matvec(np.zeros(64, np.float32), out=np.zeros(10, np.float32))


def test_from_f32_quantizes_on_the_gpu(ctx):
    v = O.normal(8, 64 * 128, 0, 0.5)
    m = H.WeightMatrix.from_f32(ctx, 64, 128, "q4_0", v)
    assert (m.bytes() == O.encode_matrix(O.Q4_0, v.reshape(64, 128))).all()


# ---------------------------------------------------------------------------
# Expert::forward
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_0])
@pytest.mark.parametrize("hidden,inter", [(2048, 768), (64, 32), (4096, 1536), (1024, 8256)])
def test_expert_forward_bit_exact(ctx, dtype, hidden, inter):
    # 1024 x 8256: 258 gate/up tiles, more work-groups than the GPU holds at
    # once for q4_0 (16 waves): two tiles per work-group
    L = O.OracleMoe.synthetic(dtype, hidden, inter, 1, 1, seed=hidden + inter, with_router=False)
    gate = H.WeightMatrix.new(ctx, inter, hidden, dtype, L.gate[0])
    up = H.WeightMatrix.new(ctx, inter, hidden, dtype, L.up[0])
    down = H.WeightMatrix.new(ctx, hidden, inter, dtype, L.down[0])
    x = O.normal(9, hidden)
    got = H.Expert(gate, up, down).forward(x)
    want = O.expert_forward(dtype, hidden, inter, L.gate[0], L.up[0], L.down[0], x, nthreads=8)
    assert_parity(got, want)


@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_0])
def test_expert_forward_device_equals_host(ctx, dtype):
    hidden, inter = 2048, 768
    L = O.OracleMoe.synthetic(dtype, hidden, inter, 1, 1, seed=17, with_router=False)
    ex = H.Expert(H.WeightMatrix.new(ctx, inter, hidden, dtype, L.gate[0]),
                  H.WeightMatrix.new(ctx, inter, hidden, dtype, L.up[0]),
                  H.WeightMatrix.new(ctx, hidden, inter, dtype, L.down[0]))
    x = O.normal(19, hidden)
    bx, bo = ctx.malloc(hidden * 4), ctx.malloc(hidden * 4)
    bx.upload(x)
    ex.forward_device(bx.address, bo.address)
    got = bo.download(np.float32, hidden)
    assert same_bits(got, ex.forward(x))
    assert_parity(got, O.expert_forward(dtype, hidden, inter, L.gate[0], L.up[0], L.down[0], x,
                                        nthreads=8))
    bx.free()
    bo.free()


@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_0])
@pytest.mark.parametrize("hidden,inter,shift", [(2048, 768, 4), (8192, 96, 0), (4096, 64, 0),
                                                 (32, 32, 0), (96, 64, 0), (4128, 64, 0)])
def test_expert_forward_device_unfused_activation(ctx, dtype, hidden, inter, shift):
    """The gate/up kernel quantizes an aligned x of up to 128 blocks itself
    (here also 1 and 3 blocks); a misaligned x (shift bytes) or a wider one
    (8192: 256 blocks, 4128: 129) takes the separate quantization kernel.
    Both give the reference's bits."""
    L = O.OracleMoe.synthetic(dtype, hidden, inter, 1, 1, seed=23 + hidden + shift, with_router=False)
    ex = H.Expert(H.WeightMatrix.new(ctx, inter, hidden, dtype, L.gate[0]),
                  H.WeightMatrix.new(ctx, inter, hidden, dtype, L.up[0]),
                  H.WeightMatrix.new(ctx, hidden, inter, dtype, L.down[0]))
    x = O.normal(29, hidden)
    bx, bo = ctx.malloc(hidden * 4 + 16), ctx.malloc(hidden * 4)
    raw = np.zeros(hidden + 4, np.float32)
    raw[shift // 4:shift // 4 + hidden] = x
    bx.upload(raw)
    ex.forward_device(bx.offset(shift), bo.address)
    got = bo.download(np.float32, hidden)
    assert_parity(got, O.expert_forward(dtype, hidden, inter, L.gate[0], L.up[0], L.down[0], x,
                                        nthreads=8))
    bx.free()
    bo.free()


# ---------------------------------------------------------------------------
# MoeLayer
# ---------------------------------------------------------------------------

def make_layer(ctx, L: "O.OracleMoe", layer_id=0):
    router = None
    if L.router is not None:
        router = H.WeightMatrix.new(ctx, L.num_experts, L.hidden, "f32", L.router.view(np.uint8))
    moe = H.MoeLayer(ctx, layer_id, L.num_experts, L.hidden, L.inter, L.dtype, L.top_k,
                     L.normalize, router)
    for e in range(L.num_experts):
        moe.set_expert(e, L.gate[e], L.up[e], L.down[e])
    return moe


@pytest.fixture(scope="module")
def qwen30b_q4(ctx):
    """128 experts, H 2048, I 768, q4_0, top-8 renormalised, f32 router."""
    L = O.OracleMoe.synthetic(O.Q4_0, 2048, 768, 128, 8, normalize_topk=True, seed=101)
    return L, make_layer(ctx, L)


def test_moe_route_matches_oracle(ctx, qwen30b_q4):
    L, moe = qwen30b_q4
    for seed in range(5):
        x = O.normal(1000 + seed, 2048)
        routes = moe.route(x)
        idx, w = L.route(x)
        assert [r.key.expert for r in routes] == list(idx)
        assert same_bits([r.weight for r in routes], w)


def test_moe_decode_qwen30b_q4_bit_exact(ctx, qwen30b_q4):
    L, moe = qwen30b_q4
    for seed in range(4):
        x = O.normal(2000 + seed, 2048)
        out, idx, w = moe.forward(x, return_routes=True)
        o_out, o_idx, o_w = L.forward(x, nthreads=8)
        assert list(idx) == list(o_idx)
        assert same_bits(w, o_w)
        assert_parity(out, o_out)


def test_moe_multi_token_equals_per_token(ctx, qwen30b_q4):
    L, moe = qwen30b_q4
    xs = O.normal(3000, 6 * 2048).reshape(6, 2048)
    out, idx, w = moe.forward(xs, return_routes=True)
    o_out, o_idx, o_w = L.prefill(xs, nthreads=8)
    assert (idx == o_idx).all()
    assert same_bits(w, o_w)
    assert_parity(out, o_out)


def test_routing_stats_count_decode_selections(ctx):
    """The decode path (below the grouped threshold: 6 tokens for this top-3
    layer) counts each token's k experts in the gate/up prologue."""
    L = O.OracleMoe.synthetic(O.Q8_0, 64, 32, 8, 3, seed=5)
    moe = make_layer(ctx, L, layer_id=3)
    xs = O.normal(6, 10 * 64).reshape(10, 64)
    idx = []
    for t in range(7):  # one token at a time
        _, i, _ = moe.forward(xs[t], return_routes=True)
        idx.append(i)
    _, i3, _ = moe.forward(xs[7:10], return_routes=True)  # 3 tokens in one call
    idx = np.concatenate([np.stack(idx), i3])
    counts = moe.experts.routing_counts()
    assert counts.sum() == 30
    assert (counts == np.bincount(idx.ravel(), minlength=8)).all()


def test_routing_stats_count_grouped_selections(ctx):
    """The grouped path (6+ tokens) adds each expert's group size once."""
    L = O.OracleMoe.synthetic(O.Q8_0, 64, 32, 8, 3, seed=5)
    moe = make_layer(ctx, L, layer_id=3)
    xs = O.normal(6, 10 * 64).reshape(10, 64)
    _, idx, _ = moe.forward(xs, return_routes=True)
    counts = moe.experts.routing_counts()
    assert counts.sum() == 30
    assert (counts == np.bincount(idx.ravel(), minlength=8)).all()


def test_missing_expert_is_reported(ctx):
    moe = H.MoeLayer(ctx, 0, 4, 64, 32, "q8_0", 2, True, None)
    with pytest.raises(KeyError):
        moe.forward(np.zeros(64, np.float32), logits=np.zeros(4, np.float32))


@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_0])
@pytest.mark.parametrize("T,gmin,bmax", [(7, None, None), (10, None, None), (11, None, None),
                                         (12, None, None), (21, None, None), (24, None, None),
                                         (40, None, None), (44, None, None),
                                         (8, 8, None), (12, None, 0), (16, 17, None)])
def test_moe_logits_given_zipf_routing(ctx, dtype, T, gmin, bmax):
    """Router logits supplied directly (the skewed-routing workloads).  This
    top-4 layer of 32 experts takes the decode path below 11 tokens (q4_0)
    or 12 (q8_0), the row-chain grouped kernels up to 4.75 * 32 / 4 = 38
    tokens (q4_0) or 5 * 32 / 4 = 40 (q8_0) and the grouped matrix
    products above: 7 and 10 decode, 11 row chains (q4_0) or decode (q8_0),
    12 and 21 row chains (non-temporal weight loads), 24 row
    chains (cached loads: more than two assignments per expert), 40 the
    matrix products (q4_0) or row chains (q8_0), 44 the matrix products;
    then 8 tokens with the threshold set to 8 (row
    chains), 12 with the row chains off (matrix products) and 16 with the
    threshold above them (a decode pass with cached weight loads)."""
    E, Hd, I, k = 32, 256, 64, 4
    L = O.OracleMoe.synthetic(dtype, Hd, I, E, k, normalize_topk=True, seed=77, with_router=False)
    moe = make_layer(ctx, L)
    assert moe.grouped_min_tokens == (11 if dtype == H.Q4_0 else 12)
    assert moe.band_max_tokens == (38 if dtype == H.Q4_0 else 40)
    if gmin:
        moe.set_grouped_min_tokens(gmin)
    if bmax is not None:
        moe.set_band_max_tokens(bmax)
    rng = np.random.default_rng(1)
    p = np.arange(1, E + 1, dtype=np.float64) ** -1.1
    logits = (np.log(p / p.sum())[rng.permutation(E)] + rng.gumbel(size=(T, E))).astype(np.float32)
    xs = O.normal(8, T * Hd).reshape(T, Hd)
    out, idx, w = moe.forward(xs, logits=logits, return_routes=True)
    o_out, o_idx, o_w = L.prefill(xs, logits=logits, nthreads=8)
    assert (idx == o_idx).all()
    assert same_bits(w, o_w)
    assert_parity(out, o_out)


def _few_tokens_check(L, moe, xs):
    """The decode path over T tokens at once, below the layer's grouped
    threshold (one gate/up and one down launch for all of them), against the
    oracle's token-at-a-time forward and against the same layer called one
    token at a time."""
    out, idx, w = moe.forward(xs, return_routes=True)
    o_out, o_idx, o_w = L.prefill(xs, nthreads=8)
    assert (np.asarray(idx) == np.asarray(o_idx)).all()
    assert same_bits(w, o_w)
    assert_parity(out, o_out)
    for t in range(xs.shape[0]):
        assert same_bits(moe.forward(xs[t]), out[t])


@pytest.mark.parametrize("dtype,hidden,inter,E,k,T", [
    (H.Q8_0, 2048, 768, 32, 8, 3),     # q8_0 gate/up at 8 waves: 24 x 24 tile-slots, one tile per work-group
    (H.Q8_0, 2048, 768, 32, 8, 5),     # 24 x 40 = 960 > 512: two tiles per work-group
    (H.Q4_0, 2080, 2080, 6, 2, 5),     # top-2: spread-term down, 65 blocks, 132 x 5 16-row groups (no XCD permutation)
    (H.Q8_0, 1024, 16384, 4, 2, 2),    # top-2, down rows of 512 blocks (the most the spread-term kernel stages)
    (H.Q4_0, 512, 16416, 4, 2, 2),     # top-2, 513 blocks: the pipelined down kernel
    (H.Q8_0, 1024, 1024, 8, 3, 4),     # top-3 q8_0: spread-term down (a ghost half-wave)
    (H.Q4_0, 1024, 8192, 8, 3, 2),     # top-3, 256-block down rows: the whole-chain kernel
    (H.Q4_0, 4096, 1408, 64, 6, 2),    # top-6: spread-term down, three slot pairs (twelve waves)
    (H.Q8_0, 4096, 1024, 16, 5, 1),    # top-5 q8_0: twelve waves, a ghost half-wave
    (H.Q4_0, 4096, 1536, 16, 7, 3),    # top-7: a ghost half-wave, 16-row groups
    (H.Q4_0, 1024, 256, 8, 1, 5),      # top-1: spread-term down, 16-row groups of 4 consecutive blocks per wave-load
    (H.Q8_0, 2048, 4096, 4, 1, 1),     # top-1 q8_0, 128-block down rows, one token
    (H.Q4_0, 5120, 2048, 4, 1, 3),     # top-1, H 5120 (160 tiles): 16-row groups, no XCD permutation
    (H.Q4_0, 256, 64, 300, 16, 3),     # more than 256 experts: eight-wave selection, 16 slots
    (H.Q4_0, 4160, 64, 16, 4, 2),      # spread-term down, top-4, 520 16-row groups (no XCD permutation)
    (H.Q8_0, 4096, 512, 16, 4, 3),     # spread-term down, top-4 q8_0, 16-row groups
    (H.Q4_0, 4096, 1536, 16, 8, 2),    # spread-term down, top-8, 32-row groups (two tokens of H 4096)
    (H.Q8_0, 4096, 512, 16, 4, 2),     # ... q8_0, 32-row groups
])
def test_moe_decode_few_tokens(ctx, dtype, hidden, inter, E, k, T):
    L = O.OracleMoe.synthetic(dtype, hidden, inter, E, k, normalize_topk=True,
                              seed=hidden + inter + E + k + T)
    moe = make_layer(ctx, L)
    _few_tokens_check(L, moe, O.normal(9100 + T, T * hidden).reshape(T, hidden))
    moe.close()


@pytest.mark.parametrize("dtype,hidden,inter,E,k,T", [
    (H.Q4_0, 256, 768, 16, 8, 12),     # q4_0 16-wave gate/up; down rows of 24 blocks
    (H.Q8_0, 512, 1024, 16, 6, 13),    # q8_0 8-wave gate/up; 32 blocks
    (H.Q4_0, 2080, 1536, 16, 8, 14),   # q4_0 rows of 65 blocks: 8-wave gate/up; 48 blocks
    (H.Q8_0, 256, 2048, 16, 5, 17),    # 64 blocks
    (H.Q4_0, 256, 4096, 16, 4, 21),    # 128 blocks
    (H.Q4_0, 256, 64, 300, 8, 12),     # more than 256 experts: the 1024-expert selection
])
def test_moe_decode_cached_weight_loads(ctx, dtype, hidden, inter, E, k, T):
    """Decode passes of 12 to 21 tokens (the grouped threshold raised above
    them; by default these take the grouped path) load the weights through
    the caches: every gate/up form and every down row class of that path,
    bit-exact per token."""
    L = O.OracleMoe.synthetic(dtype, hidden, inter, E, k, normalize_topk=True,
                              seed=hidden + inter + E + k + T)
    moe = make_layer(ctx, L)
    moe.set_grouped_min_tokens(T + 1)
    _few_tokens_check(L, moe, O.normal(9200 + T, T * hidden).reshape(T, hidden))
    moe.close()


@pytest.mark.parametrize("dtype,hidden,inter,k,T", [
    (H.Q4_0, 256, 32, 4, 1),      # one block per row: a partial first group
    (H.Q8_0, 512, 224, 5, 2),     # 7 blocks
    (H.Q4_0, 2048, 768, 6, 1),    # 24 blocks: three whole groups
    (H.Q8_0, 1024, 1280, 7, 3),   # 40 blocks, rows up to 64 blocks staged
    (H.Q4_0, 4096, 2048, 8, 1),   # 64 blocks, the XCD row permutation (512 row groups)
    (H.Q8_0, 256, 2080, 8, 2),    # 65 blocks: the 128-block variant, refilled ring (q8_0)
    (H.Q4_0, 1024, 3200, 4, 4),   # 100 blocks
    (H.Q8_0, 2080, 4096, 8, 1),   # 128 blocks, rows not a multiple of 32 row groups
])
def test_moe_decode_down_one_wave_per_route(ctx, dtype, hidden, inter, k, T):
    """The down projection and combine of 4 to 8 routes over rows of up to
    128 blocks: one work-group per 8 rows, one wave per route folding its
    chains, then the route-order combine; every token bit-exact."""
    E = 16
    L = O.OracleMoe.synthetic(dtype, hidden, inter, E, k, normalize_topk=bool(k % 2),
                              seed=hidden + inter + k + T)
    moe = make_layer(ctx, L)
    _few_tokens_check(L, moe, O.normal(9300 + T, T * hidden).reshape(T, hidden))
    moe.close()


@pytest.mark.parametrize("T", [2, 7, 10, 11, 15, 21])
def test_moe_decode_few_tokens_qwen30b(ctx, qwen30b_q4, T):
    """Config 1's layer over 2, 7 and 10 tokens (below its grouped threshold
    of 11) and, with the threshold raised, 11, 15 and 21: 16-wave gate/up
    with two tiles per work-group (24 tiles x 8 slots x T > 256); from 12
    tokens on the weights load through the caches."""
    L, moe = qwen30b_q4
    assert moe.grouped_min_tokens == 11
    moe.set_grouped_min_tokens(max(11, T + 1))
    try:
        _few_tokens_check(L, moe, O.normal(9200 + T, T * 2048).reshape(T, 2048))
    finally:
        moe.set_grouped_min_tokens(11)


@pytest.mark.parametrize("dtype,hidden,inter,E,k,gmin,bmax", [
    (H.Q4_0, 2048, 768, 128, 8, 11, 76),    # Qwen3-30B-A3B q4_0: 4.75 E / k
    (H.Q4_0, 4096, 1536, 128, 8, 9, 68),    # Qwen3-235B-A22B q4_0: 4.25 E / k
    (H.Q8_0, 2048, 768, 128, 8, 12, 80),    # Qwen3-30B-A3B q8_0: 5 E / k
    (H.Q8_0, 4096, 1536, 128, 8, 8, 60),    # Qwen3-235B-A22B q8_0: 3.75 E / k
    (H.Q4_0, 4096, 14336, 8, 2, 7, 13),     # Mixtral-8x7B: 3.25 E / k (448-block down rows)
])
def test_default_thresholds_by_layer_type(ctx, dtype, hidden, inter, E, k, gmin, bmax):
    """A new layer's grouped and row-chain thresholds follow its type and
    shape (the measured crossovers)."""
    moe = H.MoeLayer(ctx, 0, E, hidden, inter, dtype, k, True, None)
    assert (moe.grouped_min_tokens, moe.band_max_tokens) == (gmin, bmax)
    moe.close()


def test_grouped_threshold_moves_the_path_not_the_bits(ctx):
    """The thresholds only choose the kernels: the same 12 tokens through
    the decode path (threshold 13), the row-chain grouped kernels (threshold
    2 and 12) and the grouped matrix products (row chains off) and one
    token at a time give the same bits.  Out-of-range thresholds are
    refused."""
    L = O.OracleMoe.synthetic(O.Q4_0, 512, 128, 16, 4, normalize_topk=True, seed=41)
    moe = make_layer(ctx, L)
    xs = O.normal(42, 12 * 512).reshape(12, 512)
    o_out, _, _ = L.prefill(xs, nthreads=8)
    assert moe.band_max_tokens == 19
    for gmin, bmax in ((13, 19), (2, 19), (12, 19), (12, 0), (2, 0), (257, 19)):
        moe.set_grouped_min_tokens(gmin)
        moe.set_band_max_tokens(bmax)
        assert moe.grouped_min_tokens == gmin and moe.band_max_tokens == bmax
        assert_parity(moe.forward(xs), o_out)
        assert same_bits(moe.forward(xs[:3]), o_out[:3])
    for bad in (0, 1, 258):
        with pytest.raises(ValueError):
            moe.set_grouped_min_tokens(bad)
    with pytest.raises(ValueError):
        moe.set_band_max_tokens(1 << 40)
    moe.close()


def test_moe_top_k_clamped_and_unnormalised(ctx):
    L = O.OracleMoe.synthetic(O.Q4_0, 64, 32, 4, 6, normalize_topk=False, seed=3)
    moe = make_layer(ctx, L)
    x = O.normal(4, 64)
    out, idx, w = moe.forward(x, return_routes=True)
    o_out, o_idx, o_w = L.forward(x)
    assert len(idx) == 4 and list(idx) == list(o_idx)
    assert same_bits(w, o_w)
    assert_parity(out, o_out)


def test_moe_decode_mixtral_q4_bit_exact(ctx):
    """Mixtral-8x7B-shaped layer: 8 q4_0 experts, H 4096, I 14336 (gate/up
    rows of 2304 B, down rows of 448 blocks), f32 router [8 x 4096], top-2."""
    L = O.OracleMoe.synthetic(O.Q4_0, 4096, 14336, 8, 2, normalize_topk=True, seed=202)
    moe = make_layer(ctx, L)
    for seed in range(3):
        x = O.normal(4000 + seed, 4096)
        out, idx, w = moe.forward(x, return_routes=True)
        o_out, o_idx, o_w = L.forward(x, nthreads=8)
        assert list(idx) == list(o_idx)
        assert same_bits(w, o_w)
        assert_parity(out, o_out)
    # two and three tokens in one decode pass: the down kernel's 32-row and
    # 16-row work-groups (one token took the 16-row ones)
    for T in (2, 3):
        _few_tokens_check(L, moe, O.normal(4100 + T, T * 4096).reshape(T, 4096))
    moe.close()


@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_0])
@pytest.mark.parametrize("hidden,E,k", [(4096, 16, 3), (4096, 8, 8), (4160, 8, 2), (2048, 8, 8),
                                        (2080, 8, 4)])
def test_moe_decode_wide_hidden(ctx, dtype, hidden, E, k):
    # wide hidden sizes for both dtypes; 2, 3, 4 and 8 slots per token.
    # 2 slots run the spread-term down kernel (H 4160: 130 groups of 32
    # rows), 3 the whole-chain one (16-row groups: H 4160 gives 260
    # work-groups, not a multiple of 16, so its XCD permutation is off), 4
    # and 8 a wave per route (8-row groups: H 2080 gives 260, its
    # permutation off too).  Gate/up: H 2048 is one chunk per row (16 waves
    # for q4_0), H 2080 is 65 blocks (8 waves, two chunks)
    L = O.OracleMoe.synthetic(dtype, hidden, 256, E, k, normalize_topk=True, seed=hidden + E + k)
    moe = make_layer(ctx, L)
    for seed in range(2):
        x = O.normal(7000 + seed, hidden)
        out, idx, w = moe.forward(x, return_routes=True)
        o_out, o_idx, o_w = L.forward(x, nthreads=8)
        assert list(idx) == list(o_idx)
        assert same_bits(w, o_w)
        assert_parity(out, o_out)
    moe.close()


def test_copy_device(ctx):
    n = 3 * 1024 * 1024 + 48
    a, b = ctx.malloc(n), ctx.malloc(n)
    a.fill_normal(7, n // 4)
    b.copy_from(a, n)
    assert (b.download(np.uint8, n) == a.download(np.uint8, n)).all()
    with pytest.raises(ValueError):
        b.copy_from(a, n - 8)
    a.free()
    b.free()


from routing_cases import TIE_LOGITS  # noqa: E402


@pytest.mark.parametrize("k", [2, 3])
def test_moe_probability_tie_hidden_in_exp_values(ctx, k):
    L = O.OracleMoe.synthetic(O.Q8_0, 64, 32, 8, k, normalize_topk=True, seed=9, with_router=False)
    moe = make_layer(ctx, L)
    lgs = np.array([t[0] for t in TIE_LOGITS], np.float32)
    xs = O.normal(31, len(TIE_LOGITS) * 64).reshape(-1, 64)
    for t in range(len(TIE_LOGITS)):  # decode path, one token at a time
        out, idx, w = moe.forward(xs[t], logits=lgs[t], return_routes=True)
        o_out, o_idx, o_w = L.forward(xs[t], logits=lgs[t])
        assert list(idx) == list(o_idx)
        assert same_bits(w, o_w)
        assert_parity(out, o_out)
    xs8 = np.repeat(xs, 4, axis=0)  # 8 tokens: the grouped path
    lg8 = np.repeat(lgs, 4, axis=0)
    out, idx, w = moe.forward(xs8, logits=lg8, return_routes=True)
    o_out, o_idx, o_w = L.prefill(xs8, logits=lg8)
    assert (idx == o_idx).all()
    assert same_bits(w, o_w)
    assert_parity(out, o_out)
    moe.close()


@pytest.fixture(scope="module")
def qwen235b_q4(ctx):
    """The Qwen3-235B-A22B decode shape: 128 q4_0 experts, H 4096, I 1536,
    top-8 renormalised, f32 router [128 x 4096]."""
    L = O.OracleMoe.synthetic(O.Q4_0, 4096, 1536, 128, 8, normalize_topk=True, seed=303)
    moe = make_layer(ctx, L)
    yield L, moe
    moe.close()


def test_moe_decode_qwen235b_q4_bit_exact(ctx, qwen235b_q4):
    L, moe = qwen235b_q4
    xs = O.normal(5000, 4 * 4096).reshape(4, 4096)
    for t in range(4):  # one token per call, as the decode loop calls it
        out, idx, w = moe.forward(xs[t], return_routes=True)
        o_out, o_idx, o_w = L.forward(xs[t], nthreads=8)
        assert list(idx) == list(o_idx)
        assert same_bits(w, o_w)
        assert_parity(out, o_out)
    out, idx, w = moe.forward(xs, return_routes=True)  # 4 tokens in one call
    o_out, o_idx, o_w = L.prefill(xs, nthreads=8)
    assert (idx == o_idx).all()
    assert same_bits(w, o_w)
    assert_parity(out, o_out)


@pytest.mark.parametrize("dtype,hidden,inter", [(H.Q4_0, 2048, 2080), (H.Q4_0, 4096, 2080),
                                                (H.Q8_0, 2048, 1056), (H.Q8_0, 4096, 1056)])
def test_moe_decode_down_chunk_boundary(ctx, dtype, hidden, inter):
    """Pipelined down + combine over more (slot, 8-block group) pairs than one
    chunk holds (32 for q4_0, 16 for q8_0): 8 slots x 9 groups = 72 and
    8 x 5 = 40 pairs, with slot 3 straddling the first chunk boundary, so the
    running per-slot sums cross chunks.  H 2048 and 4096: 256 and 512
    work-groups, the XCD permutation on."""
    L = O.OracleMoe.synthetic(dtype, hidden, inter, 12, 8, normalize_topk=True,
                              seed=hidden + inter)
    moe = make_layer(ctx, L)
    for seed in range(2):
        x = O.normal(8000 + seed, hidden)
        out, idx, w = moe.forward(x, return_routes=True)
        o_out, o_idx, o_w = L.forward(x, nthreads=8)
        assert list(idx) == list(o_idx)
        assert same_bits(w, o_w)
        assert_parity(out, o_out)
    moe.close()


@pytest.mark.parametrize("dtype,hidden,inter,E,k", [
    (H.Q4_0, 2048, 2080, 6, 1),    # 1 slot: 32-row groups; 65 blocks, 9 groups: ring of 16, one partial batch
    (H.Q8_0, 2080, 2080, 6, 1),    # q8_0 ring of 8; 66 groups of 32 over the rows padded to 2112
    (H.Q4_0, 4160, 1056, 6, 2),    # 33 blocks, 5 groups: ring of 8; 260 groups of 16, no permutation
    (H.Q8_0, 4096, 1056, 6, 3),    # 3 slots: 6 waves; 256 groups of 16, permuted
    (H.Q4_0, 2048, 1024, 8, 3),    # 32 blocks: ring of 4 at its limit, 3 x 32 blocks staged
    (H.Q8_0, 2048, 1024, 8, 2),    # q8_0 ring of 4 at its limit
    (H.Q4_0, 2048, 2048, 8, 3),    # 64 blocks: q4_0 ring of 8 at its limit, 3 x 64 blocks staged
    (H.Q4_0, 4096, 2048, 8, 1),    # the same ring with one slot (4 waves)
    (H.Q4_0, 2048, 10912, 4, 3),   # 3 x 341 = 1023 activation blocks: the LDS limit, ring of 16
    (H.Q4_0, 2048, 11264, 4, 3),   # 3 x 352 = 1056 blocks: over the limit, pipelined kernel
])
def test_moe_decode_down_whole_chain(ctx, dtype, hidden, inter, E, k):
    """Top-1 to top-3 down + combine run one wave per (slot, 8 rows) with
    all activation blocks in LDS, folding each row's chain in block order by
    lane shifts: row-group sizes, ring depths, partial last batches, the
    XCD permutation on and off, and the LDS-size switch to the pipelined
    kernel."""
    L = O.OracleMoe.synthetic(dtype, hidden, inter, E, k, normalize_topk=True,
                              seed=hidden + inter + k)
    moe = make_layer(ctx, L)
    for seed in range(2):
        x = O.normal(8100 + seed, hidden)
        out, idx, w = moe.forward(x, return_routes=True)
        o_out, o_idx, o_w = L.forward(x, nthreads=8)
        assert list(idx) == list(o_idx)
        assert same_bits(w, o_w)
        assert_parity(out, o_out)
    moe.close()


@pytest.mark.parametrize("dtype,hidden,inter,E,k", [
    (H.Q4_0, 256, 2080, 300, 16),  # 300 experts (the 1024-expert selection) and 65 x 16 > 256 resident
    (H.Q8_0, 256, 2080, 8, 8),     # 65 tiles x 8 slots = 520 > 512 resident (8 waves): 2 per group, odd
    (H.Q4_0, 2080, 1056, 16, 16),  # 33 x 16 = 528 > 512 (8 waves, two chunks per row): odd
    (H.Q4_0, 1024, 8256, 2, 2),    # 258 x 2 = 516 > 256 resident (16 waves, one chunk)
    (H.Q4_0, 4096, 1056, 16, 8),   # 33 x 8 = 264 tile-slots of two chunks: 16 waves, two tiles, odd
    (H.Q4_0, 4096, 4128, 8, 4),    # 129 x 4 = 516: 16 waves, four tiles, the last group one
])
def test_moe_decode_gate_up_two_tiles_per_group(ctx, dtype, hidden, inter, E, k):
    """Gate/up grids larger than the GPU holds at once give each work-group
    two tiles (the second one's loads issued under the first one's fold),
    and so do q4_0 rows of two chunks with 257 to 2048 tile-slots (sixteen
    waves, two or four tiles): odd tile counts leave the last group one
    tile."""
    L = O.OracleMoe.synthetic(dtype, hidden, inter, E, k, normalize_topk=True,
                              seed=hidden + inter + k + 11)
    moe = make_layer(ctx, L)
    for seed in range(2):
        x = O.normal(8300 + seed, hidden)
        out, idx, w = moe.forward(x, return_routes=True)
        o_out, o_idx, o_w = L.forward(x, nthreads=8)
        assert list(idx) == list(o_idx)
        assert same_bits(w, o_w)
        assert_parity(out, o_out)
    moe.close()


def test_moe_top_k_zero_routes_nowhere(ctx):
    """top_k = 0: top_k returns nothing, so the reference's forward leaves
    the output at zero on the decode and the grouped path alike."""
    L = O.OracleMoe.synthetic(O.Q8_0, 64, 32, 4, 0, normalize_topk=True, seed=2)
    moe = make_layer(ctx, L)
    assert moe.route(O.normal(1, 64)) == []
    for T in (1, 3, 12):
        xs = O.normal(T, T * 64).reshape(T, 64)
        out, idx, w = moe.forward(xs, return_routes=True)
        o_out, _, _ = L.prefill(xs)
        assert idx.shape == (T, 0)
        assert same_bits(out, o_out) and not out.any()
    assert not moe.experts.routing_counts().any()
    moe.close()


def test_moe_forward_device_rejects_misaligned_x(ctx):
    """The router reads device x as float4: a d_x that is not 16-byte
    aligned (or d_logits not float-aligned) fails with ValueError before
    anything is enqueued; aligned buffers at any 16-byte offset work."""
    L = O.OracleMoe.synthetic(O.Q8_0, 64, 32, 4, 2, normalize_topk=True, seed=3)
    moe = make_layer(ctx, L)
    x = O.normal(5, 64)
    bx, bo, bl = ctx.malloc(64 * 4 + 64), ctx.malloc(64 * 4), ctx.malloc(4 * 4 + 8)
    for off in (4, 8, 12):
        with pytest.raises(ValueError, match="16-byte aligned"):
            moe.forward_device(1, bx.address + off, bo.address)
    with pytest.raises(ValueError, match="4-byte aligned"):
        moe.forward_device(1, bx.address, bo.address, d_logits=bl.address + 2)
    bx.upload(np.concatenate([np.zeros(4, np.float32), x]))
    moe.forward_device(1, bx.address + 16, bo.address)
    ctx.synchronize()
    o_out, _, _ = L.forward(x)
    assert same_bits(bo.download(np.float32, 64), o_out)
    for b in (bx, bo, bl):
        b.free()
    moe.close()


def _special_logits(E, case, seed):
    rng = np.random.default_rng(seed)
    lg = rng.normal(0.0, 2.0, E).astype(np.float32)
    ninf, f = np.float32(-np.inf), np.float32
    if case == "neg_inf":      # fewer finite logits than routes: zero probabilities tie, by index
        lg[:] = ninf
        lg[5] = 3.0
        lg[E - 2] = -200.0
    elif case == "below_window":  # probabilities that underflow to zero and tie, by index
        lg[:] = -150.0 - np.arange(E, dtype=np.float32)
        lg[3], lg[E - 1] = 0.0, -70.0
    elif case == "signed_zero":   # +0 and -0 are one logit and one probability
        lg = -np.abs(lg) - 1.0
        lg[E - 1], lg[1] = f(0.0), f(-0.0)
    elif case == "exact_ties":
        lg[[7, 2, 11]] = lg.max() + 1.0
    elif case == "near_ties":     # neighbours one ulp apart at the top
        top = f(lg.max() + 1.0)
        lg[4] = top
        lg[9] = np.nextafter(top, f(-np.inf))
        lg[1] = np.nextafter(lg[9], f(-np.inf))
    elif case == "neg_nan":       # a NaN makes every probability NaN
        lg[6] = np.frombuffer(np.uint32(0xFFC01234).tobytes(), np.float32)[0]
    return lg


@pytest.mark.parametrize("E", [16, 256, 300])
@pytest.mark.parametrize("case", ["neg_inf", "below_window", "signed_zero", "exact_ties",
                                  "near_ties", "neg_nan"])
def test_moe_decode_special_logits(ctx, E, case):
    """Router logits given, one token: the work-groups' own expert choice
    (logit rank, checked for near-ties around it) must equal the reference's
    probability ranking, or fall back to it.  NaN logits make every weight
    and output NaN in the reference; NaN payloads are the platform's, so
    that case compares the routes and the NaN-ness."""
    k = 4
    L = O.OracleMoe.synthetic(O.Q8_0, 64, 32, E, k, normalize_topk=True, seed=E, with_router=False)
    moe = make_layer(ctx, L)
    for seed in range(2):
        lg = _special_logits(E, case, seed)
        x = O.normal(9000 + seed, 64)
        out, idx, w = moe.forward(x, logits=lg, return_routes=True)
        o_out, o_idx, o_w = L.forward(x, logits=lg)
        assert list(idx) == list(o_idx), (case, seed)
        if case == "neg_nan":
            assert np.isnan(w).all() and np.isnan(o_w).all()
            assert np.isnan(out).all() and np.isnan(o_out).all()
        else:
            assert same_bits(w, o_w)
            assert_parity(out, o_out)
    moe.close()
