"""GPU parity of the float-weight matvec (f32 / f16 / bf16) and of the
half-format encoder, against the oracle, through the C ABI.

Bar: bit-exact.  The reference's float dot (src/tensor/quant.rs:146-233)
sums eight lane accumulators, reduces them in a fixed tree and adds the
tail of cols % 8 products; every output here equals the oracle's bits,
including rows whose byte length is not a multiple of 16 (the kernel then
reads value by value) and rows shorter than one octet.  The accumulation-order
tolerance (rel-L2 <= 1e-5) is asserted as well.
"""
import numpy as np
import pytest

import hale_moe as H
import oracle as O

pytestmark = pytest.mark.gpu

REL_L2 = 1e-5
FLOATS = [O.F32, O.F16, O.BF16]


def same_bits(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and bool((a.view(np.uint32) == b.view(np.uint32)).all())


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def check_matvec(ctx, dtype, rows, cols, seed, std=0.02):
    v = O.normal(seed, rows * cols, 0.0, std).reshape(rows, cols)
    data = O.encode_matrix(dtype, v)
    x = O.normal(seed + 1, cols)
    m = H.WeightMatrix.new(ctx, rows, cols, dtype, data)
    got = m.matvec(x)
    want = O.matvec(dtype, rows, cols, data, x, nthreads=O.max_threads())
    assert rel_l2(got, want) <= REL_L2
    assert same_bits(got, want), (dtype, rows, cols)
    return m


@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("rows,cols", [(2048, 2048), (1000, 4096), (9, 1024), (37, 1000),
                                       (100, 13), (61, 2047), (8, 8), (5, 3), (257, 3000)])
def test_float_matvec_bit_exact(ctx, dtype, rows, cols):
    check_matvec(ctx, dtype, rows, cols, seed=rows * 7 + cols)


@pytest.mark.parametrize("dtype", FLOATS)
def test_float_matvec_lm_head_shape(ctx, dtype):
    # a vocabulary-sized output (Qwen3's 151936 rows) over hidden 2048
    check_matvec(ctx, dtype, 151936, 2048, seed=77)


@pytest.mark.parametrize("dtype", [O.F16, O.BF16])
def test_float_matvec_lanes_kept_across_decode_chunks(ctx, dtype):
    """dot_decoded's 64-value chunks share the eight lane accumulators
    (src/tensor/quant.rs:166-184): the closed-form row of
    tests/test_oracle.py gives 2^24 + 4, where a reduce per chunk gives
    2^24 + 6.  Rows 1 and 2 shift the same products by one octet and hold
    zeros, to land the terms in other lanes and a zero row."""
    from test_oracle import decoded_chunk_case

    w, x, kept, reset = decoded_chunk_case()
    rows = np.stack([w, np.roll(w, 8), np.zeros_like(w)])
    xs = np.roll(x, 0)
    data = O.encode_matrix(dtype, rows)
    m = H.WeightMatrix.new(ctx, 3, w.size, dtype, data)
    got = m.matvec(xs)
    want = O.matvec(dtype, 3, w.size, data, xs)
    assert got[0] == kept and got[0] != reset
    assert same_bits(got, want)
    m.close()


def test_float_matvec_lane_order_closed_form(ctx):
    # w = [1, 1, 0, 0, 2^24, 0, 0, 0], x = 1: lanes give (1 + 2^24) + 1 -> 2^24
    # with two round-to-even steps; a left-to-right sum would give 2^24 + 2.
    # With a 4-element tail [1, 1, 0, 0] the tail sum 2 is added last.
    w = np.array([[1, 1, 0, 0, 2 ** 24, 0, 0, 0, 0, 0, 0, 0],
                  [1, 1, 0, 0, 2 ** 24, 0, 0, 0, 1, 1, 0, 0]], dtype=np.float32)
    m = H.WeightMatrix.new(ctx, 2, 12, "f32", w.view(np.uint8))
    got = m.matvec(np.ones(12, np.float32))
    assert got[0] == 16777216.0 and got[1] == 16777218.0


@pytest.mark.parametrize("dtype", FLOATS)
def test_float_matvec_special_values(ctx, dtype):
    rows, cols = 16, 96
    v = O.normal(5, rows * cols).reshape(rows, cols)
    v[0] = 0.0
    v[1] = -0.0                         # all products -0: the sum is +0
    v[2, :8] = 1e-40                    # f32 subnormals (zero in f16 / bf16)
    v[3, 5] = np.inf                    # inf row
    v[4, 7] = np.nan
    v[5, :] = 3.0e38                    # overflow to inf in the lanes
    data = O.encode_matrix(dtype, v)
    x = O.normal(6, cols)
    x[5] = 0.0                          # row 3: inf * 0 = nan in lane 5
    x[6] = -x[6]
    got = H.WeightMatrix.new(ctx, rows, cols, dtype, data).matvec(x)
    want = O.matvec(dtype, rows, cols, data, x)
    assert same_bits(got, want)


@pytest.mark.parametrize("dtype", [O.F16, O.BF16])
def test_half_encode_bit_exact(ctx, dtype):
    n = 1 << 16
    v = O.normal(9, n, 0.0, 3.0)
    # halfway cases, subnormals, overflow, signed zeros, infinities, NaN payloads
    bits = np.array([0x3f808000, 0x3f818000, 0x3f800fff, 0x3f801000, 0x3f803000, 0x33000001,
                     0x387fc000, 0x477ff000, 0x477fefff, 0x7f7fffff, 0x80000000, 0x00000001,
                     0x7f800000, 0xff800000, 0x7fc00001, 0xffa12345, 0x7f800001, 0x00800000],
                    dtype=np.uint32)
    v[:bits.size] = bits.view(np.float32)
    v = v.reshape(256, 256)
    got = H.encode_rows(ctx, dtype, v)
    want = O.encode_matrix(dtype, v)
    assert (got == want).all()


@pytest.mark.parametrize("dtype", FLOATS)
def test_from_f32_and_bytes_round_trip(ctx, dtype):
    rows, cols = 33, 77
    v = O.normal(12, rows * cols).reshape(rows, cols)
    m = H.WeightMatrix.from_f32(ctx, rows, cols, dtype, v)
    assert (m.bytes() == O.encode_matrix(dtype, v)).all()
    with pytest.raises(ValueError):
        m.matvec(np.zeros(cols + 1, np.float32))
