"""GPU parity of decode_row, WeightMatrix::{row_to_f32, to_f32, convert}
against the CPU oracle, through the C ABI (src/tensor/quant.rs:236-269,
src/tensor/matrix.rs:88-109).

Bar: bit-exact.  F32 / F16 / BF16 decoding is pure bit conversion, so every
value matches bit for bit, NaNs included (half's to_f32 keeps the payload
and sets the quiet bit; the oracle's conversion is pinned to F16C on all
2^16 halves).  Q8_0 / Q4_0 values are one f32 product scale * code: they
match bit for bit except that a NaN matches any NaN, because the NaN an
invalid product returns is the platform's (x86's default NaN is negative,
AArch64's and the GPU's positive), so the reference itself has no single
answer there.  Conversions compare the converted matrix's bytes with the
oracle's encode_row over its decode_row of the source.
"""
import numpy as np
import pytest

import hale_moe as H
import oracle as O

pytestmark = pytest.mark.gpu

DTYPES = [H.F32, H.F16, H.BF16, H.Q8_0, H.Q4_0]
QUANT = (H.Q8_0, H.Q4_0)


def same_values(got, want, dtype):
    got = np.ascontiguousarray(got, np.float32).reshape(-1)
    want = np.ascontiguousarray(want, np.float32).reshape(-1)
    if got.shape != want.shape:
        return False
    same = got.view(np.uint32) == want.view(np.uint32)
    if dtype in QUANT:
        same |= np.isnan(got) & np.isnan(want)
    return bool(same.all())


def random_bytes(seed, n):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)


# ---------------------------------------------------------------------------
# decode_row
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols", [(1, 32), (37, 96), (64, 4096), (3, 14336)])
def test_decode_rows_bit_exact(ctx, dtype, rows, cols):
    """Random bytes (every scale and value pattern, NaN and inf included)."""
    data = random_bytes(rows * cols + dtype, rows * O.row_bytes(dtype, cols))
    got = H.decode_rows(ctx, dtype, data, rows, cols)
    want = O.decode_row(dtype, data, rows * cols)
    assert same_values(got, want, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shift", [1, 2, 3])
def test_decode_rows_device_any_alignment(ctx, dtype, shift):
    """Rows at any byte offset decode as the aligned ones do (the reference's
    unaligned_rows_give_the_same_answer_as_aligned_ones, src/tensor/quant.rs:
    406-420, for every dtype)."""
    rows, cols = 5, 160
    nb = rows * O.row_bytes(dtype, cols)
    data = random_bytes(50 + dtype, nb)
    src, dst = ctx.malloc(nb + 16), ctx.malloc(rows * cols * 4)
    src.upload(np.concatenate([np.zeros(shift, np.uint8), data]))
    ctx.check(H.lib().hale_decode_rows_device(ctx.handle, dtype, rows, cols,
                                              H._vp(src.address + shift), H._vp(dst.address)))
    ctx.synchronize()
    got = dst.download(np.float32, rows * cols)
    assert same_values(got, O.decode_row(dtype, data, rows * cols), dtype)
    assert same_values(got, H.decode_rows(ctx, dtype, data, rows, cols), dtype)
    src.free()
    dst.free()


@pytest.mark.parametrize("dtype", [H.F16, H.BF16])
def test_decode_every_half(ctx, dtype):
    """All 2^16 patterns of a half format, bit for bit (signalling NaNs come
    back quiet for f16; bf16 is a shift, so every payload stays)."""
    data = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.uint8)
    got = H.decode_rows(ctx, dtype, data, 1, 1 << 16).reshape(-1)
    want = O.decode_row(dtype, data, 1 << 16)
    assert same_values(got, want, dtype)
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    if dtype == H.F16:  # the quiet bit on every NaN, payload and sign kept
        nan = ((h & 0x7C00) == 0x7C00) & ((h & 0x3FF) != 0)
        bits = got.view(np.uint32)[nan]
        assert ((bits & 0x7FC00000) == 0x7FC00000).all()
        assert (((bits >> 13) & 0x3FF) == ((h[nan] & 0x3FF) | 0x200)).all()
        assert ((bits >> 31) == (h[nan] >> 15)).all()


@pytest.mark.parametrize("dtype", QUANT)
def test_decode_every_scale(ctx, dtype):
    """Every f16 scale, each block holding every code of its format: the
    product scale * code (q4_0: code - 8) for all of them."""
    bb = O.block_bytes(dtype)
    blocks = np.zeros((1 << 16, bb), np.uint8)
    blocks[:, 0:2] = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.uint8).reshape(-1, 2)
    if dtype == H.Q8_0:
        codes = np.arange(32, dtype=np.int64)
        blocks[:, 2:] = ((codes[None, :] * 8 + np.arange(1 << 16)[:, None]) % 256).astype(np.uint8)
    else:
        lo = np.arange(16, dtype=np.uint8)
        blocks[:, 2:] = lo | (((lo + np.arange(1 << 16)[:, None] % 16) % 16) << 4).astype(np.uint8)
    data = blocks.reshape(-1)
    got = H.decode_rows(ctx, dtype, data, 1 << 10, 64 * 32)
    want = O.decode_row(dtype, data, (1 << 16) * 32)
    assert same_values(got, want, dtype)


def test_decode_rejects_ragged_quantized_rows(ctx):
    """Q8_0 / Q4_0 rows must hold whole blocks (DType::row_bytes)."""
    src, out = np.zeros(64, np.uint8), np.zeros(48, np.float32)
    for dt in QUANT:
        with pytest.raises(ValueError, match="divisible by 32"):
            ctx.check(H.lib().hale_decode_rows(ctx.handle, dt, 1, 48, src.ctypes.data_as(H._vp),
                                               out.ctypes.data_as(H._fp)))


# ---------------------------------------------------------------------------
# WeightMatrix::row_to_f32 / to_f32 from the HBM layout
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES)
def test_matrix_to_f32_and_rows(ctx, dtype):
    """70 rows (a partial last 32-row tile) x 160 columns, uploaded from
    random reference-layout bytes: to_f32, single rows and a row range all
    equal decode_row of the uploaded bytes."""
    rows, cols = 70, 160
    rb = O.row_bytes(dtype, cols)
    data = random_bytes(70 + dtype, rows * rb)
    m = H.WeightMatrix.new(ctx, rows, cols, dtype, data)
    want = O.decode_row(dtype, data, rows * cols).reshape(rows, cols)
    assert same_values(m.to_f32(), want, dtype)
    for r in (0, 31, 32, 69):
        assert same_values(m.row_to_f32(r), want[r], dtype)
    assert same_values(m.rows_to_f32(33, 5), want[33:38], dtype)
    with pytest.raises(ValueError):
        m.rows_to_f32(68, 3)
    buf = ctx.malloc(7 * cols * 4)
    m.rows_to_f32_device(60, 7, buf.address)  # the device form, last tile's rows
    ctx.synchronize()
    assert same_values(buf.download(np.float32, 7 * cols), want[60:67], dtype)
    with pytest.raises(ValueError):
        m.rows_to_f32_device(64, 7, buf.address)
    buf.free()
    m.close()


# ---------------------------------------------------------------------------
# WeightMatrix::convert
# ---------------------------------------------------------------------------

def expected_convert(src_dtype, data, rows, cols, dst_dtype):
    if src_dtype == dst_dtype:
        return data
    vals = O.decode_row(src_dtype, data, rows * cols).reshape(rows, cols)
    return O.encode_matrix(dst_dtype, vals)


@pytest.mark.parametrize("src", DTYPES)
@pytest.mark.parametrize("dst", DTYPES)
def test_convert_equals_decode_then_encode(ctx, src, dst):
    """Every (source, target) pair over finite values with zero, tiny and
    huge blocks: the converted bytes equal encode_row(decode_row(source)),
    the shape stays and the same dtype gives an independent copy."""
    rows, cols = 40, 64
    v = O.normal(src * 5 + dst, rows * cols).reshape(rows, cols)
    v[3, :32] = 0.0
    v[5, 32:] *= 1e-6
    v[7] *= 1e4  # large, still finite in f16
    data = O.encode_matrix(src, v)
    m = H.WeightMatrix.new(ctx, rows, cols, src, data)
    q = m.convert(dst)
    assert (q.rows(), q.cols(), q.dtype()) == (rows, cols, dst)
    want = expected_convert(src, data, rows, cols, dst)
    assert (q.bytes() == want).all()
    m.close()  # the converted matrix owns its memory
    assert (q.bytes() == want).all()
    q.close()


@pytest.mark.parametrize("src", [H.F32, H.F16, H.BF16])
@pytest.mark.parametrize("dst", DTYPES)
def test_convert_from_any_float_bits(ctx, src, dst):
    """Float sources from random bytes (NaNs with payloads, infinities,
    subnormals): their decoding is exact, so the conversion is bit-exact
    everywhere, NaN handling of encode_row included."""
    rows, cols = 16, 96
    data = random_bytes(90 + 5 * src + dst, rows * O.row_bytes(src, cols))
    m = H.WeightMatrix.new(ctx, rows, cols, src, data)
    q = m.convert(dst)
    assert (q.bytes() == expected_convert(src, data, rows, cols, dst)).all()
    q.close()
    m.close()


def test_convert_quantizes_and_keeps_shape(ctx):
    """The reference's convert_quantizes_and_keeps_shape
    (src/tensor/matrix.rs:184-190): a 4 x 64 f32 matrix of sin(i) converts
    to Q8_0 with its shape and under a third of the bytes."""
    w = np.sin(np.arange(4 * 64, dtype=np.float32))
    m = H.WeightMatrix.from_f32(ctx, 4, 64, H.F32, w)
    q = m.convert(H.Q8_0)
    assert (q.rows(), q.cols(), q.dtype()) == (4, 64, H.Q8_0)
    assert q.size_bytes() < m.size_bytes() / 3
    q.close()
    m.close()


def test_convert_rejects_ragged_rows_for_quantized_targets(ctx):
    """from_f32 into Q8_0 / Q4_0 needs rows of whole blocks (row_bytes
    fails on 48 columns); float targets take any length."""
    m = H.WeightMatrix.from_f32(ctx, 4, 48, H.F32, O.normal(1, 4 * 48))
    for dt in QUANT:
        with pytest.raises(ValueError, match="multiple of 32"):
            m.convert(dt)
    q = m.convert(H.BF16)
    assert (q.bytes() == O.encode_matrix(H.BF16, O.normal(1, 4 * 48).reshape(4, 48))).all()
    q.close()
    m.close()


def test_convert_in_several_passes(ctx):
    """A 4100 x 4096 q4_0 matrix (the f32 rows of one pass fill 64 MiB at
    4096 rows, so this takes two passes, the second of 4 rows) to q8_0."""
    rows, cols = 4100, 4096
    v = O.normal(77, rows * cols).reshape(rows, cols)
    data = O.encode_matrix(H.Q4_0, v)
    m = H.WeightMatrix.new(ctx, rows, cols, H.Q4_0, data)
    q = m.convert(H.Q8_0)
    assert (q.bytes() == expected_convert(H.Q4_0, data, rows, cols, H.Q8_0)).all()
    q.close()
    m.close()
