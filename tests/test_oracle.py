"""Pins of the CPU oracle (oracle/hale_oracle.c) against things other than
itself: the reference's own unit tests and known answers, closed forms,
library routines (numpy's IEEE half conversion) and brute force.

Each test names the oracle function it pins and the mistake it would catch.
No GPU is needed.
"""
import math
import os
import subprocess

import numpy as np
import pytest

import oracle as O

F2 = np.float32


def f16_bits(v: float) -> int:
    """IEEE binary16 bits of v by numpy (round to nearest even)."""
    return int(np.array([v], dtype=np.float32).astype(np.float16).view(np.uint16)[0])


def q8_block(scale_bits: int, codes) -> np.ndarray:
    b = np.zeros(34, dtype=np.uint8)
    b[0], b[1] = scale_bits & 0xFF, scale_bits >> 8
    b[2:] = np.asarray(codes, dtype=np.int8).view(np.uint8)
    return b


# ---------------------------------------------------------------------------
# geometry: DType::row_bytes (src/tensor/dtype.rs:53-61)
# ---------------------------------------------------------------------------

def test_row_bytes_known_answers():
    # src/tensor/dtype.rs:120-127
    assert O.row_bytes(O.F32, 64) == 256
    assert O.row_bytes(O.BF16, 64) == 128
    assert O.row_bytes(O.Q8_0, 64) == 68
    assert O.row_bytes(O.Q4_0, 64) == 36
    assert O.row_bytes(O.Q4_0, 33) == -1
    # bits_per_weight 4.5 for q4_0 (dtype.rs:140)
    assert O.block_bytes(O.Q4_0) * 8 / 32 == 4.5


# ---------------------------------------------------------------------------
# f16 conversion (half 2.7.1, used at src/tensor/quant.rs:44-46,299,316)
# ---------------------------------------------------------------------------

def test_f16_conversions_match_f16c_on_every_value(tmp_path):
    """f32 -> f16 exhaustive over all 2^32 bit patterns against the F16C
    instruction (NaN payloads excluded): catches truncation instead of RNE,
    a missing subnormal path or a wrong overflow threshold.  f16 -> f32 over
    all 2^16 halves, bit for bit with NaNs (half's to_f32 on x86 is that
    instruction): catches a signalling NaN left unquieted or a lost
    payload, sign or subnormal."""
    here = os.path.dirname(os.path.abspath(__file__))
    exe = tmp_path / "f16c_check"
    odir = os.path.dirname(O.__file__)
    subprocess.run(["gcc", "-O2", "-mf16c", "-mavx", os.path.join(here, "native", "f16c_check.c"),
                    "-o", str(exe), f"-L{odir}", "-lhale_oracle", f"-Wl,-rpath,{odir}", "-lm"],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    assert [int(v) for v in out.split()] == [0, 0]


def test_f32_to_f16_matches_numpy_on_a_sample():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    bits[:65536] = (np.arange(65536, dtype=np.uint32) << 13) + 0x1000  # ties
    vals = bits.view(np.float32)
    ours = np.array([O.f32_to_f16(float(v)) for v in vals[:4096]], dtype=np.uint16)
    with np.errstate(over="ignore"):
        ref = vals[:4096].astype(np.float16).view(np.uint16)
    ok = (ours == ref) | np.isnan(vals[:4096])
    assert ok.all()


def test_f16_to_f32_is_exact_for_all_halves():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    ours = np.array([O.f16_to_f32(int(v)) for v in h], dtype=np.float32)
    same = (ours.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(ours) & np.isnan(ref))
    assert same.all()


# ---------------------------------------------------------------------------
# encode / decode (src/tensor/quant.rs:236-321)
# ---------------------------------------------------------------------------

def test_q8_encode_known_answer_rounds_half_away_from_zero():
    """amax = 127 makes scale = inv = 1, so codes = round(v): 2.5 -> 3 and
    -2.5 -> -3 (banker's rounding would give 2 / -2)."""
    v = np.zeros(32, dtype=np.float32)
    v[:8] = [127, -126.5, 2.5, -2.5, 0.5, -0.5, 0.49999997, 1.5]
    b = O.encode_row(O.Q8_0, v)
    assert b.size == 34
    assert (int(b[0]) | (int(b[1]) << 8)) == 0x3C00  # f16(1.0)
    codes = b[2:].view(np.int8)
    assert list(codes[:8]) == [127, -127, 3, -3, 1, -1, 0, 2]
    assert (codes[8:] == 0).all()


def test_q8_encode_scale_is_f16_of_unrounded_f32_scale():
    v = O.test_values(32, 5)
    b = O.encode_row(O.Q8_0, v)
    amax = np.max(np.abs(v))
    s = F2(amax) / F2(127.0)
    assert (int(b[0]) | (int(b[1]) << 8)) == f16_bits(float(s))


def test_q4_encode_known_answers():
    """extreme = -8 gives scale 1: q = trunc(v + 8.5) clamped to 0..15;
    element j sits in the low nibble of byte j, element j+16 in the high."""
    v = np.zeros(32, dtype=np.float32)
    v[0] = -8.0
    v[1:8] = [7.0, -0.5, -0.6, 3.4, 3.5, 7.6, -7.9]
    v[16:20] = [1.0, 2.0, -1.0, 7.4]
    b = O.encode_row(O.Q4_0, v)
    assert b.size == 18
    assert (int(b[0]) | (int(b[1]) << 8)) == 0x3C00
    lo = [int(x) & 0xF for x in b[2:]]
    hi = [int(x) >> 4 for x in b[2:]]
    # v+8.5 truncated: -8->0, 7->15, -0.5->8, -0.6->7, 3.4->11, 3.5->12, 7.6->15(clamp), -7.9->0
    assert lo[:8] == [0, 15, 8, 7, 11, 12, 15, 0]
    assert hi[:4] == [9, 10, 7, 15]
    assert lo[8:] == [8] * 8 and hi[4:] == [8] * 12


def test_q4_encode_positive_extreme_gives_negative_scale_and_first_tie_wins():
    v = np.zeros(32, dtype=np.float32)
    v[0], v[1] = 8.0, -8.0   # |8| == |-8|: the first one is the extreme
    b = O.encode_row(O.Q4_0, v)
    assert (int(b[0]) | (int(b[1]) << 8)) == 0xBC00  # f16(-1.0)
    # inv = -1: 8 -> trunc(-8 + 8.5) = 0; -8 -> trunc(8 + 8.5) = 16 -> 15
    assert int(b[2]) & 0xF == 0 and int(b[3]) & 0xF == 15
    v[0], v[1] = -8.0, 8.0
    b = O.encode_row(O.Q4_0, v)
    assert (int(b[0]) | (int(b[1]) << 8)) == 0x3C00


def test_every_dtype_round_trips_within_its_precision():
    # src/tensor/quant.rs:344-366 (values(96, 7), the reference's tolerances)
    v = O.test_values(96, 7)
    for dtype, tol in [(O.F32, 0.0), (O.F16, 1e-3), (O.BF16, 1e-2), (O.Q8_0, 1e-2), (O.Q4_0, 0.15)]:
        b = O.encode_row(dtype, v)
        assert b.size == O.row_bytes(dtype, v.size)
        back = O.decode_row(dtype, b, v.size)
        assert np.max(np.abs(v - back)) <= tol, dtype


def test_zero_block_quantizes_to_zero():
    # src/tensor/quant.rs:422-432.  q8_0 stores f16(0/127) = +0; q4_0 stores
    # f16(0 / -8) = -0 (0x8000); both decode to zeros.
    z = np.zeros(32, dtype=np.float32)
    for dtype, bits in ((O.Q8_0, 0x0000), (O.Q4_0, 0x8000)):
        b = O.encode_row(dtype, z)
        assert (int(b[0]) | (int(b[1]) << 8)) == bits
        assert (b[2:] == (0 if dtype == O.Q8_0 else 0x88)).all()
        assert (O.decode_row(dtype, b, 32) == 0).all()


def test_decode_q4_nibble_order():
    b = np.zeros(18, dtype=np.uint8)
    b[0], b[1] = 0x00, 0x3C
    b[2] = 0x9F   # element 0 = 15-8 = 7, element 16 = 9-8 = 1
    b[17] = 0x30  # element 15 = 0-8 = -8, element 31 = 3-8 = -5
    d = O.decode_row(O.Q4_0, b, 32)
    assert d[0] == 7 and d[16] == 1 and d[15] == -8 and d[31] == -5


# ---------------------------------------------------------------------------
# activation quantization: Q8Activations::quantize (quant.rs:77-93)
# ---------------------------------------------------------------------------

def test_activation_scale_stays_f32_and_codes_round_half_away():
    x = np.zeros(64, dtype=np.float32)
    x[0:4] = [1.0, -0.25, 0.5, 0.0]              # amax 1 -> scale 1/127 (f32)
    x[32:36] = [127.0, 2.5, -2.5, -126.5]        # amax 127 -> scale 1
    s, q = O.q8_quantize(x)
    assert s[0] == F2(1.0) / F2(127.0)            # not rounded to f16
    assert f16_bits(float(s[0])) != int(np.float32(s[0]).view(np.uint32) >> 16)
    assert s[1] == 1.0
    assert list(q[32:36]) == [127, 3, -3, -127]
    assert q[0] == 127 and q[3] == 0
    with pytest.raises(ValueError):
        O.q8_quantize(np.zeros(33, dtype=np.float32))


# ---------------------------------------------------------------------------
# block dot products: dot_q8_0 / dot_q4_0 (quant.rs:115-144)
# ---------------------------------------------------------------------------

def test_block_sums_equal_brute_force_int64():
    """isum_b from the decoded codes in int64 (scale 1 blocks make decode
    return the codes themselves); catches a wrong nibble pairing."""
    rng = np.random.default_rng(3)
    for dtype in (O.Q8_0, O.Q4_0):
        nb = 5
        row = np.zeros(nb * O.block_bytes(dtype), dtype=np.uint8)
        for b in range(nb):
            blk = row[b * O.block_bytes(dtype):(b + 1) * O.block_bytes(dtype)]
            blk[0], blk[1] = 0x00, 0x3C
            blk[2:] = rng.integers(0, 256, blk.size - 2, dtype=np.uint8)
        x = rng.normal(size=nb * 32).astype(np.float32)
        xs, xq = O.q8_quantize(x)
        _, isums = O.dot_quantized(dtype, row, xs, xq)
        codes = O.decode_row(dtype, row, nb * 32).astype(np.int64)
        brute = (codes.reshape(nb, 32) * xq.astype(np.int64).reshape(nb, 32)).sum(axis=1)
        assert (isums == brute).all()


def test_block_terms_are_summed_left_to_right():
    """Terms t = [1, 2^24, 1, -2^24]: left to right gives 0 (1 is absorbed
    twice by round-to-even), a pairwise sum gives 1, right-to-left gives 2."""
    x = np.zeros(4 * 32, dtype=np.float32)
    for b in range(4):
        x[b * 32:b * 32 + 3] = [127.0, 127.0, 1.0]   # scale 1, codes [127,127,1,0..]
    xs, xq = O.q8_quantize(x)
    assert (xs == 1.0).all()
    # isum = 127*(a0+a1) + a2; (dw, codes) per wanted term
    blocks = [
        q8_block(0x3C00, [0, 0, 1] + [0] * 29),           # 1 * 1
        q8_block(0x6400, [127, 2, 1] + [0] * 29),         # 1024 * 16384 = 2^24
        q8_block(0x3C00, [0, 0, 1] + [0] * 29),           # 1
        q8_block(0xE400, [127, 2, 1] + [0] * 29),         # -1024 * 16384
    ]
    row = np.concatenate(blocks)
    total, isums = O.dot_quantized(O.Q8_0, row, xs, xq)
    assert list(isums) == [1, 16384, 1, 16384]
    assert total == 0.0


def test_block_term_is_scale_product_times_isum():
    """(d_w * d_x) * isum, not d_w * (d_x * isum): search a case where the two
    differ in f32 and check the oracle follows the reference's grouping."""
    rng = np.random.default_rng(11)
    for _ in range(2000):
        dw_bits = int(rng.integers(0x2000, 0x3C00))
        dw = np.float32(np.uint16(dw_bits).view(np.float16))
        x = rng.normal(size=32).astype(np.float32)
        xs, xq = O.q8_quantize(x)
        codes = rng.integers(-127, 128, 32)
        isum = int((codes * xq.astype(np.int64)).sum())
        a = (dw * xs[0]) * F2(isum)
        b = dw * (xs[0] * F2(isum))
        if a != b:
            total, _ = O.dot_quantized(O.Q8_0, q8_block(dw_bits, codes), xs, xq)
            assert total == F2(0.0) + a
            return
    pytest.fail("no distinguishing case found")


def test_dot_equals_dot_of_decoded_row():
    # src/tensor/quant.rs:368-398
    w, x = O.test_values(64, 3), O.test_values(64, 11)
    for dtype in (O.F32, O.F16, O.BF16, O.Q8_0, O.Q4_0):
        b = O.encode_row(dtype, w)
        dec = O.decode_row(dtype, b, 64)
        expect = float(np.dot(dec.astype(np.float64), x.astype(np.float64)))
        got = O.dot(dtype, b, x)
        tol = 2e-2 * max(abs(expect), 1.0) if dtype in (O.Q8_0, O.Q4_0) else 1e-4
        assert abs(expect - got) < tol, dtype
    w13, x13 = O.test_values(13, 5), O.test_values(13, 9)
    assert abs(O.dot(O.F32, O.encode_row(O.F32, w13), x13) - float(np.dot(w13, x13))) < 1e-5


def test_dot_f32_uses_eight_lane_order():
    """w = [1,1,0,0,2^24,0,0,0], x = 1: lanes give (1 + 2^24) + 1 -> 2^24
    after two round-to-even steps; a left-to-right sum gives 2^24 + 2."""
    w = np.array([1, 1, 0, 0, 2 ** 24, 0, 0, 0], dtype=np.float32)
    assert O.dot_f32(w, np.ones(8, dtype=np.float32)) == 16777216.0
    # a 4-element tail is summed after the lanes: (2^24) + (1 + 1) = 2^24 + 2
    w2 = np.concatenate([w, np.array([1, 1, 0, 0], dtype=np.float32)])
    assert O.dot_f32(w2, np.ones(12, dtype=np.float32)) == 16777218.0


def decoded_chunk_case():
    """A 132-element f16 / bf16 row for dot_decoded (src/tensor/quant.rs:166-184),
    which decodes 64 values at a time but keeps its eight lane accumulators
    across the chunks and adds the chunks' tails last.  Products: element 0
    (chunk 0, lane 0) 256 * 65536 = 2^24; elements 64 and 65 (chunk 1, lanes
    0 and 1) 1 each; element 128 (the last chunk, a 4-element tail) 1 * 4.
    Lanes kept: lane 0 = 2^24 + 1 -> 2^24 (ties to even), lane 1 = 1, the
    reduce (2^24 + 1) -> 2^24, then + 4: 2^24 + 4.  Lanes reset per chunk
    (a reduce per chunk, summed): 2^24 + 2 + 4.  One sum over the products
    in order: 2^24 + 1 -> 2^24, + 1 -> 2^24, + 4."""
    n = 132
    w = np.zeros(n, np.float32)
    x = np.zeros(n, np.float32)
    w[0], x[0] = 256.0, 65536.0
    w[64] = w[65] = x[64] = x[65] = 1.0
    w[128], x[128] = 1.0, 4.0
    return w, x, 16777220.0, 16777222.0


def test_dot_decoded_keeps_lanes_across_chunks():
    w, x, kept, reset = decoded_chunk_case()
    for dtype in (O.F16, O.BF16):
        b = O.encode_row(dtype, w)
        assert (O.decode_row(dtype, b, w.size) == w).all()  # every value exact in both formats
        got = O.dot(dtype, b, x)
        assert got == kept and got != reset, dtype
    # the whole-row f32 dot adds the same lanes in the same order
    assert O.dot_f32(w, x) == kept


# ---------------------------------------------------------------------------
# matvec (src/tensor/matrix.rs:115-143, tests :150-189)
# ---------------------------------------------------------------------------

def test_matvec_parallel_equals_serial_and_naive():
    rows, cols = 70, 64
    i = np.arange(rows * cols)
    w = (((i * 37) % 101).astype(np.float32) - 50.0) / 50.0
    x = (np.arange(cols, dtype=np.float32) / cols) - 0.5
    expect = w.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
    data = w.astype(np.float32).view(np.uint8)
    par = O.matvec(O.F32, rows, cols, data, x, nthreads=4)
    ser = O.matvec(O.F32, rows, cols, data, x, nthreads=1)
    assert (par.view(np.uint32) == ser.view(np.uint32)).all()
    assert np.max(np.abs(par - expect)) < 1e-4
    for dtype in (O.Q8_0, O.Q4_0):
        wq = O.encode_matrix(dtype, np.sin(np.arange(96 * 128, dtype=np.float32)).reshape(96, 128))
        xr = O.test_values(128, 2)
        a = O.matvec(dtype, 96, 128, wq, xr, nthreads=4)
        b = O.matvec(dtype, 96, 128, wq, xr, nthreads=1)
        assert (a.view(np.uint32) == b.view(np.uint32)).all()


def test_convert_quantizes_and_keeps_shape():
    # src/tensor/matrix.rs:182-189: q8 size < f32 size / 3
    assert O.row_bytes(O.Q8_0, 64) * 4 < O.row_bytes(O.F32, 64) * 4 / 3


def test_matvec_rejects_bad_shapes():
    with pytest.raises(ValueError):
        O.matvec(O.Q4_0, 2, 33, np.zeros(100, np.uint8), np.zeros(33, np.float32))


# ---------------------------------------------------------------------------
# ops (src/ops/activation.rs, src/ops/topk.rs)
# ---------------------------------------------------------------------------

def test_softmax_reference_cases_and_closed_forms():
    # activation.rs:38-44
    p = O.softmax([1000.0, 1001.0, 1002.0])
    assert abs(float(p.sum()) - 1.0) < 1e-6 and p[2] > p[1] > p[0]
    # equal logits: exp(0) = 1 each, 1/4 exactly
    assert (O.softmax([3.0, 3.0, 3.0, 3.0]) == 0.25).all()
    # [0, ln2] up to rounding of ln2 in f32: ratio 2
    q = O.softmax([0.0, math.log(2.0)])
    assert abs(q[1] / q[0] - 2.0) < 1e-6


def _e(v) -> np.float32:
    return np.float32(O.expf(float(v)))


def _f32_exp(v) -> np.float32:
    """exp rounded once to f32 (the correctly rounded value, independent of
    the oracle)."""
    return np.float32(math.exp(float(np.float32(v))))


def test_softmax_sums_in_index_order():
    # activation.rs:14-17: `sum += *v` over the slice in index order.  With
    # exp values 1, e, e, e and e just above 2^-24, each in-order addition
    # rounds up by one ulp of 1 (sum 1 + 3 * 2^-23); a pairwise sum
    # (1 + e) + (e + e) gives 1 + 2 * 2^-23 and a reversed sum
    # ((e + e) + e) + 1 also 1 + 2 * 2^-23.
    f = np.float32
    l = f(-16.63553)
    e = _f32_exp(l)
    assert f(2.0 ** -24) < e < f(2.0 ** -24 * 1.01)
    assert f(O.expf(float(l))) == e and O.expf(0.0) == 1.0
    es = [f(1.0), e, e, e]
    in_order = f(0.0)
    for v in es:
        in_order = f(in_order + v)
    assert in_order == f(1.0 + 3 * 2.0 ** -23)
    pairwise = f(f(es[0] + es[1]) + f(es[2] + es[3]))
    reverse = f(f(f(es[3] + es[2]) + es[1]) + es[0])
    assert pairwise == reverse == f(1.0 + 2 * 2.0 ** -23)
    p = O.softmax([0.0, float(l), float(l), float(l)])
    assert p[0] == f(1.0) / in_order and p[1] == e / in_order
    assert p[0] != f(1.0) / pairwise
    # the max is subtracted before exp: logits 100, 100 + l, ... give
    # exp(0) = 1 for the first, exp((100 + l) - 100) for the others, summed
    # in the same order
    m = f(100.0)
    d = _e(f(f(m + l) - m))
    s3 = f(f(f(f(1.0) + d) + d) + d)
    q = O.softmax([float(m)] + [float(f(m + l))] * 3)
    assert q[0] == f(1.0) / s3 and q[1] == d / s3


def test_softmax_divides_each_value_by_the_sum():
    # activation.rs:18-20: `*v /= sum`, one correctly rounded division per
    # value, not a multiplication by 1 / sum.  Exp values 1 and exp(-l) for
    # a few logits: the ones where v / sum and v * (1 / sum) differ must give
    # the division.
    f = np.float32
    differ = 0
    for l in np.linspace(-3.0, -0.1, 60, dtype=np.float32):
        e = _f32_exp(l)
        assert f(O.expf(float(l))) == e
        s = f(f(1.0) + e)
        p = O.softmax([0.0, float(l)])
        assert p[0] == f(1.0) / s and p[1] == e / s
        if p[1] != e * (f(1.0) / s) or p[0] != f(1.0) * (f(1.0) / s):
            differ += 1
    assert differ >= 5  # the two forms really are told apart


def test_silu_divides_by_one_plus_exp():
    # activation.rs:5-7: x / (1 + exp(-x)).  The plausible alternatives,
    # x * (1 / (1 + exp(-x))) (x * sigmoid) and x * sigmoid computed from
    # exp(x) / (1 + exp(x)), round differently for some x; the oracle must
    # give the division form for every x.  exp is the oracle's, which
    # tests/test_expf.py holds equal to glibc expf on every f32 input.
    f = np.float32
    differ_recip = differ_sig = 0
    for x in np.linspace(-12.0, 12.0, 481, dtype=np.float32):
        en = f(O.expf(float(-x)))
        assert abs(float(en) / math.exp(-float(x)) - 1.0) < 2e-7
        div = f(x / f(f(1.0) + en))
        assert f(O.silu(float(x))) == div, x
        recip = f(x * f(f(1.0) / f(f(1.0) + en)))
        ep = f(O.expf(float(x)))
        sig = f(x * f(ep / f(f(1.0) + ep)))
        differ_recip += recip != div
        differ_sig += sig != div
    assert differ_recip >= 20 and differ_sig >= 20


def test_expf_is_glibc():
    for v in (-103.0, -20.5, -1.0, 0.0, 1e-7, 0.5, 1.0, 10.0, 88.5, 89.0):
        assert O.expf(v) == float(np.float32(math.exp(np.float32(v)))) or \
            abs(O.expf(v) / math.exp(np.float32(v)) - 1) < 1.2e-7


def test_silu_and_argmax_basics():
    # activation.rs:46-51
    assert O.silu(0.0) == 0.0
    assert abs(O.silu(10.0) - 10.0) < 1e-3
    assert O.argmax([1.0, 3.0, 3.0, -1.0]) == 1
    for v in np.linspace(-30, 30, 601, dtype=np.float32):
        exact = float(v) / (1.0 + math.exp(-float(v)))
        assert abs(O.silu(float(v)) - exact) <= 4e-7 * max(abs(exact), 1e-30) + 1e-38


def test_top_k_matches_full_sort():
    # topk.rs:67-76
    scores = np.array([((i * 73) % 128) * 0.37 - 20.0 for i in range(128)], dtype=np.float32)
    order = sorted(range(128), key=lambda i: (-scores[i], i))
    idx, sc = O.top_k(scores, 8)
    assert list(idx) == order[:8]
    assert list(sc) == [scores[i] for i in order[:8]]


def test_top_k_ties_prefer_lower_index_and_k_is_clamped():
    # topk.rs:78-87
    idx, _ = O.top_k([1.0, 5.0, 5.0, 5.0], 2)
    assert list(idx) == [1, 2]
    assert len(O.top_k([1.0, 2.0], 10)[0]) == 2
    assert len(O.top_k([1.0], 0)[0]) == 0
    # total_cmp: +0.0 ranks above -0.0
    assert list(O.top_k([-0.0, 0.0], 1)[0]) == [1]


def test_top_k_equals_stable_sort_on_random_ties():
    rng = np.random.default_rng(5)
    for _ in range(50):
        s = rng.integers(0, 6, 40).astype(np.float32)
        k = int(rng.integers(1, 40))
        order = sorted(range(40), key=lambda i: (-s[i], i))
        assert list(O.top_k(s, k)[0]) == order[:k]


# ---------------------------------------------------------------------------
# route / expert / MoE layer
# ---------------------------------------------------------------------------

def _tiny_layer(dtype, normalize=True, E=8, H=64, I=32, k=3, seed=7):
    return O.OracleMoe.synthetic(dtype, H, I, E, k, normalize_topk=normalize, seed=seed)


def test_route_closed_form_for_equal_logits():
    L = _tiny_layer(O.Q8_0, normalize=True, E=4, k=2)
    idx, w = L.route(np.zeros(64, np.float32), logits=np.zeros(4, np.float32))
    assert list(idx) == [0, 1] and list(w) == [0.5, 0.5]
    L2 = _tiny_layer(O.Q8_0, normalize=False, E=4, k=2)
    idx, w = L2.route(np.zeros(64, np.float32), logits=np.zeros(4, np.float32))
    assert list(w) == [0.25, 0.25]


def test_route_uses_router_matvec_softmax_topk_renorm():
    L = _tiny_layer(O.Q4_0)
    x = O.normal(99, 64)
    logits = np.array([O.dot_f32(L.router[e], x) for e in range(8)], dtype=np.float32)
    p = O.softmax(logits)
    order = sorted(range(8), key=lambda i: (-p[i], i))[:3]
    idx, w = L.route(x)
    assert list(idx) == order
    norm = F2(-0.0)
    for i in order:
        norm = F2(norm + p[i])
    assert list(w) == [F2(p[i] / norm) for i in order]


def test_expert_forward_close_to_float64_model():
    """Only the q8 activation rounding separates the oracle from an f64 SwiGLU
    on the dequantized weights."""
    H, I = 256, 64
    for dtype in (O.Q8_0, O.Q4_0):
        L = O.OracleMoe.synthetic(dtype, H, I, 1, 1, seed=3, with_router=False)
        x = O.normal(5, H)
        got = O.expert_forward(dtype, H, I, L.gate[0], L.up[0], L.down[0], x)
        dq = lambda data, r, c: np.stack([O.decode_row(dtype, data[i * O.row_bytes(dtype, c):(i + 1) * O.row_bytes(dtype, c)], c) for i in range(r)]).astype(np.float64)
        G, U, D = dq(L.gate[0], I, H), dq(L.up[0], I, H), dq(L.down[0], H, I)
        g, u = G @ x, U @ x
        h = g / (1 + np.exp(-g)) * u
        ref = D @ h
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert rel < 0.02, (dtype, rel)


def test_moe_forward_is_weighted_sum_of_experts_in_route_order():
    L = _tiny_layer(O.Q8_0, E=8, k=3)
    x = O.normal(17, 64)
    out, idx, w = L.forward(x)
    acc = np.zeros(64, dtype=np.float32)
    for e, wt in zip(idx, w):
        y = O.expert_forward(O.Q8_0, 64, 32, L.gate[e], L.up[e], L.down[e], x)
        acc = (acc + F2(wt) * y).astype(np.float32)
    assert (out.view(np.uint32) == acc.view(np.uint32)).all()


def test_prefill_equals_token_by_token_forward():
    # tests/litmus.rs:47-59: prefill == per-token forward, bit for bit
    L = _tiny_layer(O.Q4_0, E=8, k=2)
    xs = O.normal(23, 5 * 64).reshape(5, 64)
    out, idx, w = L.prefill(xs, nthreads=3)
    for t in range(5):
        o1, i1, w1 = L.forward(xs[t])
        assert (o1.view(np.uint32) == out[t].view(np.uint32)).all()
        assert list(i1) == list(idx[t]) and list(w1) == list(w[t])


def test_threads_do_not_change_bits():
    L = O.OracleMoe.synthetic(O.Q4_0, 256, 64, 16, 4, seed=9)
    x = O.normal(2, 256)
    a = L.forward(x, nthreads=1)[0]
    b = L.forward(x, nthreads=6)[0]
    c = L.forward(x, nthreads=6, variant="_v3")[0]
    assert (a.view(np.uint32) == b.view(np.uint32)).all()
    assert (a.view(np.uint32) == c.view(np.uint32)).all()


# ---------------------------------------------------------------------------
# seeded generators
# ---------------------------------------------------------------------------

def test_xorshift64star_matches_its_definition():
    # src/generate/sampler.rs:135-140 restated with Python integers
    s = 42
    want = []
    for _ in range(5):
        s ^= s >> 12
        s ^= (s << 25) & (2 ** 64 - 1)
        s ^= s >> 27
        want.append((s * 0x2545F4914F6CDD1D) & (2 ** 64 - 1))
    assert O.xorshift64star(42, 5) == want
    assert O.xorshift64star(0, 1) == O.xorshift64star(1, 1)  # seed.max(1)


def test_values_helper_matches_reference_definition():
    # src/tensor/quant.rs:328-338
    seed = 7
    s = (seed * 2654435761) & 0xFFFFFFFF
    s = max(s, 1)
    want = []
    for _ in range(6):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        want.append(F2(F2(s) / F2(4294967295.0)) * F2(2.0) - F2(1.0))
    assert list(O.test_values(6, 7)) == want


def test_normals_have_the_requested_moments():
    v = O.normal(1, 200000, 0.0, 0.02)
    assert abs(float(v.mean())) < 2e-4 and abs(float(v.std()) - 0.02) < 2e-4


def test_probability_ties_hidden_in_exp_values():
    """The GPU decode test's tie logits: the two named experts have exp values
    one ulp apart but equal probabilities, so ranking by exp value puts the
    higher index first while the reference order puts the lower index first."""
    from routing_cases import TIE_LOGITS

    for lg, (a, b) in TIE_LOGITS:
        lg = np.array(lg, np.float32)
        mx = lg.max()
        e = [O.expf(float(np.float32(v - mx))) for v in lg]
        p = O.softmax(lg)
        assert e[a] > e[b] and a > b
        assert p[a] == p[b]
        idx, _ = O.top_k(p, 2)
        assert list(idx) == [b, a]


# ---------------------------------------------------------------------------
# RMSNorm, RoPE and attention (src/ops/norm.rs, src/ops/rope.rs,
# src/model/attention.rs)
# ---------------------------------------------------------------------------

def test_rms_norm_reference_case():
    # src/ops/norm.rs:34-48
    x = np.array([3.0, -4.0, 0.0, 5.0], dtype=np.float32)
    out = O.rms_norm(x, np.ones(4, np.float32), 0.0)
    assert abs(np.sqrt(np.mean(out.astype(np.float64) ** 2)) - 1.0) < 1e-6
    y = O.rms_norm_in_place(x, np.full(4, 2.0, np.float32), 0.0)
    assert np.max(np.abs(y - 2.0 * out)) < 1e-6


def test_rms_norm_sums_squares_in_order():
    # squares [2^24, 1, 1]: in order (2^24 + 1) + 1 = 2^24 (two ties to even);
    # summed pairwise the total would be 2^24 + 2, giving another scale
    x = np.array([4096.0, 1.0, 1.0], dtype=np.float32)
    got = O.rms_norm(x, np.ones(3, np.float32), 0.0)
    in_order = np.float32(1.0) / np.sqrt(np.float32(16777216.0) / np.float32(3.0))
    pairwise = np.float32(1.0) / np.sqrt(np.float32(16777218.0) / np.float32(3.0))
    assert in_order != pairwise
    assert got[1] == in_order


def test_rms_norm_and_in_place_associate_differently():
    # rms_norm is (x * scale) * w; rms_norm_in_place is x * (scale * w).  The
    # scale is read back from a unit-weight norm of a row whose first value
    # is 1 (1 * scale * 1 = scale), then both associations are checked on
    # rows where they round differently.
    rng = np.random.default_rng(3)
    differ = 0
    for _ in range(200):
        x = rng.standard_normal(8).astype(np.float32)
        x[0] = 1.0
        w = rng.standard_normal(8).astype(np.float32)
        scale = O.rms_norm(x, np.ones(8, np.float32), 1e-6)[0]
        a, b = O.rms_norm(x, w, 1e-6), O.rms_norm_in_place(x, w, 1e-6)
        assert np.array_equal(a, (x * scale) * w)
        assert np.array_equal(b, x * (scale * w))
        differ += int(not np.array_equal(a, b))
    assert differ > 0


def test_rope_reference_case_and_quarter_turn():
    # src/ops/rope.rs:52-69: position 0 is the identity, a rotation keeps the norm
    h = np.arange(1, 9, dtype=np.float32)
    c0, s0 = O.rope_angles(8, 10000.0, 0)
    assert np.array_equal(O.rope_apply(h, c0, s0), h)
    c, s = O.rope_angles(8, 10000.0, 17)
    r = O.rope_apply(h, c, s)
    assert abs(float(np.sum(r * r)) - float(np.sum(h * h))) < 1e-3 and not np.array_equal(r, h)
    # cos 0, sin 1: (a, b) -> (-b, a) exactly (rotate-half pairs i and i + d/2)
    q = O.rope_apply(h, np.zeros(4, np.float32), np.ones(4, np.float32))
    assert np.array_equal(q, np.concatenate([-h[4:], h[:4]]))


def _attention(dtype, H, nh, nkv, hd, seed, qk_norm=True, identity_o=False, std=0.05):
    mats = []
    for j, (r, c) in enumerate(((nh * hd, H), (nkv * hd, H), (nkv * hd, H), (H, nh * hd))):
        if j == 3 and identity_o:
            mats.append(O.encode_matrix(dtype, np.eye(r, c, dtype=np.float32)))
        else:
            mats.append(O.encode_matrix(dtype, O.normal(seed + j, r * c, 0.0, std).reshape(r, c)))
    qn = kn = None
    if qk_norm:
        qn, kn = O.normal(seed + 10, hd, 1.0, 0.1), O.normal(seed + 11, hd, 1.0, 0.1)
    return O.OracleAttention(dtype, H, nh, nkv, hd, 1e-6, *mats, q_norm=qn, k_norm=kn, max_len=64), mats


def test_attention_first_position_returns_the_value_heads():
    # seq_len 1: softmax gives p = 1, so the context is each head's value head
    # (GQA: query heads h share value head h // group); with an identity
    # o_proj the output is the context itself
    H, nh, nkv, hd = 64, 4, 2, 16
    A, mats = _attention(O.F32, H, nh, nkv, hd, seed=5, identity_o=True)
    x = O.normal(9, H)
    c, s = O.rope_angles(hd, 1e6, 0)
    out = A.forward(x, c, s)
    v = O.matvec(O.F32, nkv * hd, H, mats[2], x)
    want = np.concatenate([v[(h // (nh // nkv)) * hd:(h // (nh // nkv) + 1) * hd] for h in range(nh)])
    assert np.array_equal(out, want)


def test_attention_equal_keys_average_the_values():
    # the same token twice: equal keys, p = 0.5 each, context 0.5 v + 0.5 v = v
    H, nh, nkv, hd = 64, 4, 4, 16
    A, mats = _attention(O.F32, H, nh, nkv, hd, seed=6, identity_o=True, qk_norm=False)
    x = O.normal(10, H)
    c, s = np.ones(hd // 2, np.float32), np.zeros(hd // 2, np.float32)
    first = A.forward(x, c, s)
    second = A.forward(x, c, s)
    assert np.array_equal(first, second)


def test_attention_close_to_float64_model():
    H, nh, nkv, hd = 64, 4, 2, 16
    A, mats = _attention(O.F32, H, nh, nkv, hd, seed=7, qk_norm=True)
    W = [O.decode_row(O.F32, m, m.size // 4).astype(np.float64) for m in mats]
    Wq, Wk, Wv = W[0].reshape(nh * hd, H), W[1].reshape(nkv * hd, H), W[2].reshape(nkv * hd, H)
    Wo = W[3].reshape(H, nh * hd)
    qn, kn = A.q_norm.astype(np.float64), A.k_norm.astype(np.float64)
    Ks, Vs = [], []

    def norm_rope(hv, w, c, s):
        hv = hv / np.sqrt(np.mean(hv * hv) + 1e-6) * w
        a, b = hv[:hd // 2], hv[hd // 2:]
        return np.concatenate([a * c - b * s, b * c + a * s])

    for pos in range(6):
        x = O.normal(20 + pos, H).astype(np.float64)
        c, s = (v.astype(np.float64) for v in O.rope_angles(hd, 1e6, pos))
        got = A.forward(x.astype(np.float32), c.astype(np.float32), s.astype(np.float32))
        q, k, v = Wq @ x, Wk @ x, Wv @ x
        q = np.concatenate([norm_rope(q[h * hd:(h + 1) * hd], qn, c, s) for h in range(nh)])
        k = np.concatenate([norm_rope(k[h * hd:(h + 1) * hd], kn, c, s) for h in range(nkv)])
        Ks.append(k)
        Vs.append(v)
        ctx = []
        for h in range(nh):
            g = h // (nh // nkv)
            sc = np.array([q[h * hd:(h + 1) * hd] @ K[g * hd:(g + 1) * hd] for K in Ks]) / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            p /= p.sum()
            ctx.append(sum(pi * V[g * hd:(g + 1) * hd] for pi, V in zip(p, Vs)))
        want = Wo @ np.concatenate(ctx)
        assert np.max(np.abs(got - want)) < 1e-4 * max(1.0, np.max(np.abs(want)))
