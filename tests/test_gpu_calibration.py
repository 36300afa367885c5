"""The calibration kernels the measurements rest on, through the C ABI:
hale_copy_device (the yardstick of the HBM traffic counters) copies every
byte, and hale_stream_read_device (the one-launch streaming-read ceiling
timed beside the decode kernels) reads every byte of its range: each
work-group's XOR equals numpy's over the same chunk, for chunk counts that
divide the range, that do not, and that leave work-groups without a chunk.
Bar: exact bytes and checksums."""
import numpy as np
import pytest

import hale_moe as H

pytestmark = pytest.mark.gpu


def chunk_xors(words, workgroups):
    n16 = words.size // 4
    chunk = -(-n16 // workgroups)
    out = np.zeros(workgroups, np.uint32)
    for g in range(workgroups):
        b0, b1 = min(n16, g * chunk), min(n16, g * chunk + chunk)
        if b1 > b0:
            out[g] = np.bitwise_xor.reduce(words[4 * b0:4 * b1])
    return out


def test_copy_device_copies_every_byte(ctx):
    n = (3 << 20) + 80
    data = np.random.default_rng(1).integers(0, 2**32, n // 4, dtype=np.uint32)
    a, b = ctx.malloc(n), ctx.malloc(n + 64)
    a.upload(data)
    b.upload(np.full((n + 64) // 4, 0xDEADBEEF, np.uint32))
    b.copy_from(a, n)
    got = b.download(np.uint32, (n + 64) // 4)
    assert (got[:n // 4] == data).all()
    assert (got[n // 4:] == 0xDEADBEEF).all()  # nothing past n written
    a.free()
    b.free()


@pytest.mark.parametrize("nbytes,workgroups", [
    ((1 << 20) + 48, 1), ((1 << 20) + 48, 7), ((1 << 20) + 48, 512),
    (4096, 1000),           # 256 chunks of one load: work-groups past them read nothing
    (64 << 20, 2048),       # the size class of the decode kernels
])
def test_stream_read_checksums(ctx, nbytes, workgroups):
    data = np.random.default_rng(nbytes + workgroups).integers(0, 2**32, nbytes // 4, dtype=np.uint32)
    buf = ctx.malloc(nbytes + 16)
    buf.upload(data, offset=16)
    out = ctx.malloc(4 * workgroups)
    out.upload(np.full(workgroups, 0xFFFFFFFF, np.uint32))
    buf.stream_read(nbytes, workgroups, out, offset=16)
    got = out.download(np.uint32, workgroups)
    assert (got == chunk_xors(data, workgroups)).all()
    buf.free()
    out.free()


def test_stream_read_refuses_bad_arguments(ctx):
    buf, out = ctx.malloc(4096), ctx.malloc(4 * 65536)
    for nbytes, wg, off in ((4096, 0, 0), (4096, 65536, 0), (4008, 4, 0), (4080, 4, 8)):
        with pytest.raises(ValueError):
            buf.stream_read(nbytes, wg, out, offset=off)
    buf.free()
    out.free()
