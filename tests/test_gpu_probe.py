"""nmoe_hip_read_probe, the streaming-ceiling measurement entry point: it
must read every byte it is given exactly once (its fold is checked word for
word against numpy) and reject what it cannot read."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

BLOCKS, THREADS, LOADS = 256, 512, 8


def probe_fold(words: np.ndarray) -> np.ndarray:
    """sink[b*8 + wave]: the XOR of every u32 that wave's lanes load.  Block b
    owns 16-byte items [b*per, min((b+1)*per, n)), per = ceil(n / 256); lane
    t of the block loads items b*per + t + 512*j, j < 8."""
    n = words.size // 4
    per = -(-n // BLOCKS)
    lanes = np.bitwise_xor.reduce(words.reshape(n, 4), axis=1)
    sink = np.zeros(BLOCKS * THREADS // 64, np.uint32)
    for b in range(BLOCKS):
        lo, hi = b * per, min((b + 1) * per, n)
        if lo >= hi:
            continue
        for t0 in range(0, THREADS, 64):
            acc = np.uint32(0)
            for j in range(LOADS):
                i0, i1 = lo + t0 + THREADS * j, min(lo + t0 + 64 + THREADS * j, hi)
                if i0 < i1:
                    acc ^= np.bitwise_xor.reduce(lanes[i0:i1])
            sink[b * 8 + t0 // 64] = acc
    return sink


@pytest.mark.parametrize("nbytes", [16, 4096 + 48, 14155776, 16 << 20])
def test_read_probe_folds_every_word(nbytes):
    import nmoe_hip as nh

    rng = np.random.default_rng(nbytes)
    words = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    with nh.Context(0, max_tokens=1) as ctx:
        src = ctx.to_device(words)
        sink = ctx.alloc(BLOCKS * 8 * 4)
        ctx._check(ctx.read_probe(src, nbytes, sink))
        ctx.sync()
        got = sink.download(np.uint32, BLOCKS * 8)
    np.testing.assert_array_equal(got, probe_fold(words))


def test_read_probe_rejects():
    import nmoe_hip as nh

    with nh.Context(0, max_tokens=1) as ctx:
        src, sink = ctx.alloc((16 << 20) + 64), ctx.alloc(BLOCKS * 8 * 4)
        for ptr, n in ((src.ptr, 0), (src.ptr, 24), (src.ptr + 8, 64), (src.ptr, (16 << 20) + 16)):
            assert ctx.read_probe(ptr, n, sink) == nh.EINVAL
        assert ctx.read_probe(src, 64, None) == nh.EINVAL
