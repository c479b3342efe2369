"""nmoe_hip_read_probe and nmoe_hip_read_probe_grid, the streaming-ceiling
measurement entry points: they must read every byte they are given exactly
once, at every launch shape and past one round of loads (the fold is
checked word for word against numpy), and reject what they cannot read."""
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


def grid_fold(words: np.ndarray, blocks: int, threads: int) -> np.ndarray:
    """The same fold for any shape and any number of rounds: within block b's
    span, item i is loaded by lane (i - b*per) % threads, whatever the round
    and the load slot, so wave w's word is the XOR over the span's items
    whose position modulo threads falls in [64w, 64w + 64)."""
    n = words.size // 4
    per = -(-n // blocks)
    lanes = np.bitwise_xor.reduce(words.reshape(n, 4), axis=1)
    sink = np.zeros(blocks * threads // 64, np.uint32)
    for b in range(blocks):
        span = lanes[b * per:min((b + 1) * per, n)]
        if span.size == 0:
            continue
        pad = np.zeros(-(-span.size // threads) * threads, np.uint32)
        pad[:span.size] = span
        per_lane = np.bitwise_xor.reduce(pad.reshape(-1, threads), axis=0)
        sink[b * threads // 64:(b + 1) * threads // 64] = np.bitwise_xor.reduce(per_lane.reshape(-1, 64), axis=1)
    return sink


@pytest.mark.parametrize("nbytes,blocks,threads,loads", [
    ((40 << 20) + 4096, 256, 512, 8),   # past one round: 2.5 rounds a block
    (14155776, 1024, 256, 16),
    (14155776, 2048, 1024, 4),
    (3 * 16 * 1000 + 16, 3, 64, 1),     # ragged spans, several rounds
    (16, 256, 1024, 2),                 # the near-empty launch: one item
    ((96 << 20), 8192, 64, 2),
])
def test_read_probe_grid_folds_every_word(nbytes, blocks, threads, loads):
    import nmoe_hip as nh

    print(f"[probe] grid {blocks}x{threads}x{loads} {nbytes} B", flush=True)
    rng = np.random.default_rng(nbytes + blocks)
    words = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    with nh.Context(0, max_tokens=1) as ctx:
        src = ctx.to_device(words)
        nw = blocks * threads // 64
        sink = ctx.alloc(nw * 4)
        ctx._check(ctx.read_probe_grid(src, nbytes, blocks, threads, loads, sink))
        ctx.sync()
        got = sink.download(np.uint32, nw)
    np.testing.assert_array_equal(got, grid_fold(words, blocks, threads))
    if (blocks, threads, loads) == (256, 512, 8):
        np.testing.assert_array_equal(got, probe_fold_rounds(words))


def probe_fold_rounds(words: np.ndarray) -> np.ndarray:
    """The default shape's fold written out load by load over its rounds
    (lane t of block b, round r, slot j: item b*per + r*4096 + t + 512*j)."""
    n = words.size // 4
    per = -(-n // BLOCKS)
    lanes = np.bitwise_xor.reduce(words.reshape(n, 4), axis=1)
    sink = np.zeros(BLOCKS * THREADS // 64, np.uint32)
    for b in range(BLOCKS):
        lo, hi = b * per, min((b + 1) * per, n)
        for base in range(lo, hi, THREADS * LOADS):
            for t0 in range(0, THREADS, 64):
                for j in range(LOADS):
                    i0, i1 = base + t0 + THREADS * j, min(base + t0 + 64 + THREADS * j, hi)
                    if i0 < i1:
                        sink[b * 8 + t0 // 64] ^= np.bitwise_xor.reduce(lanes[i0:i1])
    return sink


def test_read_probe_rejects():
    import nmoe_hip as nh

    with nh.Context(0, max_tokens=1) as ctx:
        src, sink = ctx.alloc((16 << 20) + 64), ctx.alloc(BLOCKS * 8 * 4)
        for ptr, n in ((src.ptr, 0), (src.ptr, 24), (src.ptr + 8, 64)):
            assert ctx.read_probe(ptr, n, sink) == nh.EINVAL
        assert ctx.read_probe(src, 64, None) == nh.EINVAL
        for blocks, threads, loads in ((0, 512, 8), (8193, 512, 8), (256, 32, 8), (256, 1088, 8), (256, 96, 8),
                                       (256, 512, 3), (256, 512, 32)):
            assert ctx.read_probe_grid(src, 64, blocks, threads, loads, sink) == nh.EINVAL
