"""The .bin shard format and batch order of train.py:27-62.  CPU only."""

import itertools

import numpy as np
import pytest

from attention_nn_amd.data import SHARD_MAGIC, batch_iterator, load_shard, write_shard


def _shards(tmp_path, sizes):
    out = []
    base = 0
    for i, n in enumerate(sizes):
        path = tmp_path / f"fineweb_train_{i:06d}.bin"
        write_shard(path, (np.arange(n) + base) % 65536)
        base += n
        out.append(load_shard(path))
    return out


def test_header_and_tokens(tmp_path):
    path = tmp_path / "s.bin"
    toks = np.random.default_rng(0).integers(0, 50257, 1000)
    write_shard(path, toks)
    head = np.fromfile(path, dtype=np.int32, count=256)
    assert head[0] == SHARD_MAGIC and head[2] == 1000
    assert path.stat().st_size == 256 * 4 + 1000 * 2
    got = load_shard(path)
    assert got.dtype == np.uint16 and np.array_equal(got, toks)
    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"\0" * 2048)
    with pytest.raises(ValueError, match="magic"):
        load_shard(bad)


def test_batches_are_shifted_and_contiguous(tmp_path):
    sh = _shards(tmp_path, [200])
    it = batch_iterator(sh, 2, 8)
    x0, y0 = next(it)
    x1, _ = next(it)
    assert x0.shape == (2, 8) and x0.dtype == np.int32
    flat = np.concatenate([x0.ravel(), x1.ravel()])
    assert np.array_equal(flat, np.arange(32))                 # consecutive spans of B*T
    assert np.array_equal(y0.ravel(), np.arange(1, 17))        # targets = inputs shifted by one


def test_wraps_to_next_shard_and_cycles(tmp_path):
    sh = _shards(tmp_path, [40, 30])
    starts = [int(x[0, 0]) for x, _ in itertools.islice(batch_iterator(sh, 1, 10), 6)]
    # shard 0 holds spans at 0, 10, 20 (20 + 10 + 1 < 40 ... 30 + 11 >= 40 moves on),
    # shard 1 (tokens 40..69) at 40, 50, then back to shard 0
    assert starts == [0, 10, 20, 40, 50, 0]


def test_start_tokens_equals_skipping_batches(tmp_path):
    """Exact while the skip stays inside the first shard, and across shards
    when their lengths minus (B*T + 1) are multiples of B*T."""
    B, T = 2, 16
    sh = _shards(tmp_path, [500, 300, 420])
    full = list(itertools.islice(batch_iterator(sh, B, T), 40))
    for k in (0, 3, 11, 14):                  # 14 * 32 = 448 < 500 - 33
        resumed = list(itertools.islice(batch_iterator(sh, B, T, start_tokens=k * B * T), 5))
        for (a, b), (c, d) in zip(full[k:k + 5], resumed):
            assert np.array_equal(a, c) and np.array_equal(b, d), k
    al = _shards(tmp_path, [33 + 4 * 32, 33 + 3 * 32])   # 4 and 3 whole spans
    full = list(itertools.islice(batch_iterator(al, B, T), 20))
    for k in (4, 6, 9, 13):
        resumed = list(itertools.islice(batch_iterator(al, B, T, start_tokens=k * B * T), 3))
        for (a, _), (c, _) in zip(full[k:k + 3], resumed):
            assert np.array_equal(a, c), k


def test_start_tokens_offset_past_an_unaligned_shard(tmp_path):
    """The reference's arithmetic past a shard of 500 tokens, span 32: the
    skip of 15 spans (480) lands 13 tokens into shard 1 (480 - 467), while a
    continuous run's 16th batch starts shard 1 at its first token."""
    sh = _shards(tmp_path, [500, 300])
    x, _ = next(batch_iterator(sh, 2, 16, start_tokens=15 * 32))
    assert int(x[0, 0]) == 500 + 13
    cont = list(itertools.islice(batch_iterator(sh, 2, 16), 16))
    assert int(cont[15][0][0, 0]) == 500


def _stream_by_walking(shards, B, T, start, n):
    """The batch starts of the order as specified: skip `start` tokens over the
    shard rooms, then walk each shard by spans below its room, cyclically."""
    span = B * T
    rooms = [len(s) - span - 1 for s in shards]
    skip = start % sum(rooms)
    si = 0
    while skip >= rooms[si]:
        skip -= rooms[si]
        si += 1
    out, p = [], skip
    while len(out) < n:
        if p >= rooms[si]:
            si, p = (si + 1) % len(shards), 0
            continue
        out.append((si, p))
        p += span
    return out


@pytest.mark.parametrize("sizes,B,T", [([500, 300, 420], 2, 16), ([97, 61], 1, 7),
                                       ([40, 30], 1, 10), ([1000], 4, 8)])
def test_order_equals_specification(tmp_path, sizes, B, T):
    """Against a step-by-step walk of the order at many resume offsets,
    including every offset inside the first few spans and past each shard."""
    sh = _shards(tmp_path, sizes)
    base = np.concatenate([[0], np.cumsum(sizes)])
    rooms = [n - B * T - 1 for n in sizes]
    starts = set(range(0, 3 * B * T)) | {sum(rooms[:i]) + d for i in range(len(sizes) + 1)
                                         for d in (-1, 0, 1)} | {sum(rooms) * 2 + 5}
    for st in sorted(s for s in starts if s >= 0):
        want = _stream_by_walking(sh, B, T, st, 2 * len(sizes) + 6)
        got = list(itertools.islice(batch_iterator(sh, B, T, start_tokens=st), len(want)))
        for (si, p), (x, y) in zip(want, got):
            assert int(x[0, 0]) == int(base[si] + p) % 65536, (st, si, p)
            assert int(y[-1, -1]) == int(base[si] + p + B * T) % 65536
