"""Token shards of the training data: the ``.bin`` format and batch order of
``train.py:27-62``.

A shard is a header of 256 little-endian int32 (word 0 = 20240520, word 2 =
token count) followed by the tokens as little-endian uint16.

Batch order.  With span = B*T, a batch is the span + 1 consecutive tokens
starting at some offset p of a shard (inputs = the first span, targets = the
last span).  A shard of n tokens has *room* n - span - 1: the offsets that
still fit are exactly the p < room, and the shard is walked at p = p0,
p0 + span, ... below its room, after which the next shard (cyclically) starts
at p = 0.  A resumed run skips ``start_tokens`` counted over the rooms of
the shards in order (modulo their sum), which is how the reference's resume
counts them: the skip lands in the shard whose cumulative room first
exceeds it, at the remainder.  That equals skipping start_tokens / span
batches while the skip stays inside the first shard, or when every room is a
multiple of span; past a shard whose room is not, the resumed offset is the
reference's, not the batch boundary a continuous run would reach.
"""

import itertools

import numpy as np

SHARD_MAGIC = 20240520
HEADER_INTS = 256
HEADER_BYTES = HEADER_INTS * 4


def load_shard(path):
    """Tokens of one shard as a read-only uint16 memmap (``train.py:27-33``)."""
    with open(path, "rb") as f:
        head = np.frombuffer(f.read(HEADER_BYTES), dtype="<i4")
    if head.size != HEADER_INTS or int(head[0]) != SHARD_MAGIC:
        raise ValueError(f"{path}: magic number mismatch")
    count = int(head[2])
    return np.memmap(path, dtype="<u2", mode="r", offset=HEADER_BYTES, shape=(count,))


def write_shard(path, tokens, version=1):
    """Write ``tokens`` (< 65536) as a shard in the same layout (for tests and tools)."""
    tokens = np.asarray(tokens)
    if tokens.size and (tokens.min() < 0 or tokens.max() > 65535):
        raise ValueError("shard tokens must fit in uint16")
    head = np.zeros(HEADER_INTS, dtype="<i4")
    head[[0, 1, 2]] = SHARD_MAGIC, version, tokens.size
    with open(path, "wb") as f:
        f.write(head.tobytes() + tokens.astype("<u2").tobytes())


def resume_point(rooms, start_tokens):
    """(shard index, offset) where a run resumed after ``start_tokens`` begins."""
    ends = np.cumsum(rooms)
    skip = int(start_tokens) % int(ends[-1])
    shard = int(np.searchsorted(ends, skip, side="right"))
    return shard, skip - (int(ends[shard - 1]) if shard else 0)


def batch_iterator(shards, batch_size, seq_len, start_tokens=0):
    """Endless (inputs, targets) int32 numpy batches of shape (B, T) in the
    order described in the module docstring (``train.py:36-62``)."""
    if not isinstance(shards, (list, tuple)):
        shards = [shards]
    span = batch_size * seq_len
    rooms = [len(s) - span - 1 for s in shards]
    if min(rooms) <= 0:
        raise ValueError("every shard must hold more than batch_size * seq_len + 1 tokens")
    first, p0 = resume_point(rooms, start_tokens)
    order = itertools.chain(range(first, len(shards)), itertools.cycle(range(len(shards))))
    for n, si in enumerate(order):
        for p in range(p0 if n == 0 else 0, rooms[si], span):
            window = np.asarray(shards[si][p:p + span + 1], dtype=np.int32)
            yield window[:span].reshape(batch_size, seq_len), window[1:].reshape(batch_size, seq_len)
