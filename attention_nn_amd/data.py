"""Token shards of the training data (``train.py:27-62``).

A shard is a ``.bin`` file: a header of 256 int32 (header[0] = 20240520,
header[2] = token count) followed by the tokens as uint16.  ``load_shard``
memory-maps the tokens; ``batch_iterator`` yields consecutive (inputs,
targets) int32 batches of shape (B, T), targets being the inputs shifted by
one token, cycling through the shards in order, with ``start_tokens``
fast-forwarding a resumed run without reading data.
"""

import numpy as np

SHARD_MAGIC = 20240520
HEADER_INTS = 256


def load_shard(path):
    """Tokens of one shard as a read-only uint16 memmap (``train.py:27-33``)."""
    header = np.fromfile(path, dtype=np.int32, count=HEADER_INTS)
    if header.size < HEADER_INTS or int(header[0]) != SHARD_MAGIC:
        raise ValueError(f"{path}: magic number mismatch")
    n = int(header[2])
    return np.memmap(path, dtype=np.uint16, mode="r", offset=HEADER_INTS * 4, shape=(n,))


def write_shard(path, tokens, version=1):
    """Write ``tokens`` (< 65536) as a shard in the same layout (for tests and tools)."""
    tokens = np.asarray(tokens)
    if tokens.size and (tokens.min() < 0 or tokens.max() > 65535):
        raise ValueError("shard tokens must fit in uint16")
    header = np.zeros(HEADER_INTS, dtype=np.int32)
    header[0], header[1], header[2] = SHARD_MAGIC, version, tokens.size
    with open(path, "wb") as f:
        f.write(header.tobytes())
        f.write(tokens.astype(np.uint16).tobytes())


def batch_iterator(shards, batch_size, seq_len, start_tokens=0):
    """Endless (inputs, targets) int32 numpy batches of shape (B, T)
    (``train.py:36-62``).

    Each batch reads B*T + 1 consecutive tokens at the current offset; the
    offset advances by B*T.  A shard whose remaining tokens cannot hold the
    next span is left for the next shard (cyclic), from its start.
    ``start_tokens`` skips that many tokens first, counted as the reference
    counts them: over shard lengths minus (B*T + 1).  That equals skipping
    start_tokens / (B*T) batches while the skip stays inside the first shard
    (or when every such length is a multiple of B*T); past a shard whose
    length is not, the resumed offset is the reference's, not the batch
    boundary a continuous run would reach."""
    if not isinstance(shards, (list, tuple)):
        shards = [shards]
    span = batch_size * seq_len
    sizes = [len(s) - span - 1 for s in shards]
    if any(n <= 0 for n in sizes):
        raise ValueError("every shard must hold more than batch_size * seq_len + 1 tokens")
    offset = start_tokens % sum(sizes)
    si = 0
    while offset >= sizes[si]:
        offset -= sizes[si]
        si += 1
    pos = offset
    while True:
        tokens = shards[si]
        if pos + span + 1 >= len(tokens):
            si = (si + 1) % len(shards)
            pos = 0
            tokens = shards[si]
        buf = np.asarray(tokens[pos:pos + span + 1]).astype(np.int32)
        yield buf[:-1].reshape(batch_size, seq_len), buf[1:].reshape(batch_size, seq_len)
        pos += span
