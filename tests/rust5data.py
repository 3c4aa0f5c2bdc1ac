"""Reconstruction of the labs/rust-5 GEMV input file (r5data.bin).

Prose spec (labs/rust-5/reports/rust-5/BUILD.md:12): integer-only splitmix64,
seed 20261004, value = (int24 - 2^23) * 2^-24; a 64-byte header ("R5DATA01",
5 sets, 5 shapes, M and K list), then for set 0..4, for shape 576x1536,
576x576, 1536x576, 2048x2048, 256x256: W (row-major fp32) then x.
The int24 is the top 24 bits of each splitmix64 output, one continuous
stream; the header is "R5DATA01", u32 5, u32 5, (M, K) u32 pairs, zero pad.
This reproduces the published file sha256 3989ed8d... (box1/run.log:4).
"""
import hashlib
import struct

import numpy as np

SHAPES = [(576, 1536), (576, 576), (1536, 576), (2048, 2048), (256, 256)]
SEED = 20261004
GAMMA = np.uint64(0x9E3779B97F4A7C15)


def splitmix64(seed, start, n):
    i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + i * GAMMA
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def values(z):
    v = (z >> np.uint64(40)).astype(np.int64) - (1 << 23)
    return (v.astype(np.float64) * 2.0 ** -24).astype(np.float32)


def sets():
    """Yields (set, (M, K), W float32[M,K], x float32[K]) in file order."""
    off = 0
    for st in range(5):
        for (M, K) in SHAPES:
            n = M * K + K
            v = values(splitmix64(SEED, off, n))
            off += n
            yield st, (M, K), v[:M * K].reshape(M, K), v[M * K:]


def file_sha256():
    h = hashlib.sha256()
    hdr = b"R5DATA01" + struct.pack("<II", 5, 5) + b"".join(struct.pack("<II", m, k) for m, k in SHAPES)
    h.update(hdr + b"\0" * (64 - len(hdr)))
    for _, _, W, x in sets():
        h.update(W.tobytes())
        h.update(x.tobytes())
    return h.hexdigest()
