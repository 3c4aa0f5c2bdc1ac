"""The oracle's seeded sampler (CIS-2 v0.4 draft section 14,
code/patches/cis2-spec__seeded-sampling.patch:57-196) against the draft's
own known answers, and its sort-based rank/top-k/top-p against a
brute-force restatement of the rank definition on small vocabularies."""
import struct

import numpy as np
import pytest

import _oracle as O


def f32(bits):
    return struct.unpack("<f", struct.pack("<I", bits))[0]


def bits(x):
    return struct.unpack("<I", struct.pack("<f", float(np.float32(x))))[0]


def test_murmur3_published_empty_key():
    # draft 14.2: the empty key gives 00000000 (hash seed 0) and 514e28b7 (seed 1)
    L = O.lib()
    assert L.orc_murmur3_32(None, 0, 0) == 0x00000000
    assert L.orc_murmur3_32(None, 0, 1) == 0x514E28B7


@pytest.mark.parametrize("seed,step,index,h,u,g", [
    (0x0000000000000001, 0, 0, 0x07731EA2, 0x3CEE63E0, 0xBFA1B32B),
    (0x0000000000000001, 0, 1, 0xC832451B, 0x3F483245, 0x3FB392C7),
    (0x0000000000000001, 1, 0, 0xC0D0C4FA, 0x3F40D0C5, 0x3FA15FFE),
    (0xFFFFFFFFFFFFFFFF, 7, 49151, 0xE682298D, 0x3F668229, 0x40104F5A),
])
def test_noise_known_answers(seed, step, index, h, u, g):
    # draft 14.6 table
    hh, uu, gg = O.sample_noise(seed, step, index)
    assert hh == h
    assert bits(uu) == u
    assert bits(gg) == g


def test_noise_key_layout_is_murmur_of_16_le_bytes():
    # the key is seed (u64 LE) || step (u32 LE) || index (u32 LE), hash seed "CIS2"
    L = O.lib()
    rng = np.random.default_rng(3)
    for _ in range(64):
        seed = int(rng.integers(0, 2**63)) * 2 + int(rng.integers(0, 2))
        step, idx = int(rng.integers(0, 2**32)), int(rng.integers(0, 2**32))
        key = struct.pack("<QII", seed, step, idx)
        buf = np.frombuffer(key, dtype=np.uint8).copy()
        assert O.sample_noise(seed, step, idx)[0] == L.orc_murmur3_32(buf.ctypes.data, 16,
                                                                        0x43495332)


def test_toy_vector():
    # draft 14.6: V = 8, seed 1, step 0, T = 0.8, top_k 4, top_p 0.9
    lg = np.array([1.0, 2.0, 2.0, -1.0, 0.5, 3.0, 3.0, -4.0], np.float32)
    nid, z, nk = O.sample(lg, 1, 0, f32(0x3F4CCCCD), 4, f32(0x3F666666))
    assert nid == 1
    assert nk == 4
    zb = [bits(v) for v in z]
    assert zb[1] == 0x4079C964 and zb[2] == 0x4026F5C5
    assert zb[5] == 0x407320FD and zb[6] == 0x4011C83A
    assert all(zb[i] == 0xFF800000 for i in (0, 3, 4, 7))


@pytest.mark.parametrize("T,k,p", [
    (0.0, 0, 1.0), (-1.0, 0, 1.0), (float("inf"), 0, 1.0), (float("nan"), 0, 1.0),
    (1.0, 0, 0.0), (1.0, 0, 1.5), (1.0, 0, float("nan")), (1.0, 0, -0.5),
])
def test_invalid_parameters(T, k, p):
    assert O.lib().orc_sample_params_ok(T, k, p) != 0
    nid, _, _ = O.sample(np.zeros(4, np.float32), 1, 0, T, k, p)
    assert nid is None


def test_nan_logit_is_refused():
    lg = np.array([0.5, np.nan, 1.0], np.float32)
    assert O.sample(lg, 1, 0, 1.0, 0, 1.0)[0] is None


def brute(lg, seed, step, T, top_k, top_p):
    """The draft's definitions taken literally, O(V^2): rank(i) = number of
    indices that precede i; the kept set by rank; z; the section 11.2 scan."""
    V = lg.size
    s = [np.float32(v) / np.float32(T) for v in lg]
    rank = [sum(1 for j in range(V) if s[j] > s[i] or (s[j] == s[i] and j < i))
            for i in range(V)]
    by_rank = [0] * V
    for i in range(V):
        by_rank[rank[i]] = i
    K = top_k if 0 < top_k < V else V
    keep = K
    if np.float32(top_p) < np.float32(1.0):
        m = s[by_rank[0]]
        e = [np.float32(O.lib().orc_exp(float(np.float32(s[by_rank[r]] - m)))) for r in range(K)]
        den = np.float32(0.0)
        for r in range(K):
            den = np.float32(den + e[r])
        c = np.float32(0.0)
        for r in range(K):
            if r > 0 and not (c < np.float32(top_p)):
                keep = r
                break
            c = np.float32(c + np.float32(e[r] / den))
    kept = set(by_rank[:keep])
    z = [np.float32(-np.inf)] * V
    for i in kept:
        z[i] = np.float32(s[i] + np.float32(O.sample_noise(seed, step, i)[2]))
    best, bi = z[0], 0
    for i in range(1, V):
        if z[i] > best:
            best, bi = z[i], i
    return bi, keep


def test_rank_order_top_k_top_p_brute_force():
    O.lib()  # pins FTZ/DAZ on this thread before any float work
    rng = np.random.default_rng(11)
    cases = 0
    for V in (1, 2, 3, 7, 16, 33, 64):
        for trial in range(6):
            kind = trial % 3
            if kind == 0:
                lg = rng.standard_normal(V).astype(np.float32)
            elif kind == 1:  # many ties, signed zeros
                lg = rng.integers(-2, 3, V).astype(np.float32) * np.float32(0.5)
                lg[rng.random(V) < 0.3] = np.float32(-0.0)
            else:  # wide spread: exp underflows for the tail
                lg = (rng.standard_normal(V) * 60).astype(np.float32)
            seed = int(rng.integers(0, 2**63))
            step = int(rng.integers(0, 1000))
            T = float(np.float32(rng.choice([0.25, 0.8, 1.0, 3.0])))
            k = int(rng.choice([0, 1, 2, V, V + 3, max(1, V // 2)]))
            p = float(np.float32(rng.choice([1.0, 0.9, 0.5, 0.05])))
            want = brute(lg, seed, step, T, k, p)
            nid, _, nk = O.sample(lg, seed, step, T, k, p)
            assert (nid, nk) == want, (V, trial, T, k, p)
            cases += 1
    assert cases == 42
