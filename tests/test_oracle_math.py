"""The oracle's pinned math, pinned against the reference's published KATs,
the reference's own cis2_math.h compiled here, and closed forms."""
import struct

import numpy as np
import pytest

import _oracle as O

FNS = ["exp", "sin", "cos", "ln", "silu", "rsqrt", "sqrt"]


def bits(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


def test_fpenv_pin():
    assert O.lib().orc_fpenv_pin() == 0


def test_table_digest_kat():
    # code/cis2-fp/verify3/selftest.c:41-59
    assert O.table_digest() == "23c7bfaf5cef0095fd021af2eb1808abb4928bae4219756d86bdac670a06b35d"


def test_inv_freq_digest_kat_smollm2():
    # code/cis2-fp/verify3/selftest.c:61-83 (theta 1e5, head_dim 64)
    _, d = O.inv_freq(100000.0, 64)
    assert d == "da9f6dcfde0425588815509e874515cdcd3d6b8818b6d0136590052e7bbf6f12"


def test_rsqrt_64_is_exactly_one_eighth():
    assert struct.pack("<f", O.lib().orc_rsqrt(64.0)) == struct.pack("<I", 0x3E000000)


def test_dot_seq_order_kat():
    # (1e8 + 1) - 1e8 == 0 in strict left-to-right fp32 (math.rs:614-624)
    a = np.array([1e8, 1.0, -1e8], dtype=np.float32)
    b = np.ones(3, dtype=np.float32)
    assert O.lib().orc_dot_seq(O.ptr(a, O.c_fp), O.ptr(b, O.c_fp), 3) == 0.0


def test_exp_closed_forms():
    v = O.math_map("exp", np.array([0.0, -0.0, 88.5, -88.5, np.nan, np.inf, -np.inf], np.float32))
    assert list(bits(v)) == [0x3F800000, 0x3F800000, 0x7F800000, 0, 0x7FC00000, 0x7F800000, 0]


def test_ln_closed_forms():
    v = O.math_map("ln", np.array([1.0, 0.0, -0.0, -1.0, np.nan], np.float32))
    assert list(bits(v)) == [0, 0xFF800000, 0xFF800000, 0x7FC00000, 0x7FC00000]


def test_sin_cos_at_zero():
    assert bits(O.math_map("sin", np.array([0.0], np.float32)))[0] == 0
    assert bits(O.math_map("cos", np.array([0.0], np.float32)))[0] == 0x3F800000


def _ulp_err(got, ref):
    # ULP of the binary32 result computed in binary64 (the oracle pins FTZ on
    # this thread, so float32 helpers like np.spacing would flush)
    ulp = 2.0 ** (np.floor(np.log2(np.abs(ref))) - 23)
    return np.abs(got.astype(np.float64) - ref) / ulp


def test_math_accuracy_against_libm():
    # spec accuracy statements (CIS2_SPEC_v0.3.md:893-905): exp <= 1 ulp in
    # the working range, sin/cos <= 1.5 ulp over the RoPE angle range.
    rng = np.random.default_rng(7)
    x = rng.uniform(-80, 80, 20000).astype(np.float32)
    assert np.max(_ulp_err(O.math_map("exp", x), np.exp(x.astype(np.float64)))) <= 1.0
    a = rng.uniform(0.01, 8192, 20000).astype(np.float32)
    for fn, ref in (("sin", np.sin), ("cos", np.cos)):
        err = _ulp_err(O.math_map(fn, a), ref(a.astype(np.float64)))
        assert np.percentile(err, 99.9) <= 1.5, fn


@pytest.mark.parametrize("fn", FNS)
def test_oracle_matches_fixture_chunk(fn, math_fixture):
    # one full chunk of 2^24 inputs per function, chosen so the seven
    # functions cover different exponent ranges, recomputed and compared to
    # the exhaustive fixture (which was checked against the reference build)
    chunk = {"exp": 0x42, "sin": 0x45, "cos": 0x3F, "ln": 0x00, "silu": 0xC2,
             "rsqrt": 0x80, "sqrt": 0x7F}[fn]
    h = O.lib().orc_math_chunk_hash(O.FN_IDS[fn], chunk << 24, 1 << 24)
    assert "%016x" % h == math_fixture["chunks"][fn][chunk]


def test_fixture_was_checked_against_reference(math_fixture):
    assert math_fixture["checked_against_reference"] is True
    for fn in FNS:
        assert len(math_fixture["chunks"][fn]) == 256


def test_oracle_matches_reference_math_random():
    R = O.ref_math()
    if R is None:
        pytest.skip("reference cis2_math.h not built here (oracle/_ref)")
    rng = np.random.default_rng(11)
    x = rng.integers(0, 2 ** 32, 1 << 18, dtype=np.uint64).astype(np.uint32).view(np.float32)
    for i, fn in enumerate(FNS):
        want = np.empty_like(x)
        R.ref_math_map(i, O.ptr(x, O.c_fp), O.ptr(want, O.c_fp), x.size)
        assert np.array_equal(bits(O.math_map(fn, x)), bits(want)), fn


def test_tree_sum_closed_form():
    # ((1+2)+(3+4))+5 with the 32-leaf zero-padded block (math.rs:644-651)
    a = np.arange(1, 6, dtype=np.float32)
    assert O.lib().orc_sum_tree(O.ptr(a, O.c_fp), 5) == 15.0
    assert O.lib().orc_sum_tree(O.ptr(a, O.c_fp), 0) == 0.0


def _tree_sum_py(v):
    """Pairwise halving on 32-leaf zero-padded blocks, block partials folded
    left to right (CIS2_V04_TREE_REDUCTION.md:35-98), via numpy float32."""
    acc = np.float32(0.0)
    for s in range(0, len(v), 32):
        leaf = np.zeros(32, np.float32)
        blk = v[s:s + 32]
        leaf[:len(blk)] = blk
        while leaf.size > 1:
            leaf = (leaf[0::2] + leaf[1::2]).astype(np.float32)
        acc = np.float32(acc + leaf[0])
    return acc


def test_tree_sum_brute_force_ragged():
    rng = np.random.default_rng(3)
    for n in [1, 2, 31, 32, 33, 63, 64, 65, 100, 577]:
        v = rng.standard_normal(n).astype(np.float32)
        got = O.lib().orc_sum_tree(O.ptr(v, O.c_fp), n)
        assert np.float32(got).view(np.uint32) == _tree_sum_py(v).view(np.uint32)
        R = O.ref_math()
        if R is not None:
            assert np.float32(R.ref_sum_tree(O.ptr(v, O.c_fp), n)).view(np.uint32) == \
                np.float32(got).view(np.uint32)


def test_softmax_matches_reference_and_closed_form():
    v = np.array([0.5, 2.0, 2.0, -1.0], np.float32)
    o = v.copy()
    O.lib().orc_softmax(O.ptr(o, O.c_fp), 4, 0)
    assert abs(float(o.sum()) - 1.0) < 1e-6 and o[1] == o[2]
    R = O.ref_math()
    if R is not None:
        rng = np.random.default_rng(5)
        for n in [1, 7, 64, 300]:
            for mode in (0, 1):
                x = rng.standard_normal(n).astype(np.float32)
                a, b = x.copy(), x.copy()
                O.lib().orc_softmax(O.ptr(a, O.c_fp), n, mode)
                R.ref_softmax(O.ptr(b, O.c_fp), n, mode)
                assert np.array_equal(bits(a), bits(b))


def test_argmax_first_maximum_wins():
    # strict > scan: tie goes to the lowest index (coverage vector semantics,
    # labs/w1x-coverage/plans/2026-10-16-w1x-coverage-PLAN.md:12-13)
    v = np.zeros(20, np.float32)
    v[5] = v[17] = 3.0
    assert O.lib().orc_argmax(O.ptr(v, O.c_fp), 20) == 5
    w = np.array([-0.0, 0.0, -1.0], np.float32)
    assert O.lib().orc_argmax(O.ptr(w, O.c_fp), 3) == 0
