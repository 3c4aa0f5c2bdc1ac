"""Device pinned math against the oracle: exhaustive over all 2^32 binary32
inputs for exp, sin, cos, ln, silu, rsqrt and sqrt (chunk-hash fixture that
was itself checked against the reference's cis2_math.h), the FTZ/DAZ probes,
and the divide at the subnormal boundary."""
import numpy as np
import pytest

import _oracle as O
from cis2amd import model as M

pytestmark = pytest.mark.gpu

FNS = ["exp", "sin", "cos", "ln", "silu", "rsqrt", "sqrt"]


def test_device_fpenv_probes():
    # spec §1.3: 2^-126 * 1e-10 -> +0.0 and smallest subnormal + 0.0 -> +0.0
    assert M.fpenv_probe() == (0, 0)


def test_wait_counters_cover_more_operations_than_their_fields():
    """One wave issues 128 vector loads (the vmcnt field holds 63) or 40 LDS
    reads (lgkmcnt: 15) and waits once for zero: every register holds its
    load's value, so the hardware holds issue at a field's maximum.  The
    decode kernel's score tasks keep 64 or 128 loads per thread in flight
    and rely on this."""
    assert M.wait_probe() == (0, 0)


@pytest.mark.parametrize("fn", FNS)
def test_exhaustive_all_inputs(fn, math_fixture):
    got = M.device_math_chunk_hashes(fn)
    want = [int(h, 16) for h in math_fixture["chunks"][fn]]
    bad = [i for i in range(256) if int(got[i]) != want[i]]
    assert not bad, "%s differs in chunks %s" % (fn, [hex(b) for b in bad[:16]])


@pytest.mark.parametrize("fn", FNS)
def test_edge_inputs_bitwise(fn):
    edge = np.array([0x00000000, 0x80000000, 0x00000001, 0x80000001, 0x007FFFFF, 0x807FFFFF,
                     0x00800000, 0x80800000, 0x3F800000, 0xBF800000, 0x7F7FFFFF, 0xFF7FFFFF,
                     0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00000, 0x7F800001, 0xFFA00000,
                     0x42B00000, 0xC2B00000, 0x42AFFFFF, 0xC2B00001, 0x4B000000, 0x5F000000],
                    dtype=np.uint32).view(np.float32)
    got = M.device_math(fn, edge).view(np.uint32)
    want = O.math_map(fn, edge).view(np.uint32)
    assert np.array_equal(got, want), list(zip(edge.view(np.uint32), got, want))


def test_divide_subnormal_boundary():
    # quotients straddling 2^-126: FTZ decides after rounding on x86
    rng = np.random.default_rng(17)
    n = 1 << 20
    b = rng.uniform(1.0, 2.0, n).astype(np.float32)
    scale = rng.uniform(0.5, 2.0, n).astype(np.float64)
    a = (b.astype(np.float64) * 2.0 ** -126 * scale).astype(np.float32)
    got = M.device_div(a, b).view(np.uint32)
    want = O.div_map(a, b).view(np.uint32)
    assert np.array_equal(got, want)
    x = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    y = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    ok = np.isfinite(x) & np.isfinite(y)
    g = M.device_div(x[ok], y[ok]).view(np.uint32)
    w = O.div_map(x[ok], y[ok]).view(np.uint32)
    nan = np.isnan(w.view(np.float32))
    assert np.array_equal(g[~nan], w[~nan])
    assert np.all(np.isnan(g[nan].view(np.float32)))
