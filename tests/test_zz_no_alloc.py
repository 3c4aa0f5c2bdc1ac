"""The no-allocation draw (cis2_sample_logits_noalloc) against the
allocating one (cis2_sample_logits) on the same logit rows: device-resident
inputs and outputs, the sampler's scratch in the library's static per-GPU
array.  Two calls in a row, the second with a smaller input (fewer rows and
a smaller vocabulary), so stale scratch contents from the first call would
show; then the error paths (NaN logit, vocabulary above the scratch
maximum, sampling off)."""
import ctypes

import numpy as np
import pytest

from cis2amd import Cis2Error, Cis2Model, _lib, artifacts
from cis2amd._lib import check

pytestmark = pytest.mark.gpu

_hip = None


def hip():
    """hipMalloc / hipMemcpy / hipFree of the HIP runtime, for the test's own
    device buffers (the library under test allocates nothing here)."""
    global _hip
    if _hip is None:
        h = ctypes.CDLL("libamdhip64.so")
        h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        h.hipFree.argtypes = [ctypes.c_void_p]
        h.hipDeviceSynchronize.argtypes = []
        _hip = h
    return _hip


H2D, D2H = 1, 2


class DevBuf:
    def __init__(self, nbytes):
        self.p = ctypes.c_void_p()
        assert hip().hipMalloc(ctypes.byref(self.p), max(nbytes, 4)) == 0
        self.n = nbytes

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.n
        assert hip().hipMemcpy(self.p, arr.ctypes.data, arr.nbytes, H2D) == 0

    def get(self, dtype, count):
        out = np.empty(count, dtype=dtype)
        assert hip().hipMemcpy(out.ctypes.data, self.p, out.nbytes, D2H) == 0
        return out

    def free(self):
        if self.p:
            hip().hipFree(self.p)
            self.p = ctypes.c_void_p()


def tiny_with_vocab(V):
    return artifacts.ModelSpec("tiny-v%d" % V, 64, 128, 1, 4, 2, V, 1e-5, 10000.0, True)


def logit_rows(rng, V, n):
    out = []
    for t in range(n):
        if t % 3 == 0:
            lg = rng.standard_normal(V).astype(np.float32)
        elif t % 3 == 1:  # ties and signed zeros
            lg = rng.integers(-3, 4, V).astype(np.float32) * np.float32(0.25)
            lg[rng.random(V) < 0.2] = np.float32(-0.0)
        else:  # near-flat: top-p keeps most of the vocabulary
            lg = (rng.standard_normal(V) * 0.01).astype(np.float32)
        out.append(lg)
    return np.stack(out)


def draw_noalloc(m, rows, steps, with_nkeep=True):
    n, V = rows.shape
    L = _lib.lib()
    dl, di, dk = DevBuf(rows.nbytes), DevBuf(4 * n), DevBuf(4 * n)
    try:
        dl.put(rows)
        st = np.ascontiguousarray(steps, dtype=np.uint32)
        check(L.cis2_sample_logits_noalloc(m.ctx, dl.p, n, st.ctypes.data_as(_lib.c_u32p), di.p,
                                           dk.p if with_nkeep else None), m.ctx)
        return di.get(np.uint32, n), (dk.get(np.uint32, n) if with_nkeep else None)
    finally:
        for b in (dl, di, dk):
            b.free()


# (V, rows, T, top_k, top_p): the second call is smaller in rows and vocabulary
CALLS = [
    (49152, 5, 0.8, 40, 0.95),
    (4097, 2, 0.8, 0, 0.95),
]


def test_noalloc_equals_allocating_draw():
    rng = np.random.default_rng(2026)
    models = {}
    try:
        for V, n, T, k, p in CALLS:
            spec = tiny_with_vocab(V)
            m = models.setdefault(V, Cis2Model(spec, artifacts.Weights(spec, 5), max_pos=8))
            rows = logit_rows(rng, V, n)
            steps = [int(x) for x in rng.integers(0, 2**32, n)]
            for params in [(T, k, p), (1.0, 0, 1.0), (0.5, 1, 1.0), (1.3, 0, 1e-6)]:
                seed = int(rng.integers(0, 2**63))
                m.set_sampling(seed, *params)
                want_ids, want_nk = m.sample_logits(rows, steps)
                got_ids, got_nk = draw_noalloc(m, rows, steps)
                assert list(got_ids) == [int(x) for x in want_ids], (V, n, params)
                assert list(got_nk) == [int(x) for x in want_nk], (V, n, params)
                ids_only, _ = draw_noalloc(m, rows, steps, with_nkeep=False)
                assert list(ids_only) == list(got_ids)
    finally:
        for m in models.values():
            m.close()


def test_noalloc_error_paths():
    spec = tiny_with_vocab(256)
    m = Cis2Model(spec, artifacts.Weights(spec, 5), max_pos=8)
    try:
        rows = logit_rows(np.random.default_rng(1), 256, 2)
        with pytest.raises(Cis2Error) as e:  # sampling not enabled
            draw_noalloc(m, rows, [0, 1])
        assert e.value.code == -1
        m.set_sampling(7, 1.0, 0, 1.0)
        bad = rows.copy()
        bad[1, 17] = np.float32("nan")
        with pytest.raises(Cis2Error) as e:
            draw_noalloc(m, bad, [0, 1])
        assert e.value.code == -10
        # the flag was cleared: the next clean call succeeds and matches
        ids, _ = draw_noalloc(m, rows, [3, 4])
        want, _ = m.sample_logits(rows, [3, 4])
        assert list(ids) == [int(x) for x in want]
    finally:
        m.close()
    big = tiny_with_vocab(262145)
    mb = Cis2Model(big, artifacts.Weights(big, 5), max_pos=4)
    try:
        mb.set_sampling(7, 1.0, 0, 1.0)
        rows = np.zeros((1, 262145), dtype=np.float32)
        with pytest.raises(Cis2Error) as e:
            draw_noalloc(mb, rows, [0])
        assert e.value.code == -1
    finally:
        mb.close()


def test_noalloc_two_threads_take_turns():
    """Two contexts on one GPU, each driven by its own host thread, draw
    through the shared scratch at the same time; the per-GPU lock makes them
    take turns, so every draw equals its context's allocating draw."""
    import threading

    rng = np.random.default_rng(99)
    jobs = []
    for V, seed in ((49152, 11), (30000, 12)):
        spec = tiny_with_vocab(V)
        m = Cis2Model(spec, artifacts.Weights(spec, 5), max_pos=8)
        m.set_sampling(seed, 0.8, 40, 0.95)
        rows = logit_rows(rng, V, 3)
        steps = [int(x) for x in rng.integers(0, 2**32, 3)]
        jobs.append((m, rows, steps, m.sample_logits(rows, steps)))
    errors = []

    def worker(m, rows, steps, want):
        try:
            for _ in range(20):
                ids, nk = draw_noalloc(m, rows, steps)
                assert list(ids) == [int(x) for x in want[0]]
                assert list(nk) == [int(x) for x in want[1]]
        except BaseException as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=j) for j in jobs]
    try:
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=120)
        assert not any(t.is_alive() for t in threads), "a drawing thread did not finish"
        assert not errors, errors[0]
    finally:
        for m, *_ in jobs:
            m.close()
