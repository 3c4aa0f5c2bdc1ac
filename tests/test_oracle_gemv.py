"""The oracle's strict-order GEMV, pinned against the 25 output hashes the
rust-5 lab published (labs/rust-5/reports/rust-5/box1/gate.out) and against
brute force."""
import hashlib

import numpy as np
import pytest

import _oracle as O
import rust5data


@pytest.mark.slow
def test_rust5_input_file_reconstruction(rust5):
    assert rust5data.file_sha256() == rust5["data_sha256"]


def test_rust5_all_published_hashes(rust5):
    n = 0
    for st, (M, K), W, x in rust5data.sets():
        y = O.gemv(W, x)
        assert hashlib.sha256(y.tobytes()).hexdigest() == rust5["y_sha256"]["%dx%d" % (M, K)][str(st)]
        n += 1
    assert n == 25


def test_gemv_brute_force_small():
    rng = np.random.default_rng(1)
    for M, K in [(1, 1), (3, 5), (17, 33), (70, 12)]:
        W = rng.standard_normal((M, K)).astype(np.float32)
        x = rng.standard_normal(K).astype(np.float32)
        want = np.zeros(M, np.float32)
        for r in range(M):
            acc = np.float32(0.0)
            for k in range(K):
                acc = np.float32(acc + np.float32(W[r, k] * x[k]))
            want[r] = acc
        assert np.array_equal(O.gemv(W, x).view(np.uint32), want.view(np.uint32))


def test_gemv_thread_count_does_not_change_bits():
    rng = np.random.default_rng(2)
    W = rng.standard_normal((300, 96)).astype(np.float32)
    x = rng.standard_normal(96).astype(np.float32)
    a = O.gemv(W, x, threads=1)
    b = O.gemv(W, x, threads=7)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_gemv_is_order_sensitive():
    # a reordered sum gives different bits: the pin is real
    W = np.array([[1e8, 1.0, -1e8]], np.float32)
    assert O.gemv(W, np.ones(3, np.float32))[0] == 0.0
    assert O.gemv(W[:, ::-1].copy(), np.ones(3, np.float32))[0] == 0.0
    W2 = np.array([[1.0, 1e8, -1e8]], np.float32)
    assert O.gemv(W2, np.ones(3, np.float32))[0] == 0.0
    W3 = np.array([[1e8, -1e8, 1.0]], np.float32)
    assert O.gemv(W3, np.ones(3, np.float32))[0] == 1.0
