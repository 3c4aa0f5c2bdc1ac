"""Device strict-order GEMV against the rust-5 published output hashes, the
oracle, and edge shapes."""
import hashlib

import numpy as np
import pytest

import _oracle as O
import rust5data
from cis2amd import GemvPlan, artifacts

pytestmark = pytest.mark.gpu


def test_rust5_all_published_hashes(rust5):
    for st, (M, K), W, x in rust5data.sets():
        y = GemvPlan(W)(x)
        assert hashlib.sha256(y.tobytes()).hexdigest() == rust5["y_sha256"]["%dx%d" % (M, K)][str(st)], (st, M, K)


def test_config1_gemv_matches_oracle():
    # W 1536x576 ~N(0,0.02) fp32, x 576 ~N(0,1), seeded
    W = artifacts.gen_f32(20261201, 1, 1536 * 576, 0.02).reshape(1536, 576)
    x = artifacts.gen_f32(20261201, 2, 576, 1.0)
    plan = GemvPlan(W, copies=3)
    y = plan(x)
    assert np.array_equal(y.view(np.uint32), O.gemv(W, x).view(np.uint32))


@pytest.mark.parametrize("M,K", [(1, 4), (63, 8), (65, 12), (100, 576), (576, 1536), (4096, 4)])
def test_edge_shapes_match_oracle(M, K):
    rng = np.random.default_rng(M * 131 + K)
    W = rng.standard_normal((M, K)).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    assert np.array_equal(GemvPlan(W)(x).view(np.uint32), O.gemv(W, x).view(np.uint32))


@pytest.mark.parametrize("M,K", [(49152, 576), (8193, 100), (8208, 576)])
def test_many_block_gemv_matches_oracle(M, K):
    """Matrices of more than 512 row blocks (the LM head of the SmolLM2 shape,
    49152x576) run on the streaming kernel: same bits as the oracle, on every
    replica."""
    W = artifacts.gen_f32(20261202, M, M * K, 0.02).reshape(M, K)
    x = artifacts.gen_f32(20261202, K, K, 1.0)
    plan = GemvPlan(W, copies=2)
    ref = O.gemv(W, x).view(np.uint32)
    assert np.array_equal(plan(x).view(np.uint32), ref)
    plan.time(3)  # both replicas used
    assert np.array_equal(plan(x).view(np.uint32), ref)


def test_cancellation_order_survives_on_device():
    W = np.array([[1e8, 1.0, -1e8, 0.0], [1e8, -1e8, 1.0, 0.0]], np.float32)
    y = GemvPlan(W)(np.ones(4, np.float32))
    assert list(y) == [0.0, 1.0]


def test_subnormal_products_flush():
    # products below 2^-126 flush to zero, as under MXCSR FTZ
    W = np.full((64, 4), 2.0 ** -70, np.float32)
    x = np.full(4, 2.0 ** -70, np.float32)
    y = GemvPlan(W)(x)
    assert np.array_equal(y.view(np.uint32), O.gemv(W, x).view(np.uint32))
    assert np.all(y == 0.0)


@pytest.mark.parametrize("M,K,n", [(1536, 576, 7), (100, 576, 3), (65, 12, 5), (576, 1536, 2)])
def test_batched_gemvs_equal_single_and_oracle(M, K, n):
    """n GEMVs in one launch (replicas rotating) give each GEMV's own bits."""
    rng = np.random.default_rng(M * 7 + K + n)
    W = rng.standard_normal((M, K)).astype(np.float32)
    X = rng.standard_normal((n, K)).astype(np.float32)
    plan = GemvPlan(W, copies=3)
    Y = plan.run_batch(X)
    for i in range(n):
        assert np.array_equal(Y[i].view(np.uint32), plan(X[i]).view(np.uint32)), i
        assert np.array_equal(Y[i].view(np.uint32), O.gemv(W, X[i]).view(np.uint32)), i
    plan.close()
