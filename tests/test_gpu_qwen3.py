"""Qwen3-0.6B shape at full context on the device: a 4096-token prompt and
256 greedy tokens (positions 0..4351, QK-norm, 16 query / 8 KV heads of 128)
against the reference driver's run of the same synthetic weights and prompt
(cis2_host_qwen3; tests/golden/make_model_fixtures.py, case qwen3-0.6b-4096).

  - bs=1 decode: the prompt prefilled in one row-batched pass, then one
    persistent-kernel launch per token; witness, argmax digest and tokens;
  - the teacher-forced verifier (cis2_verify_prefill) over all 4351 rows in
    one pass reproduces the same witness.
"""
import json
import os

import numpy as np
import pytest

from cis2amd import Cis2Model, artifacts

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qwen3_fixture.json")
CASE = "qwen3-0.6b-4096"


@pytest.fixture(scope="module")
def rec():
    return json.load(open(GOLDEN))[CASE]


def test_fixture_prompt_is_the_seeded_prompt(rec):
    """The fixture's prompt is the generator's (seed 6, 4096 ids), and its
    token list is prompt ++ generated."""
    spec = artifacts.SPECS[rec["spec"]]
    p = artifacts.prompt_ids(rec["seed"], spec.vocab, 4096)
    assert [int(t) for t in p] == rec["prompt"]
    assert rec["tokens"][:4096] == rec["prompt"]
    assert len(rec["tokens"]) == 4096 + rec["gen_toks"]


@pytest.fixture(scope="module")
def model(rec):
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    return Cis2Model(spec, w, max_pos=4096 + rec["gen_toks"])


@pytest.mark.gpu
def test_qwen3_4096_prompt_256_tokens_decode(rec, model):
    r = model.decode(rec["prompt"], rec["gen_toks"], step_digests=False)
    assert r["witness"] == rec["witness"]
    assert r["argmax_digest"] == rec["argmax_digest"]
    assert [int(t) for t in r["ids"]] == rec["tokens"]


@pytest.mark.gpu
def test_qwen3_4096_verify_prefill(rec, model):
    claimed = rec["tokens"][4096:]
    r = model.verify_prefill(rec["prompt"], claimed)
    assert r["first_mismatch"] == -1
    assert r["witness"] == rec["witness"]
    assert r["argmax_digest"] == rec["argmax_digest"]
    assert np.array_equal(np.asarray(r["generated"], dtype=np.uint32),
                          np.asarray(claimed, dtype=np.uint32))


@pytest.mark.gpu
def test_qwen3_second_prompt_and_back(rec, model):
    """Decodes of two different 4096-token prompts in turn on one context
    (each position's K/V rows, scores and tagged words overwritten with the
    other prompt's values in between): the fixture prompt reproduces the
    reference witness after the other prompt's decode, and the other
    prompt's decode equals the teacher-forced verifier over its own
    generated tokens (an independent path: the row-batched kernels)."""
    spec = artifacts.SPECS[rec["spec"]]
    other = [int(t) for t in artifacts.prompt_ids(rec["seed"] + 1, spec.vocab, 4096)]
    assert other != rec["prompt"]
    for _ in range(2):
        rb = model.decode(other, rec["gen_toks"], step_digests=False)
        gen = [int(t) for t in rb["ids"]][4096:]
        vb = model.verify_prefill(other, gen)
        assert vb["first_mismatch"] == -1
        assert rb["witness"] == vb["witness"]
        assert rb["argmax_digest"] == vb["argmax_digest"]
        ra = model.decode(rec["prompt"], rec["gen_toks"], step_digests=False)
        assert ra["witness"] == rec["witness"]
        assert ra["argmax_digest"] == rec["argmax_digest"]
