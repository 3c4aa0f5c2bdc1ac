"""Full-size prompt sets on the device, against the reference driver's digests.

  llama-160m: 300 seeded prompts of 8..64 tokens, 128 greedy tokens each
  batch stress (SmolLM2-135M shape): 64 sequences with prompts of 16..512
  tokens, 256 greedy tokens each, decoded as one batch; a smaller batch of
  the same sequences must give the same rows (batch invariance).

The expected witness / argmax digests come from tests/golden/
make_set_fixtures.py (the reference C++ driver, one process per prompt).
"""
import json
import os

import numpy as np
import pytest

from cis2amd import Cis2Model, artifacts

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_set(fname, pset):
    path = os.path.join(GOLDEN, fname)
    if not os.path.exists(path):
        pytest.skip("fixture %s not generated" % fname)
    doc = json.load(open(path))
    assert doc["set"] == pset, "fixture was generated for a different set rule"
    if len(doc["cases"]) < pset["count"]:
        pytest.skip("fixture %s incomplete (%d/%d)" % (fname, len(doc["cases"]), pset["count"]))
    return doc["cases"]


def test_llama160m_300_prompts():
    pset = artifacts.LLAMA_SET
    cases = load_set("llama160m_set.json", pset)
    spec = artifacts.SPECS[pset["spec"]]
    prompts = artifacts.set_prompts(pset)
    m = Cis2Model(spec, artifacts.Weights(spec, pset["seed"]),
                  max_pos=pset["hi"] + pset["gen_toks"])
    bad = []
    for i, p in enumerate(prompts):
        m.reset(0)
        r = m.decode(p, pset["gen_toks"], step_digests=False)
        if [r["witness"], r["argmax_digest"]] != cases[str(i)]:
            bad.append(i)
    assert not bad, "prompts whose digests differ from the reference: %s" % bad[:20]


def test_batch_stress_rows_match_reference_and_smaller_batch():
    pset = artifacts.BATCH_SET
    cases = load_set("batch_set.json", pset)
    spec = artifacts.SPECS[pset["spec"]]
    prompts = artifacts.set_prompts(pset)
    gen = pset["gen_toks"]
    w = artifacts.Weights(spec, pset["seed"])
    m = Cis2Model(spec, w, max_pos=pset["hi"] + gen, max_seqs=len(prompts))
    rows = m.decode_batch(prompts, gen)
    bad = [i for i, r in enumerate(rows) if [r["witness"], r["argmax_digest"]] != cases[str(i)]]
    assert not bad, "rows whose digests differ from the reference: %s" % bad
    small = m.decode_batch(prompts[:8], gen)
    for i in range(8):
        assert small[i]["witness"] == rows[i]["witness"]
        assert small[i]["argmax_digest"] == rows[i]["argmax_digest"]
        assert np.array_equal(small[i]["ids"], rows[i]["ids"])


@pytest.mark.parametrize("B", [1, 32])
def test_batch_stress_b1_b32_match_reference(B):
    """The batch-stress sequences decoded B at a time (B = 1 and B = 32, the
    bench's other batch sizes), every row against the reference driver's
    digests: B = 1 over sequences 0..3 one by one, B = 32 over 32..63."""
    pset = artifacts.BATCH_SET
    cases = load_set("batch_set.json", pset)
    spec = artifacts.SPECS[pset["spec"]]
    prompts = artifacts.set_prompts(pset)
    gen = pset["gen_toks"]
    m = Cis2Model(spec, artifacts.Weights(spec, pset["seed"]), max_pos=pset["hi"] + gen,
                  max_seqs=B)
    first, count = (0, 4) if B == 1 else (32, 32)
    rows = []
    for s in range(first, first + count, B):
        rows += m.decode_batch(prompts[s:s + B], gen)
    bad = [first + i for i, r in enumerate(rows)
           if [r["witness"], r["argmax_digest"]] != cases[str(first + i)]]
    assert not bad, "rows whose digests differ from the reference: %s" % bad
    m.close()


def test_llama160m_300_prompts_as_one_batch():
    """Config 3 as the bench runs it: all 300 llama-160m prompts in one
    cis2_decode_batch call (300 KV-cache slots), every sequence's digests
    equal to the reference driver's."""
    pset = artifacts.LLAMA_SET
    cases = load_set("llama160m_set.json", pset)
    spec = artifacts.SPECS[pset["spec"]]
    prompts = artifacts.set_prompts(pset)
    m = Cis2Model(spec, artifacts.Weights(spec, pset["seed"]),
                  max_pos=pset["hi"] + pset["gen_toks"], max_seqs=len(prompts))
    rows = m.decode_batch(prompts, pset["gen_toks"])
    bad = [i for i, r in enumerate(rows) if [r["witness"], r["argmax_digest"]] != cases[str(i)]]
    assert not bad, "sequences whose digests differ from the reference: %s" % bad[:20]
    m.close()
