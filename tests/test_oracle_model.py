"""The oracle's forward/decode/witness against the reference C++ driver's
outputs (CIS2_REF digest, argmax digest, tokens, --trace file hash),
recorded in tests/golden/model_fixtures.json by make_model_fixtures.py."""
import hashlib

import pytest

import _oracle as O
from cis2amd import artifacts

FAST = ["tiny-llama", "tiny-untied", "tiny-qwen3", "tiny-qwen2"]


def run(rec, trace=False):
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    m = O.OracleModel(spec, w, max_pos=len(rec["prompt"]) + rec["gen_toks"], threads=8)
    lines = [] if trace else None
    res = m.decode(rec["prompt"], rec["gen_toks"], trace=lines)
    return w, m, res, lines


@pytest.mark.parametrize("name", FAST)
def test_tiny_models_match_reference(name, model_fixtures):
    rec = model_fixtures[name]
    w, m, res, lines = run(rec, trace=True)
    assert w.file_sha256().hex() == rec["weights_sha256"]
    assert m.digests() == (rec["table_digest"], rec["inv_freq_table_digest"])
    assert list(res["ids"]) == rec["tokens"]
    assert res["argmax_digest"] == rec["argmax_digest"]
    assert res["witness"] == rec["witness"]
    assert len(lines) == rec["trace_lines"]
    assert hashlib.sha256(("\n".join(lines) + "\n").encode()).hexdigest() == rec["trace_sha256"]


@pytest.mark.slow
def test_smollm2_short_trace_matches_reference(model_fixtures):
    rec = model_fixtures["smollm2-short"]
    _, _, res, lines = run(rec, trace=True)
    assert res["witness"] == rec["witness"]
    assert hashlib.sha256(("\n".join(lines) + "\n").encode()).hexdigest() == rec["trace_sha256"]


@pytest.mark.slow
def test_smollm2_135m_256_tokens_matches_reference(model_fixtures):
    rec = model_fixtures["smollm2-135m"]
    _, _, res, _ = run(rec)
    assert list(res["ids"]) == rec["tokens"]
    assert res["witness"] == rec["witness"]
