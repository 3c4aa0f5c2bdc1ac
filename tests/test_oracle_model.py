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


def _set_cases(fname, pset):
    import json
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", fname)
    if not os.path.exists(path):
        pytest.skip("fixture %s not generated" % fname)
    doc = json.load(open(path))
    assert doc["set"] == pset
    return doc["cases"]


@pytest.mark.slow
def test_llama160m_set_fixture_matches_oracle():
    """The 300-prompt llama-160m fixture is complete and the oracle
    reproduces the reference driver's digests on prompts from it."""
    pset = artifacts.LLAMA_SET
    cases = _set_cases("llama160m_set.json", pset)
    assert sorted(int(k) for k in cases) == list(range(pset["count"]))
    spec = artifacts.SPECS[pset["spec"]]
    prompts = artifacts.set_prompts(pset)
    w = artifacts.Weights(spec, pset["seed"])
    for i in (0, 157):
        m = O.OracleModel(spec, w, max_pos=len(prompts[i]) + pset["gen_toks"], threads=8)
        r = m.decode(prompts[i], pset["gen_toks"])
        assert [r["witness"], r["argmax_digest"]] == cases[str(i)], i


TREE = ["tiny-llama-tree", "tiny-untied-tree", "tiny-qwen3-tree", "tiny-qwen2-tree"]


def run_tree(rec, trace=False):
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    m = O.OracleModel(spec, w, max_pos=len(rec["prompt"]) + rec["gen_toks"], threads=8,
                      reduction=1)
    lines = [] if trace else None
    return m.decode(rec["prompt"], rec["gen_toks"], trace=lines), lines


@pytest.mark.parametrize("name", TREE)
def test_tree_mode_tiny_models_match_reference(name, model_fixtures):
    """The oracle's v0.4 tree order against the reference driver built with
    -DCIS2_REDUCTION_TREE (witness, argmax digest, tokens, --trace hash)."""
    rec = model_fixtures[name]
    assert rec["reduction"] == "tree"
    res, lines = run_tree(rec, trace=True)
    assert list(res["ids"]) == rec["tokens"]
    assert res["argmax_digest"] == rec["argmax_digest"]
    assert res["witness"] == rec["witness"]
    assert hashlib.sha256(("\n".join(lines) + "\n").encode()).hexdigest() == rec["trace_sha256"]


@pytest.mark.slow
@pytest.mark.parametrize("name", ["tiny-wide-tree", "smollm2-135m-tree"])
def test_tree_mode_models_match_reference(name, model_fixtures):
    rec = model_fixtures[name]
    res, _ = run_tree(rec)
    assert list(res["ids"]) == rec["tokens"]
    assert res["witness"] == rec["witness"]


def _layer_digest_lines(lines, pos):
    """LAYER_DIGEST lines (the reference CLI's --layer-digests, main.rs:382-384,
    496-501, 509-514, 525-527) of the pass at `pos`, from its trace lines."""
    t = {}
    for line in lines:
        p, layer, op, sha = line.split()
        if int(p.split("=")[1]) == pos:
            t[(int(layer.split("=")[1]), op.split("=")[1])] = sha.split("=")[1]
    n = len([k for k in t if k[1] == "resid2"])
    return (["LAYER_DIGEST embed %s" % t[(-1, "embedding")]] +
            ["LAYER_DIGEST block_%d %s" % (i, t[(i, "resid2")]) for i in range(n)] +
            ["LAYER_DIGEST final_norm %s" % t[(-1, "final_norm")],
             "LAYER_DIGEST logits %s" % t[(-1, "logits")]])


@pytest.mark.parametrize("name", FAST + ["tiny-qwen3-tree"])
def test_layer_digests_match_reference_trace(name, model_fixtures):
    """The per-layer digests of the last prompt position (each block's output
    = the trace's resid2 line) computed by the oracle equal the ones read
    from the reference driver's own trace (layer_digests, recorded by
    make_model_fixtures.py); the GPU CLI's --layer-digests lines are checked
    against the same fixture."""
    rec = model_fixtures[name]
    if rec.get("reduction") == "tree":
        _, lines = run_tree(rec, trace=True)
    else:
        _, _, _, lines = run(rec, trace=True)
    got = _layer_digest_lines(lines, len(rec["prompt"]) - 1)
    assert got == rec["layer_digests"]
    assert len(got) == artifacts.SPECS[rec["spec"]].n_layers + 3
