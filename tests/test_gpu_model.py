"""The device forward pass / greedy decode / witness against the reference
driver's recorded outputs and the oracle, plus the error paths of the ABI."""
import hashlib

import numpy as np
import pytest

import _oracle as O
from cis2amd import Cis2Error, Cis2Model, artifacts

pytestmark = pytest.mark.gpu

TINY = ["tiny-llama", "tiny-untied", "tiny-qwen3", "tiny-qwen2"]
# the same cases in the v0.4-candidate tree order (reference built with
# -DCIS2_REDUCTION_TREE)
TINY_TREE = [n + "-tree" for n in TINY]


def build(rec, max_seqs=1, extra_pos=0):
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    mode = 1 if rec.get("reduction") == "tree" else 0
    return Cis2Model(spec, w, max_pos=len(rec["prompt"]) + rec["gen_toks"] + extra_pos,
                     max_seqs=max_seqs, reduction_mode=mode), w


@pytest.mark.parametrize("name", TINY + TINY_TREE)
def test_tiny_decode_and_trace_match_reference(name, model_fixtures):
    rec = model_fixtures[name]
    m, _ = build(rec)
    assert tuple(d.hex() for d in m.digests()) == (rec["table_digest"], rec["inv_freq_table_digest"])
    res, lines = m.trace(rec["prompt"], rec["gen_toks"])
    assert list(res["ids"]) == rec["tokens"]
    assert res["argmax_digest"] == rec["argmax_digest"]
    assert res["witness"] == rec["witness"]
    assert len(lines) == rec["trace_lines"]
    assert hashlib.sha256(("\n".join(lines) + "\n").encode()).hexdigest() == rec["trace_sha256"]
    # the fast path (no trace) gives the same bits
    fast = m.decode(rec["prompt"], rec["gen_toks"])
    assert fast["witness"] == rec["witness"]


@pytest.mark.parametrize("name", TINY + TINY_TREE)
def test_tiny_step_digests_match_oracle(name, model_fixtures):
    rec = model_fixtures[name]
    m, w = build(rec)
    spec = artifacts.SPECS[rec["spec"]]
    o = O.OracleModel(spec, w, max_pos=len(rec["prompt"]) + rec["gen_toks"],
                      reduction=m.reduction_mode)
    a = m.decode(rec["prompt"], rec["gen_toks"])
    b = o.decode(rec["prompt"], rec["gen_toks"])
    assert a["step_digests"] == b["step_digests"]


def test_smollm2_short_trace_matches_reference(model_fixtures):
    rec = model_fixtures["smollm2-short"]
    m, _ = build(rec)
    res, lines = m.trace(rec["prompt"], rec["gen_toks"])
    assert res["witness"] == rec["witness"]
    assert hashlib.sha256(("\n".join(lines) + "\n").encode()).hexdigest() == rec["trace_sha256"]


def test_smollm2_135m_32_prompt_256_tokens(model_fixtures):
    # the headline workload: every one of the 256 folded logit vectors
    # enters the witness, so one digest pins all of them
    rec = model_fixtures["smollm2-135m"]
    m, _ = build(rec)
    res = m.decode(rec["prompt"], rec["gen_toks"])
    assert list(res["ids"]) == rec["tokens"]
    assert res["argmax_digest"] == rec["argmax_digest"]
    assert res["witness"] == rec["witness"]
    # determinism (spec §12.4: two runs in one process agree)
    again = m.decode(rec["prompt"], rec["gen_toks"])
    assert again["witness"] == res["witness"] and again["step_digests"] == res["step_digests"]


@pytest.mark.parametrize("name", ["llama-160m-p0", "llama-160m-p1", "llama-160m-p2"])
def test_llama160m_prompts(name, model_fixtures):
    if name not in model_fixtures:
        pytest.skip("fixture not generated")
    rec = model_fixtures[name]
    m, _ = build(rec)
    res = m.decode(rec["prompt"], rec["gen_toks"])
    assert list(res["ids"]) == rec["tokens"]
    assert res["witness"] == rec["witness"]


def test_forward_logits_bitwise_vs_oracle(model_fixtures):
    rec = model_fixtures["tiny-untied"]
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    m = Cis2Model(spec, w, max_pos=16)
    o = O.OracleModel(spec, w, max_pos=16)
    toks = [3, 17, 250, 0, 299]
    for p, t in enumerate(toks):
        lg, am = m.forward_token(p, t)
        ref = np.empty(spec.vocab, np.float32)
        O.lib().orc_forward(o.m, p, t, O.ptr(ref, O.c_fp), O.TRACE_FN(), None)
        assert np.array_equal(lg.view(np.uint32), ref.view(np.uint32)), p
        assert am == O.lib().orc_argmax(O.ptr(ref, O.c_fp), spec.vocab)


def test_batch_rows_equal_solo_runs(model_fixtures):
    rec = model_fixtures["tiny-llama"]
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    prompts = [artifacts.gen_uniform(9, 100 + i, 0, spec.vocab - 1, n) for i, n in
               enumerate([16, 3, 40, 7, 25])]
    gen = 12
    m = Cis2Model(spec, w, max_pos=64, max_seqs=3)
    rows = m.decode_batch(prompts, gen)
    solo = Cis2Model(spec, w, max_pos=64, max_seqs=1)
    o = O.OracleModel(spec, w, max_pos=64)
    for p, r in zip(prompts, rows):
        s = solo.decode(p, gen)
        c = o.decode(p, gen)
        assert r["witness"] == s["witness"] == c["witness"]
        assert list(r["ids"]) == list(s["ids"]) == list(c["ids"])


def test_error_paths(model_fixtures):
    rec = model_fixtures["tiny-llama"]
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    m = Cis2Model(spec, w, max_pos=8)
    with pytest.raises(Cis2Error) as e:
        m.forward_token(0, spec.vocab)
    assert e.value.code == -9
    with pytest.raises(Cis2Error) as e:
        m.forward_token(8, 1)
    assert e.value.code == -9
    with pytest.raises(Cis2Error) as e:
        m.decode([1, 2, 3], 6)
    assert e.value.code == -9
    # missing tensor / wrong count / unknown name
    w2 = artifacts.Weights(spec, rec["seed"])
    w2.tensors = [t for t in w2.tensors if t[0] != "model.norm.weight"]
    with pytest.raises(Cis2Error) as e:
        Cis2Model(spec, w2, max_pos=8)
    assert e.value.code == -3
    w3 = artifacts.Weights(spec, rec["seed"])
    n, s, a = w3.tensors[1]
    w3.tensors[1] = (n, s, a[:-1])
    with pytest.raises(Cis2Error) as e:
        Cis2Model(spec, w3, max_pos=8)
    assert e.value.code == -4
    w4 = artifacts.Weights(spec, rec["seed"])
    w4.tensors.insert(0, ("model.layers.99.mlp.up_proj.weight", (1,), np.zeros(1, np.uint16)))
    with pytest.raises(Cis2Error) as e:
        Cis2Model(spec, w4, max_pos=8)
    assert e.value.code == -5
    # reduction orders other than sequential (0) and tree (1)
    with pytest.raises(Cis2Error) as e:
        Cis2Model(spec, w, max_pos=8, reduction_mode=2)
    assert e.value.code == -2


def test_long_context_streamed_attention_matches_oracle():
    """Positions whose cached K/V no longer fit in LDS take the streamed
    attention path (tiles of 288 positions at head_dim 128); every step's
    logits digest and the witness must equal the oracle's."""
    spec = artifacts.SPECS["tiny-wide"]
    w = artifacts.Weights(spec, 77)
    prompt = artifacts.prompt_ids(77, spec.vocab, 1180)
    gen = 20
    m = Cis2Model(spec, w, max_pos=len(prompt) + gen)
    r = m.decode(prompt, gen)
    o = O.OracleModel(spec, w, max_pos=len(prompt) + gen, threads=8)
    ro = o.decode(prompt, gen)
    assert r["step_digests"] == ro["step_digests"]
    assert r["witness"] == ro["witness"]
    assert list(r["ids"]) == list(ro["ids"])


def test_tree_mode_smollm2_135m_32_prompt_256_tokens(model_fixtures):
    """The headline shape in the tree order: persistent kernel with tree
    GEMVs, tree RMSNorm sums, tree scores and softmax denominators."""
    rec = model_fixtures["smollm2-135m-tree"]
    assert rec["reduction"] == "tree"
    m, _ = build(rec)
    r = m.decode(rec["prompt"], rec["gen_toks"], step_digests=False)
    assert list(r["ids"]) == rec["tokens"]
    assert r["argmax_digest"] == rec["argmax_digest"]
    assert r["witness"] == rec["witness"]


def test_tree_mode_long_context_streamed_attention(model_fixtures):
    """Tree order on the streamed-attention path (1180 prompt positions at
    head_dim 128): the reference's witness for the same run."""
    rec = model_fixtures["tiny-wide-tree"]
    m, _ = build(rec)
    r = m.decode(rec["prompt"], rec["gen_toks"], step_digests=False)
    assert list(r["ids"]) == rec["tokens"]
    assert r["witness"] == rec["witness"]
