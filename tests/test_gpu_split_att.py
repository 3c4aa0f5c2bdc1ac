"""Split attention in the persistent decode kernel: the ATT phase as score
tasks (256 positions of all query heads of one kv head each, the K columns
copied into an LDS tile) and mix tasks (8 output dims each: softmax, then
the V-mix chain over V tiles streamed into LDS).  It is chosen when a head's K/V rows do not fit one
workgroup (Qwen3 at 4352 positions, the 1200-position tree case);
CIS2_ATT=split forces it and CIS2_ATT=one forbids it, so both attention
forms run every fixture and must reproduce the reference's witnesses.
"""
import os

import pytest

from cis2amd import Cis2Model, artifacts

pytestmark = pytest.mark.gpu


def build(rec, att):
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    mode = 1 if rec.get("reduction") == "tree" else 0
    os.environ["CIS2_ATT"] = att
    try:
        return Cis2Model(spec, w, max_pos=len(rec["prompt"]) + rec["gen_toks"],
                         reduction_mode=mode)
    finally:
        del os.environ["CIS2_ATT"]


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen3", "tiny-qwen2", "tiny-qwen3-tree",
                                  "tiny-untied-tree", "smollm2-135m", "smollm2-135m-tree",
                                  "llama-160m-p0"])
def test_split_attention_forced_matches_reference(name, model_fixtures):
    rec = model_fixtures[name]
    m = build(rec, "split")
    r = m.decode(rec["prompt"], rec["gen_toks"])
    assert list(r["ids"]) == rec["tokens"]
    assert r["witness"] == rec["witness"]
    assert r["argmax_digest"] == rec["argmax_digest"]


def test_one_task_attention_forced_on_long_context(model_fixtures):
    """The 1200-position tree case on the one-task-per-head streamed path."""
    rec = model_fixtures["tiny-wide-tree"]
    m = build(rec, "one")
    r = m.decode(rec["prompt"], rec["gen_toks"], step_digests=False)
    assert list(r["ids"]) == rec["tokens"]
    assert r["witness"] == rec["witness"]


def test_split_and_one_task_step_digests_agree(model_fixtures):
    """Per-step logit digests of both forms on the SmolLM2 shape."""
    rec = model_fixtures["smollm2-135m"]
    a = build(rec, "split").decode(rec["prompt"], 64)
    b = build(rec, "one").decode(rec["prompt"], 64)
    assert a["step_digests"] == b["step_digests"]
    assert a["witness"] == b["witness"]


@pytest.mark.parametrize("n_heads,n_kv,mode", [(6, 2, 0), (6, 2, 1), (10, 2, 0)])
def test_split_score_groups_match_one_task(n_heads, n_kv, mode):
    """Score tasks cover all query heads of a kv head (pairs of heads, then
    a lone head for odd groups) with Qwen3's per-head QK-norm: both forms
    give the same per-step logits for groups of 3 and 5."""
    import numpy as np
    spec = artifacts.ModelSpec(f"tiny-g{n_heads // n_kv}", 96, 128, 2, n_heads, n_kv, 300, 1e-6,
                               1000000.0, True, head_dim=32, qk_norm=True)
    w = artifacts.Weights(spec, 7)
    prompt = np.arange(1, 20, dtype=np.uint32)
    out = []
    for att in ("split", "one"):
        os.environ["CIS2_ATT"] = att
        try:
            m = Cis2Model(spec, w, max_pos=64, reduction_mode=mode)
        finally:
            del os.environ["CIS2_ATT"]
        out.append(m.decode(prompt, 40))
    assert list(out[0]["ids"]) == list(out[1]["ids"])
    assert out[0]["step_digests"] == out[1]["step_digests"]
