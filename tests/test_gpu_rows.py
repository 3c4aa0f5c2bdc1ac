"""The row-batched forward pass on the device: many rows per launch (a batch
of sequences, or every position of one sequence) must give each row the
bits of its single-row run and of the reference.

  - cis2_forward with n > 1 rows (causal prefill of one sequence through the
    KV cache) against the single-row calls and the oracle;
  - cis2_verify_prefill (teacher-forced, verify3/model.c:923-1005): an
    honest claim reproduces the reference decode's witness and argmax
    digest; a claim tampered at step k reports first_mismatch == k
    (verify3/prefilltest.c:84-160);
  - cis2_decode_batch with ragged prompts equals the bs=1 decodes.
"""
import os

import numpy as np
import pytest

import _oracle as O
from cis2amd import Cis2Error, Cis2Model, artifacts

pytestmark = pytest.mark.gpu

TINY = ["tiny-llama", "tiny-untied", "tiny-qwen3", "tiny-qwen2"]


def model_for(rec, max_seqs=1, extra_pos=0):
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    mode = 1 if rec.get("reduction") == "tree" else 0
    return Cis2Model(spec, w, max_pos=len(rec["prompt"]) + rec["gen_toks"] + extra_pos,
                     max_seqs=max_seqs, reduction_mode=mode), w


@pytest.mark.parametrize("name", TINY + [n + "-tree" for n in TINY])
def test_rows_prefill_equals_single_rows_and_oracle(name, model_fixtures):
    rec = model_fixtures[name]
    m, w = model_for(rec)
    spec = m.spec
    seq = rec["prompt"] + rec["tokens"][len(rec["prompt"]):]  # prompt ++ generated
    n = len(seq)
    rows_logits, rows_arg = m.forward_rows(np.zeros(n), np.arange(n), seq)
    m.reset(0)
    for p in range(n):
        lg, am = m.forward_token(p, seq[p])
        assert np.array_equal(lg.view(np.uint32), rows_logits[p].view(np.uint32)), "row %d" % p
        assert am == rows_arg[p]
    o = O.OracleModel(spec, w, max_pos=n, reduction=m.reduction_mode)
    for p in range(n):
        ol = o.forward(p, seq[p])
        assert np.array_equal(ol.view(np.uint32), rows_logits[p].view(np.uint32)), "oracle row %d" % p


def test_rows_rows_of_two_sequences_in_any_order(model_fixtures):
    """Rows of two sequences interleaved and out of position order in one
    call: each sequence's rows equal its own prefill."""
    rec = model_fixtures["tiny-llama"]
    m, _ = model_for(rec, max_seqs=2, extra_pos=8)
    a = rec["prompt"]
    b = [int(t) for t in artifacts.prompt_ids(99, m.spec.vocab, 9)]
    la, _ = m.forward_rows(np.zeros(len(a)), np.arange(len(a)), a)
    lb, _ = m.forward_rows(np.zeros(len(b)), np.arange(len(b)), b)
    rows = [(0, p, a[p]) for p in range(len(a))] + [(1, p, b[p]) for p in range(len(b))]
    rng = np.random.default_rng(5)
    order = rng.permutation(len(rows))
    rs = np.array([rows[i] for i in order], dtype=np.uint32)
    lm, _ = m.forward_rows(rs[:, 0], rs[:, 1], rs[:, 2])
    for j, i in enumerate(order):
        s, p, _ = rows[i]
        ref = la[p] if s == 0 else lb[p]
        assert np.array_equal(lm[j].view(np.uint32), ref.view(np.uint32))


def test_rows_duplicate_row_is_refused(model_fixtures):
    rec = model_fixtures["tiny-llama"]
    m, _ = model_for(rec)
    with pytest.raises(Cis2Error) as e:
        m.forward_rows([0, 0], [1, 1], [3, 4])
    assert e.value.code == -1


@pytest.mark.parametrize("name", ["smollm2-135m", "llama-160m-p0", "tiny-qwen3", "tiny-wide-tree",
                                  "smollm2-135m-tree"])
def test_verify_prefill_honest_claim_reproduces_reference_witness(name, model_fixtures):
    rec = model_fixtures[name]
    m, _ = model_for(rec)
    n = len(rec["prompt"])
    claimed = rec["tokens"][n:]
    r = m.verify_prefill(rec["prompt"], claimed)
    assert r["first_mismatch"] == -1
    assert list(r["generated"]) == claimed
    assert r["witness"] == rec["witness"]
    assert r["argmax_digest"] == rec["argmax_digest"]


def test_verify_prefill_tampered_claim_reports_first_mismatch(model_fixtures):
    rec = model_fixtures["smollm2-135m"]
    m, _ = model_for(rec)
    n = len(rec["prompt"])
    claimed = list(rec["tokens"][n:])
    for k in (0, 17, 200, len(claimed) - 1):
        bad = list(claimed)
        bad[k] = (bad[k] + 1) % m.spec.vocab
        r = m.verify_prefill(rec["prompt"], bad)
        assert r["first_mismatch"] == k
        # positions before the tamper see the honest prefix
        assert list(r["generated"][:k + 1]) == claimed[:k + 1]
        assert r["witness"] != rec["witness"] or k == len(claimed) - 1


def test_decode_prefill_paths_agree(model_fixtures):
    """The decode's prefill runs as one row-batched pass; the position by
    position prefill (CIS2_PREFILL=seq) gives the same witness."""
    rec = model_fixtures["tiny-qwen3"]
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    os.environ["CIS2_PREFILL"] = "seq"
    try:
        ms = Cis2Model(spec, w, max_pos=len(rec["prompt"]) + rec["gen_toks"])
    finally:
        del os.environ["CIS2_PREFILL"]
    mr = Cis2Model(spec, w, max_pos=len(rec["prompt"]) + rec["gen_toks"])
    a = ms.decode(rec["prompt"], rec["gen_toks"])
    b = mr.decode(rec["prompt"], rec["gen_toks"])
    assert a["witness"] == b["witness"] == rec["witness"]
    assert a["step_digests"] == b["step_digests"]


@pytest.mark.parametrize("graph,mode", [("1", 0), ("0", 0), ("1", 1)])
@pytest.mark.parametrize("B", [2, 5])
def test_decode_batch_ragged_equals_bs1(B, graph, mode):
    """B sequences with ragged prompts through cis2_decode_batch (row-batched
    prefill and steps) against each sequence's bs=1 decode.  The steps run
    as two alternating captured graphs, replayed 23 times between host
    folds (graph "1"), or op by op (CIS2_GRAPH=0); mode 1 is tree mode."""
    spec = artifacts.SPECS["tiny-untied"]
    w = artifacts.Weights(spec, 2)
    prompts = [artifacts.set_prompt(2, i, spec.vocab, 1, 40, 9) for i in range(B)]
    gen = 24
    m = Cis2Model(spec, w, max_pos=40 + gen, max_seqs=3, reduction_mode=mode)  # B=5: two groups
    os.environ["CIS2_GRAPH"] = graph
    try:
        rows = m.decode_batch(prompts, gen)
    finally:
        del os.environ["CIS2_GRAPH"]
    solo = Cis2Model(spec, w, max_pos=40 + gen, reduction_mode=mode)
    for i, p in enumerate(prompts):
        s = solo.decode(p, gen, step_digests=False)
        assert rows[i]["witness"] == s["witness"]
        assert rows[i]["argmax_digest"] == s["argmax_digest"]
        assert np.array_equal(rows[i]["ids"], s["ids"])


@pytest.mark.parametrize("cap", ["", "64"])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("name", ["smollm2-4l", "tiny-wide"])
def test_decode_batch_kv_head_attention(name, mode, cap):
    """Decode rows of head_dim 64 and 128 attend one workgroup per (row, KV
    head), the V rows staged in LDS in chunks; CIS2_ATT_KV=64 caps a chunk
    at 64 positions, so the rows of up to 200 + 12 positions run through the
    two-buffer ring.  Each row equals its bs=1 decode and the run with one
    head per workgroup (CIS2_ATT_KV=0)."""
    spec = artifacts.SPECS[name]
    w = artifacts.Weights(spec, 7)
    prompts = [artifacts.set_prompt(7, i, spec.vocab, 1, 200, 11) for i in range(3)]
    gen = 12
    m = Cis2Model(spec, w, max_pos=200 + gen, max_seqs=3, reduction_mode=mode)
    rows = _with_env("CIS2_ATT_KV", cap, lambda: m.decode_batch(prompts, gen)) if cap else \
        m.decode_batch(prompts, gen)
    old = _with_env("CIS2_ATT_KV", "0", lambda: m.decode_batch(prompts, gen))
    solo = Cis2Model(spec, w, max_pos=200 + gen, reduction_mode=mode)
    for i, p in enumerate(prompts):
        s = solo.decode(p, gen, step_digests=False)
        assert rows[i]["witness"] == s["witness"] == old[i]["witness"], i
        assert rows[i]["argmax_digest"] == s["argmax_digest"], i
        assert np.array_equal(rows[i]["ids"], s["ids"]), i


@pytest.mark.parametrize("name", ["smollm2-135m", "smollm2-135m-tree"])
def test_rows_many_rows_gqa_grouped_attention(name, model_fixtures):
    """Enough rows that the attention groups the query heads of one KV head
    in a workgroup and the norms run as their own pass: two sequences of
    the fixture's 288 positions (576 rows, 3 KV heads) against the
    single-row forward of every position."""
    rec = model_fixtures[name]
    m, w = model_for(rec, max_seqs=2)
    seq = rec["prompt"] + rec["tokens"][len(rec["prompt"]):]
    n = len(seq)
    seqs = np.concatenate([np.zeros(n), np.ones(n)])
    lg, am = m.forward_rows(seqs, np.concatenate([np.arange(n)] * 2), seq + seq)
    m.reset(0)
    for p in range(n):
        sl, sa = m.forward_token(p, seq[p])
        for base in (0, n):
            assert np.array_equal(sl.view(np.uint32), lg[base + p].view(np.uint32)), "row %d" % p
            assert sa == am[base + p]
    # the argmax at the last prompt row is the fixture's first generated id
    assert am[len(rec["prompt"]) - 1] == rec["tokens"][len(rec["prompt"])]


@pytest.mark.parametrize("gen", [1, 2, 3])
def test_decode_batch_short_generations(gen):
    """gen = 1 (the prefill's logits only), 2 (one captured step, replayed
    once) and 3 (both alternating graphs): each row equals its bs=1 run."""
    spec = artifacts.SPECS["tiny-qwen3"]
    w = artifacts.Weights(spec, 3)
    prompts = [artifacts.set_prompt(3, i, spec.vocab, 1, 12, 9) for i in range(3)]
    m = Cis2Model(spec, w, max_pos=12 + gen, max_seqs=3)
    rows = m.decode_batch(prompts, gen)
    solo = Cis2Model(spec, w, max_pos=12 + gen)
    for i, p in enumerate(prompts):
        s = solo.decode(p, gen, step_digests=False)
        assert rows[i]["witness"] == s["witness"], i
        assert np.array_equal(rows[i]["ids"], s["ids"]), i


def test_decode_batch_one_token_prompts():
    """Prompts of a single token (the prefill is one row per sequence)."""
    spec = artifacts.SPECS["tiny-llama"]
    w = artifacts.Weights(spec, 1)
    prompts = [[5], [17], [5]]
    m = Cis2Model(spec, w, max_pos=1 + 16, max_seqs=3)
    rows = m.decode_batch(prompts, 16)
    solo = Cis2Model(spec, w, max_pos=1 + 16)
    for i, p in enumerate(prompts):
        s = solo.decode(p, 16, step_digests=False)
        assert rows[i]["witness"] == s["witness"], i
    assert rows[0]["witness"] == rows[2]["witness"]  # same prompt, same row


def _with_env(key, val, fn):
    old = os.environ.get(key)
    os.environ[key] = val
    try:
        return fn()
    finally:
        if old is None:
            del os.environ[key]
        else:
            os.environ[key] = old


@pytest.mark.parametrize("name", ["smollm2-135m", "llama-160m-p0"])
def test_verify_prefill_tiled_attention(name, model_fixtures):
    """The prefill's attention in tiles of up to 16 consecutive rows (forced
    on for these row counts): the reference's witness, and logits bitwise
    equal to the per-row attention's."""
    rec = model_fixtures[name]
    m, _ = model_for(rec)
    n = len(rec["prompt"])
    claimed = rec["tokens"][n:]
    rt = _with_env("CIS2_ATT_TILES", "1", lambda: m.verify_prefill(rec["prompt"], claimed,
                                                                   want_logits=True))
    rr = _with_env("CIS2_ATT_TILES", "0", lambda: m.verify_prefill(rec["prompt"], claimed,
                                                                   want_logits=True))
    assert rt["first_mismatch"] == -1
    assert rt["witness"] == rec["witness"]
    assert np.array_equal(rt["logits"].view(np.uint32), rr["logits"].view(np.uint32))


@pytest.mark.parametrize("shuffle", [False, True])
def test_rows_tiled_attention_two_sequences(shuffle, model_fixtures):
    """Rows of two sequences (runs of consecutive positions, or shuffled
    into runs of one) through the tiled attention equal the per-row
    attention's logits bit for bit."""
    rec = model_fixtures["smollm2-135m"]
    m, _ = model_for(rec, max_seqs=2, extra_pos=0)
    a = rec["prompt"] + rec["tokens"][len(rec["prompt"]):len(rec["prompt"]) + 40]
    b = [int(t) for t in artifacts.prompt_ids(7, m.spec.vocab, 53)]
    rows = [(0, p, a[p]) for p in range(len(a))] + [(1, p, b[p]) for p in range(len(b))]
    if shuffle:
        order = np.random.default_rng(11).permutation(len(rows))
        rows = [rows[i] for i in order]
    rs = np.array(rows, dtype=np.uint32)

    def run():
        m.reset(0)
        m.reset(1)
        return m.forward_rows(rs[:, 0], rs[:, 1], rs[:, 2])

    lt, at = _with_env("CIS2_ATT_TILES", "1", run)
    lr, ar = _with_env("CIS2_ATT_TILES", "0", run)
    assert np.array_equal(lt.view(np.uint32), lr.view(np.uint32))
    assert np.array_equal(at, ar)
