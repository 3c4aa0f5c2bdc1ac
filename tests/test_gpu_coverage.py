"""The device greedy argmax on the constructed coverage vectors
(tests/_coverage.py): exact ties in one 32-row block, across blocks and
workgroups, at index 0 and in the ragged last block; a zero step held by
-0, +0 and a flushed subnormal logit; NaN logits at index 0 and beyond.
Every device path that picks a token runs them, in both reduction orders,
against the reference driver's recorded outputs:
  - the persistent decode kernel's LM phase (per-block candidates, the
    last-finisher merge) and the row-batched prefill's argmax (cis2_decode);
  - the per-op argmax (tracing: every op's hash equals the reference trace);
  - the row-batched argmax of the batched decode and of the teacher-forced
    verifier (logits compared bit for bit with the oracle's)."""
import hashlib

import numpy as np
import pytest

import _coverage as C
from cis2amd import Cis2Model
from conftest import load_golden

pytestmark = pytest.mark.gpu

FIX = load_golden("coverage_fixture.json")
ORDERS = [("sequential", 0), ("tree", 1)]
ROUTES = ["cov-a", "cov-b", "cov-nan0"]


def model(name, rec, reduction, max_pos, max_seqs=1):
    recipe = C.RECIPES[name]
    spec = C.SPECS[recipe["spec"]]
    return Cis2Model(spec, C.build(recipe, rec.get("tuned")), max_pos=max_pos, max_seqs=max_seqs,
                     reduction_mode=reduction)


@pytest.mark.parametrize("name", ROUTES)
@pytest.mark.parametrize("order,reduction", ORDERS)
def test_decode_kernel_argmax(name, order, reduction):
    rec = FIX[name][order]
    print("coverage decode", name, order, flush=True)
    m = model(name, rec, reduction, len(rec["prompt"]) + rec["gen_toks"])
    try:
        m.profile(True)
        res = m.decode(rec["prompt"], rec["gen_toks"])
        launches, _ms, positions = m.profile_read()
        m.profile(False)
        assert [int(t) for t in res["ids"]] == rec["tokens"]
        assert res["argmax_digest"] == rec["argmax_digest"]
        assert res["witness"] == rec["witness"]
        # steps 1.. took their logits and argmax from the persistent kernel's
        # LM phase (step 0's are the prefill's); like the reference driver,
        # every step forwards its id, the last one included
        n = len(rec["prompt"])
        assert launches == rec["gen_toks"]
        assert list(positions) == list(range(n, n + rec["gen_toks"]))
    finally:
        m.close()


@pytest.mark.parametrize("name", ROUTES)
@pytest.mark.parametrize("order,reduction", ORDERS)
def test_per_op_argmax_trace(name, order, reduction):
    rec = FIX[name][order]
    print("coverage trace", name, order, flush=True)
    m = model(name, rec, reduction, len(rec["prompt"]) + rec["gen_toks"])
    try:
        res, lines = m.trace(rec["prompt"], rec["gen_toks"])
        assert [int(t) for t in res["ids"]] == rec["tokens"]
        assert res["witness"] == rec["witness"]
        assert len(lines) == rec["trace_lines"]
        assert hashlib.sha256(("\n".join(lines) + "\n").encode()).hexdigest() == \
            rec["trace_sha256"]
    finally:
        m.close()


@pytest.mark.parametrize("name", ROUTES)
@pytest.mark.parametrize("order,reduction", ORDERS)
def test_row_argmax_batch_and_verifier(name, order, reduction):
    rec = FIX[name][order]
    print("coverage rows", name, order, flush=True)
    n = len(rec["prompt"])
    m = model(name, rec, reduction, n + rec["gen_toks"], max_seqs=2)
    try:
        # two copies of the sequence in one batch: both rows take every tie
        rows = m.decode_batch([np.array(rec["prompt"])] * 2, rec["gen_toks"])
        for r in rows:
            assert [int(t) for t in r["ids"]] == rec["tokens"]
            assert r["witness"] == rec["witness"]
            assert r["argmax_digest"] == rec["argmax_digest"]
        v = m.verify_prefill(rec["prompt"], rec["tokens"][n:], want_logits=True)
        assert v["first_mismatch"] == -1
        assert [int(t) for t in v["generated"]] == rec["tokens"][n:]
        assert v["witness"] == rec["witness"]
        # the logits of every step, bit for bit (the zero step's -0 and +0 included)
        recipe = C.RECIPES[name]
        spec = C.SPECS[recipe["spec"]]
        ref = C.greedy_hidden(spec, C.build(recipe, rec.get("tuned")), rec["prompt"],
                              rec["gen_toks"], reduction, threads=4)
        for s, (lg, _h, _nid) in enumerate(ref):
            assert np.array_equal(v["logits"][s].view(np.uint32), lg.view(np.uint32)), s
        if rec.get("zero_step") is not None:
            zr = C.zero_rows(recipe)
            bits = v["logits"][rec["zero_step"]].view(np.uint32)
            assert (int(bits[zr["neg0"]]), int(bits[zr["sub"]]), int(bits[zr["pos0"]])) == \
                (0x80000000, 0, 0)
        # a claim with the first tie broken the other way is caught there
        if name != "cov-nan0":
            bad = list(rec["tokens"][n:])
            first_group = recipe["route"][0][1]
            assert bad[0] == min(first_group)
            bad[0] = max(first_group)
            v2 = m.verify_prefill(rec["prompt"], bad)
            assert v2["first_mismatch"] == 0
    finally:
        m.close()


@pytest.mark.parametrize("order,reduction", ORDERS)
def test_tied_groups(order, reduction):
    rec = FIX["cov-tied"][order]
    print("coverage tied", order, flush=True)
    seqs = rec["sequences"]
    longest = max(len(s["prompt"]) for s in seqs) + rec["gen_toks"]
    m = model("cov-tied", rec, reduction, longest, max_seqs=len(seqs))
    try:
        rows = m.decode_batch([np.array(s["prompt"]) for s in seqs], rec["gen_toks"])
        for r, s in zip(rows, seqs):
            assert [int(t) for t in r["ids"]] == s["tokens"]
            assert r["witness"] == s["witness"]
        for s in seqs:
            res = m.decode(s["prompt"], rec["gen_toks"])
            assert [int(t) for t in res["ids"]] == s["tokens"]
            assert res["witness"] == s["witness"]
    finally:
        m.close()
