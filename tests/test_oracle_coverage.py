"""The oracle on the constructed argmax coverage vectors (tests/_coverage.py)
against the reference driver's recorded outputs, the constructions
themselves (exact ties, the -0/+0/subnormal zero step, NaN rows), and the
two mistakes the vectors exist to catch: an argmax with >= (the last
maximum wins) and arithmetic without FTZ/DAZ.  The reference's coverage lab
requires both to move the digest
(labs/w1x-coverage/plans/2026-10-16-w1x-coverage-PLAN.md:7-24)."""
import hashlib

import numpy as np
import pytest

import _coverage as C
import _oracle as O
from conftest import load_golden

FIX = load_golden("coverage_fixture.json")
ORDERS = [("sequential", 0), ("tree", 1)]
ROUTES = ["cov-a", "cov-b", "cov-nan0"]


def weights(name, rec):
    return C.build(C.RECIPES[name], rec.get("tuned"))


def oracle_decode(name, rec, reduction, prompt=None, trace=None):
    recipe = C.RECIPES[name]
    spec = C.SPECS[recipe["spec"]]
    prompt = prompt if prompt is not None else rec["prompt"]
    gen = rec["gen_toks"] if "gen_toks" in rec else recipe["gen_toks"]
    o = O.OracleModel(spec, weights(name, rec), max_pos=len(prompt) + gen, threads=4,
                      reduction=reduction)
    return o.decode(prompt, gen, trace=trace)


@pytest.mark.parametrize("name", ROUTES)
@pytest.mark.parametrize("order,reduction", ORDERS)
def test_oracle_reproduces_reference(name, order, reduction):
    rec = FIX[name][order]
    assert rec["reduction"] == order
    lines = []
    res = oracle_decode(name, rec, reduction, trace=lines)
    assert [int(t) for t in res["ids"]] == rec["tokens"]
    assert res["argmax_digest"] == rec["argmax_digest"]
    assert res["witness"] == rec["witness"]
    assert len(lines) == rec["trace_lines"]
    assert hashlib.sha256(("\n".join(lines) + "\n").encode()).hexdigest() == rec["trace_sha256"]


@pytest.mark.parametrize("order,reduction", ORDERS)
def test_oracle_reproduces_reference_tied(order, reduction):
    for seq in FIX["cov-tied"][order]["sequences"]:
        res = oracle_decode("cov-tied", FIX["cov-tied"][order], reduction, prompt=seq["prompt"])
        assert [int(t) for t in res["ids"]] == seq["tokens"]
        assert res["witness"] == seq["witness"]


@pytest.mark.parametrize("name", ["cov-a", "cov-b"])
@pytest.mark.parametrize("order,reduction", ORDERS)
def test_constructions_hold(name, order, reduction):
    """Every step's maximum is held by more than one row (an exact tie), or
    at the zero step by exactly -0, +0 (subnormal flushed) and +0."""
    rec = FIX[name][order]
    recipe = C.RECIPES[name]
    spec = C.SPECS[recipe["spec"]]
    steps = C.greedy_hidden(spec, weights(name, rec), rec["prompt"], rec["gen_toks"], reduction,
                            threads=4)
    zr = C.zero_rows(recipe)
    groups = {C.winner(e): (e["zero"].values() if isinstance(e, dict) else e[1])
              for e in recipe["route"]}
    for s, (lg, _h, nid) in enumerate(steps):
        bits = lg.view(np.uint32)
        assert nid in groups, (s, nid)
        if s == rec["zero_step"]:
            assert int(bits[zr["neg0"]]) == 0x80000000
            assert int(bits[zr["sub"]]) == 0 and int(bits[zr["pos0"]]) == 0
            finite = lg[~np.isnan(lg)]
            assert finite.max() == 0.0
        elif nid not in zr.values():
            members = groups[nid]
            assert len({int(bits[r]) for r in members}) == 1, (s, members)
            assert (lg[~np.isnan(lg)] == lg[nid]).sum() == len(members)
        for r in recipe["nan_rows"]:
            assert np.isnan(lg[r])


def test_nan_at_index_zero_wins():
    rec = FIX["cov-nan0"]["sequential"]
    assert rec["tokens"][len(rec["prompt"]):] == [0] * rec["gen_toks"]


@pytest.mark.parametrize("name", ["cov-a", "cov-b"])
@pytest.mark.parametrize("order,reduction", ORDERS)
def test_argmax_ge_mutant_moves_the_digest(name, order, reduction):
    rec = FIX[name][order]
    with O.mutation(O.MUT_ARGMAX_GE):
        res = oracle_decode(name, rec, reduction)
    assert res["witness"] != rec["witness"]
    assert [int(t) for t in res["ids"]] != rec["tokens"]
    # the first tie (the route's first group) already goes to its last row
    first_group = C.RECIPES[name]["route"][0]
    assert int(res["ids"][len(rec["prompt"])]) == max(first_group[1])


def test_argmax_ge_mutant_moves_the_tied_digest():
    rec = FIX["cov-tied"]["sequential"]
    seq = rec["sequences"][0]
    with O.mutation(O.MUT_ARGMAX_GE):
        res = oracle_decode("cov-tied", rec, 0, prompt=seq["prompt"])
    assert res["witness"] != seq["witness"]


@pytest.mark.parametrize("name", ["cov-a", "cov-b"])
@pytest.mark.parametrize("order,reduction", ORDERS)
def test_no_ftz_mutant_moves_the_digest(name, order, reduction):
    """Without FTZ/DAZ the subnormal row's logit is the largest at the zero
    step: the token moves, and so does the digest."""
    rec = FIX[name][order]
    zr = C.zero_rows(C.RECIPES[name])
    with O.mutation(O.MUT_NO_FTZ):
        res = oracle_decode(name, rec, reduction)
    assert res["witness"] != rec["witness"]
    n = len(rec["prompt"])
    assert int(res["ids"][n + rec["zero_step"]]) == zr["sub"]
    # and the specified oracle is back
    again = oracle_decode(name, rec, reduction)
    assert again["witness"] == rec["witness"]
