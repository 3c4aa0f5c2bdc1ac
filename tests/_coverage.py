"""Constructed coverage vectors for the greedy argmax: exact ties, +0/-0
ties, a subnormal logit, NaN logits (test infrastructure).

The reference's coverage lab builds one tiny Llama model whose lm_head rows
5 and 17 are equal (the step-0 logits tie, strict > picks 5) and whose row
29 gives a subnormal logit that FTZ flushes
(labs/w1x-coverage/plans/2026-10-16-w1x-coverage-PLAN.md:7-24; the scan it
pins is code/cis2-fp/src/main.rs:1161-1169, spec section 11.2).  Its bytes
are not archived, so this module builds its own family from the seeded
generator, shaped to reach every place a device argmax merges candidates:

- untied models: a *route* of tie groups.  Every embedding row carries 8.0
  on one coordinate; the final-norm output is then dominated by that
  coordinate, and the tie group owning it (identical lm_head rows with 2.0
  there) takes the maximum logit by a wide margin.  The group's lowest row
  wins under strict >; its embedding routes the next step to the next
  group's coordinate.  Groups sit in one 32-row block, in adjacent blocks,
  in blocks 256 apart (one workgroup of the persistent kernel), at index 0,
  at the last row, three-way.
- one *zero step* per route: every other row carries -2.0 on its
  coordinate, so the maximum logit is zero and is held by three rows: an
  all-zero row (+0), a row whose one product is a positive subnormal
  (flushed to 0 under FTZ; the largest logit without it), and a row whose
  two products cancel to a negative subnormal (flushed to -0).  The last two
  are tuned against the oracle's final-norm output at that step, once per
  reduction order (make_coverage_fixture.py records the tuned values).
- NaN rows: one NaN weight makes that row's logit NaN at every step (never
  chosen), or, at row 0, the argmax of every step (the scan starts with
  best = logits[0] and nothing compares greater than NaN).
- a tied model: group members share one embedding row with 8.0 on the
  group's coordinate; a prompt ending in a member keeps choosing the
  group's lowest row.
"""
import numpy as np

from cis2amd import artifacts

BF16_ONE = 0x3F80
BF16_EIGHT = 0x4100
BF16_TWO = 0x4000
BF16_MINUS_TWO = 0xC000
BF16_NAN = 0x7FC0

# Llama architecture at the lab's size (hidden 64, head_dim 32, 2 layers,
# inter 128), GQA 2:1, a vocabulary of 20,011 rows: 626 LM-head blocks of
# 32 rows, the last one ragged (11 rows).
SPECS = {
    "cov-untied": artifacts.ModelSpec("cov-untied", 64, 128, 2, 2, 1, 20011, 1e-5, 10000.0,
                                      False),
    "cov-tied": artifacts.ModelSpec("cov-tied", 64, 128, 2, 2, 1, 20011, 1e-5, 10000.0, True),
}

# Tie groups (coordinate, rows).  The lowest row of each wins.
G_SAME_BLOCK = (3, [5, 17])             # one 32-row block, one wave
G_INDEX0 = (7, [0, 12000])              # the scan's starting index
G_ADJ_BLOCKS = (11, [40, 70])           # blocks 1 and 2: two workgroups
G_SAME_WG = (13, [300, 8492])           # blocks 9 and 265: one workgroup, 256 blocks apart
G_THREE_LAST = (17, [19000, 19999, 20010])  # three-way, the last (ragged) block
G_ADJ_ROWS = (19, [7777, 7778])


def zero_entry(coord, order):
    """A zero step on `coord`; order: row indices for 'neg0', 'sub', 'pos0'."""
    return {"coord": coord, "zero": dict(order)}


# name -> the recipe before tuning (route order, NaN rows, prompt, steps)
RECIPES = {
    # zero step: -0 row first, then the subnormal row, then +0
    "cov-a": {"spec": "cov-untied", "seed": 20261016,
              "route": [G_SAME_BLOCK, G_INDEX0, G_ADJ_BLOCKS,
                        zero_entry(23, {"neg0": 1234, "sub": 1300, "pos0": 2222}),
                        G_SAME_WG, G_THREE_LAST, G_ADJ_ROWS],
              "nan_rows": [555, 19998], "prompt": [101, 9999, 4242, 31], "gen_toks": 24},
    # zero step: +0 row first, then -0, then the subnormal row
    "cov-b": {"spec": "cov-untied", "seed": 20261017,
              "route": [G_ADJ_ROWS, G_THREE_LAST,
                        zero_entry(29, {"pos0": 1000, "neg0": 1010, "sub": 1020}),
                        G_INDEX0, G_SAME_BLOCK, G_SAME_WG, G_ADJ_BLOCKS],
              "nan_rows": [33], "prompt": [202, 15001, 6], "gen_toks": 24},
    # NaN at row 0: every step picks 0
    "cov-nan0": {"spec": "cov-untied", "seed": 20261018,
                 "route": [G_SAME_BLOCK, G_ADJ_BLOCKS, G_THREE_LAST],
                 "nan_rows": [0, 777], "prompt": [9, 10, 11], "gen_toks": 8},
    # tied: identical embedding rows per group; one prompt per group, ending
    # in a member that is not the lowest
    "cov-tied": {"spec": "cov-tied", "seed": 20261019,
                 "groups": [G_SAME_BLOCK, G_INDEX0, G_ADJ_BLOCKS, G_SAME_WG, G_THREE_LAST,
                            G_ADJ_ROWS],
                 "prompts": [[100, 17], [101, 102, 12000], [70], [55, 8492],
                             [3, 20010], [19999, 7778]],
                 "gen_toks": 6},
}


def _rows(t, V, H):
    return t.reshape(V, H)


def _tensor(w, name):
    for n, _shape, arr in w.tensors:
        if n == name:
            return arr
    raise KeyError(name)


def winner(entry):
    if isinstance(entry, dict):
        return min(entry["zero"].values())
    return min(entry[1])


def coord(entry):
    return entry["coord"] if isinstance(entry, dict) else entry[0]


def build(recipe, tuned=None):
    """The recipe's weights (artifacts.Weights with the constructed rows).
    tuned: {'neg0': [[k, bf16], ...], 'sub': [[k, bf16]]} for the zero step's
    two tuned rows (None: both all-zero, the untuned first pass)."""
    spec = SPECS[recipe["spec"]]
    H, V = spec.hidden, spec.vocab
    w = artifacts.Weights(spec, recipe["seed"])
    for name, _shape, arr in w.tensors:
        if name.endswith("layernorm.weight") or name == "model.norm.weight":
            arr[:] = BF16_ONE
    E = _rows(_tensor(w, "model.embed_tokens.weight"), V, H)
    if spec.tied:
        for c, rows in recipe["groups"]:
            rows = sorted(rows)
            E[rows[0], c] = BF16_EIGHT
            for r in rows[1:]:
                E[r] = E[rows[0]]
        return w
    route = recipe["route"]
    c0 = coord(route[0])
    E[:, c0] = BF16_EIGHT
    for i, e in enumerate(route):
        nxt = coord(route[(i + 1) % len(route)])
        win = winner(e)
        if nxt != c0:
            E[win, c0] = 0
            E[win, nxt] = BF16_EIGHT
    L = _rows(_tensor(w, "lm_head.weight"), V, H)
    for e in route:
        if isinstance(e, dict):
            L[:, e["coord"]] = BF16_MINUS_TWO
    for e in route:
        if isinstance(e, dict):
            continue
        c, rows = e
        rows = sorted(rows)
        L[rows[0], c] = BF16_TWO
        for r in rows[1:]:
            L[r] = L[rows[0]]
    for e in route:
        if not isinstance(e, dict):
            continue
        z = e["zero"]
        for key in ("pos0", "sub", "neg0"):
            L[z[key]] = 0
        if tuned:
            for key in ("sub", "neg0"):
                for k, bits in tuned[key]:
                    L[z[key], k] = bits
    for r in recipe.get("nan_rows", []):
        L[r, 0] = BF16_NAN
    return w


def zero_rows(recipe):
    for e in recipe.get("route", []):
        if isinstance(e, dict):
            return e["zero"]
    return None


def greedy_hidden(spec, w, prompt, gen_toks, reduction, threads=8):
    """Oracle greedy decode, position by position, keeping the final-norm
    output behind every step's logits: [(logits, hidden, argmax)]."""
    import _oracle as O
    o = O.OracleModel(spec, w, max_pos=len(prompt) + gen_toks, threads=threads,
                      reduction=reduction)
    out = []
    lg = None
    for p, t in enumerate(prompt):
        lg = o.forward(p, t)
    for s in range(gen_toks):
        hid = o.hidden()
        nid = int(O.lib().orc_argmax(O.ptr(lg, O.c_fp), spec.vocab))
        out.append((lg.copy(), hid, nid))
        if s + 1 < gen_toks:
            lg = o.forward(len(prompt) + s, nid)
    return out
