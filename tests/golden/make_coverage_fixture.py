"""Generate tests/golden/coverage_fixture.json: the constructed coverage
vectors of tests/_coverage.py, tuned against the oracle and recorded with
the reference driver.

Per recipe and reduction order (sequential, tree):
 1. untuned pass: the route's zero-step rows are all zero; the oracle's
    greedy decode gives the final-norm output h behind the first step whose
    argmax lands on a zero-step row;
 2. tuning on that h: the subnormal row gets one weight s = +-2^-126 on a
    coordinate k with |h_k| < 1 (s * h_k is a positive subnormal); the -0 row
    gets a on a coordinate i < 32 and b on coordinate 63 with
    fl(a h_i) + fl(b h_63) a negative subnormal (FTZ gives -0 in either
    order: the sequential fold and the tree fold both reduce the row to that
    one add), checked with the oracle's own dot products;
 3. tuned pass: the oracle confirms the zero step (logit bits of the three
    rows: -0, +0, +0) and that the route up to it is unchanged;
 4. the reference driver (oracle/_ref/cis2_host, cis2_host_tree: the
    archive's gpu/cis2_host.cpp built here) runs the tuned artifacts with
    --trace; its CIS2_REF digest, argmax digest, tokens and trace hash are
    recorded with the tuned values.

Usage: python tests/golden/make_coverage_fixture.py [recipe ...]
"""
import hashlib
import json
import os
import re
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "cis2-lab-archive_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import _coverage as C  # noqa: E402
import _oracle as O  # noqa: E402

OUT = os.path.join(ROOT, "tests", "golden", "coverage_fixture.json")
REF = os.path.join(ROOT, "oracle", "_ref")
TWO_M126 = 2.0 ** -126


def f32bits(x):
    return int(np.float32(x).view(np.uint32))


def bf16_value(bits):
    return np.uint32(bits << 16).view(np.float32)


def dot_bits(row_bits, h, reduction):
    w = np.array([bf16_value(int(b)) for b in row_bits], dtype=np.float32)
    fn = O.lib().orc_dot_tree if reduction else O.lib().orc_dot_seq
    return f32bits(fn(O.ptr(w, O.c_fp), O.ptr(np.ascontiguousarray(h), O.c_fp), len(h)))


def tune(h, cz, reduction):
    """(tuned dict) for the zero step whose final-norm output is h."""
    H = len(h)
    assert cz != H - 1
    # subnormal row: one product +-2^-126 * h_k, a positive subnormal
    for k in range(1, H - 1):
        if k == cz or not (2.0 ** -20 < abs(float(h[k])) < 0.9):
            continue
        s_bits = 0x0080 | (0x8000 if h[k] < 0 else 0)
        prod = float(bf16_value(s_bits)) * float(h[k])
        assert 2.0 ** -149 < prod < TWO_M126
        sub = [[k, s_bits]]
        break
    else:
        raise RuntimeError("no coordinate for the subnormal row")
    # -0 row: fl(a h_i) + fl(b h_63) in (-2^-126, 0)
    j = H - 1
    hj = np.float32(h[j])
    for i in range(0, 32):
        if i in (cz, sub[0][0]) or abs(float(h[i])) < 2.0 ** -20:
            continue
        hi = np.float32(h[i])
        for e in range(-118, -108):
            a_bits = (0x8000 if hi < 0 else 0) | ((e + 127) << 7)  # +-2^e, sign of h_i
            p = np.float32(bf16_value(a_bits)) * hi                  # > 0, exact (power of two)
            target = -float(p) / float(hj)                         # b with b h_63 = -p
            eb = int(np.floor(np.log2(abs(target))))
            for ee in (eb - 1, eb, eb + 1):
                for mant in range(128):
                    b_bits = (0x8000 if target < 0 else 0) | ((ee + 127) << 7) | mant
                    q = np.float32(bf16_value(b_bits)) * hj
                    r = float(p) + float(q)
                    if -TWO_M126 < r < 0.0:
                        row = [0] * H
                        row[i], row[j] = a_bits, b_bits
                        assert dot_bits(row, h, reduction) == 0x80000000
                        srow = [0] * H
                        srow[sub[0][0]] = sub[0][1]
                        assert dot_bits(srow, h, reduction) == 0
                        return {"sub": sub, "neg0": [[i, a_bits], [j, b_bits]]}
    raise RuntimeError("no (a, b) pair gives a negative subnormal")


def run_ref(spec, w, prompt, gen, reduction, trace=True):
    binary = os.path.join(REF, "cis2_host" + ("_tree" if reduction else ""))
    with tempfile.TemporaryDirectory(prefix="cis2cov_") as d:
        w.write_dir(d)
        ids = os.path.join(d, "ids.txt")
        with open(ids, "w") as f:
            f.write("\n".join(str(t) for t in prompt) + "\n")
        cmd = [binary, "--weights-dir", d, "--ids", ids, "--gen-toks", str(gen)]
        tpath = os.path.join(d, "trace.txt")
        if trace:
            cmd += ["--trace", tpath]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError("reference driver failed: " + r.stderr[-2000:])
        out = r.stdout
        rec = {"witness": re.search(r"CIS2_REF digest=([0-9a-f]{64})", out).group(1),
               "argmax_digest": re.search(r"run1_argmax_digest=([0-9a-f]{64})", out).group(1),
               "tokens": [int(t) for t in
                          re.search(r"run1_tokens=\[([0-9, ]*)\]", out).group(1).split(",")],
               "weights_sha256": re.search(r"weights_sha256=([0-9a-f]{64})", out).group(1),
               "reduction": re.search(r"reduction_mode=(\w+)", out).group(1)}
        if trace:
            data = open(tpath, "rb").read()
            rec["trace_sha256"] = hashlib.sha256(data).hexdigest()
            rec["trace_lines"] = data.count(b"\n")
        return rec


def make_route(name, reduction):
    recipe = C.RECIPES[name]
    spec = C.SPECS[recipe["spec"]]
    prompt, gen = recipe["prompt"], recipe["gen_toks"]
    zr = C.zero_rows(recipe)
    tuned, zstep = None, None
    if zr:
        cz = [e["coord"] for e in recipe["route"] if isinstance(e, dict)][0]
        first = C.greedy_hidden(spec, C.build(recipe), prompt, gen, reduction)
        zstep = next(s for s, (_, _, nid) in enumerate(first) if nid in zr.values())
        tuned = tune(first[zstep][1], cz, reduction)
        second = C.greedy_hidden(spec, C.build(recipe, tuned), prompt, gen, reduction)
        lg = second[zstep][0].view(np.uint32)
        assert int(lg[zr["neg0"]]) == 0x80000000 and int(lg[zr["sub"]]) == 0 and \
            int(lg[zr["pos0"]]) == 0, "zero step not as constructed"
        assert [x[2] for x in first[:zstep + 1]] == [x[2] for x in second[:zstep + 1]]
    w = C.build(recipe, tuned)
    rec = run_ref(spec, w, prompt, gen, reduction)
    rec.update({"prompt": prompt, "gen_toks": gen, "tuned": tuned, "zero_step": zstep})
    return rec


def make_tied(name, reduction):
    recipe = C.RECIPES[name]
    spec = C.SPECS[recipe["spec"]]
    w = C.build(recipe)
    out = []
    for p in recipe["prompts"]:
        r = run_ref(spec, w, p, recipe["gen_toks"], reduction, trace=False)
        r["prompt"] = p
        out.append(r)
    return {"gen_toks": recipe["gen_toks"], "sequences": out}


def main():
    names = sys.argv[1:] or list(C.RECIPES)
    doc = json.load(open(OUT)) if os.path.exists(OUT) else {}
    for name in names:
        doc[name] = {}
        for reduction, key in ((0, "sequential"), (1, "tree")):
            if "route" in C.RECIPES[name]:
                rec = make_route(name, reduction)
            else:
                rec = make_tied(name, reduction)
            doc[name][key] = rec
            print(name, key, rec.get("witness", ""), rec.get("tokens", ""), flush=True)
    with open(OUT, "w") as f:
        json.dump(doc, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
