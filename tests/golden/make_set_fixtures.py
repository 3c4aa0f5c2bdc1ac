"""Generate the prompt-set fixtures with the reference driver.

  tests/golden/llama160m_set.json   llama-160m shape, 300 prompts of 8..64
                                    tokens, 128 greedy tokens each
  tests/golden/batch_set.json       SmolLM2-135M shape, 64 sequences with
                                    prompts of 16..512 tokens, 256 greedy
                                    tokens each (the batch-stress sequences)

The seeded synthetic artifacts of the set's model are written once to a
scratch directory; the reference C++ driver compiled from the archive
(oracle/_ref/cis2_host, built by oracle/Makefile) then runs once per prompt,
several prompts in parallel.  Per prompt only its witness digest and argmax
digest (which binds the prompt and generated ids) are recorded; the prompts
themselves are regenerated from the set rule in cis2amd/artifacts.py.

Usage: python tests/golden/make_set_fixtures.py llama|batch [--jobs N] [--limit N]
"""
import argparse
import json
import os
import re
import subprocess
import sys
import tempfile
import time
from concurrent.futures import ThreadPoolExecutor

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "cis2-lab-archive_amd"))
from cis2amd import artifacts  # noqa: E402

REF = os.path.join(ROOT, "oracle", "_ref", "cis2_host")
SETS = {"llama": (artifacts.LLAMA_SET, "llama160m_set.json"),
        "batch": (artifacts.BATCH_SET, "batch_set.json")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("which", choices=sorted(SETS))
    ap.add_argument("--jobs", type=int, default=6)
    ap.add_argument("--limit", type=int, default=0)
    a = ap.parse_args()
    pset, fname = SETS[a.which]
    out = os.path.join(ROOT, "tests", "golden", fname)
    spec = artifacts.SPECS[pset["spec"]]
    prompts = artifacts.set_prompts(pset)
    if a.limit:
        prompts = prompts[:a.limit]
    doc = json.load(open(out)) if os.path.exists(out) else {}
    if doc.get("set") != pset:
        doc = {"set": pset, "cases": {}}
    w = artifacts.Weights(spec, pset["seed"])
    with tempfile.TemporaryDirectory(prefix="cis2set_") as d:
        w.write_dir(d)

        def run(i):
            ids = os.path.join(d, "ids_%d.txt" % i)
            with open(ids, "w") as f:
                f.write("\n".join(str(int(t)) for t in prompts[i]) + "\n")
            r = subprocess.run([REF, "--weights-dir", d, "--ids", ids,
                                "--gen-toks", str(pset["gen_toks"])],
                               capture_output=True, text=True)
            if r.returncode != 0:
                raise RuntimeError("prompt %d failed: %s" % (i, r.stderr[-2000:]))
            wit = re.search(r"CIS2_REF digest=([0-9a-f]{64})", r.stdout).group(1)
            adg = re.search(r"run1_argmax_digest=([0-9a-f]{64})", r.stdout).group(1)
            return i, wit, adg

        todo = [i for i in range(len(prompts)) if str(i) not in doc["cases"]]
        t0 = time.time()
        with ThreadPoolExecutor(a.jobs) as ex:
            for n, (i, wit, adg) in enumerate(ex.map(run, todo)):
                doc["cases"][str(i)] = [wit, adg]
                if n % 8 == 7 or n == len(todo) - 1:
                    with open(out, "w") as f:
                        json.dump(doc, f, indent=1, sort_keys=True)
                    print("%d/%d done, %.0fs" % (n + 1, len(todo), time.time() - t0), flush=True)


if __name__ == "__main__":
    main()
