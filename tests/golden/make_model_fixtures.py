"""Generate tests/golden/model_fixtures.json with the reference driver.

For each case this writes the seeded synthetic artifacts (model.safetensors,
config.json, tokenizer.json) and the --ids file to a scratch directory, runs
the reference C++ driver compiled from the archive (oracle/_ref/cis2_host,
cis2_host_qwen3 for QK-norm models; built by oracle/Makefile), and records
what it prints: the CIS2_REF witness digest, the argmax digest, the token
list, the table / inv_freq digests, and the sha256 of its --trace file.
Only these small results are committed; the artifacts are regenerated from
their seeds wherever a test needs them.

Usage: python tests/golden/make_model_fixtures.py [case ...] [--jobs N] [--out FILE]
"""
import argparse
import hashlib
import json
import os
import re
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "cis2-lab-archive_amd"))
from cis2amd import artifacts  # noqa: E402

OUT = os.path.join(ROOT, "tests", "golden", "model_fixtures.json")
REF = os.path.join(ROOT, "oracle", "_ref")

# name: (spec, seed, prompt_len or list, gen_toks, trace[, tree reduction])
CASES = {
    "tiny-llama": ("tiny-llama", 1, 5, 12, True),
    "tiny-untied": ("tiny-untied", 2, 7, 10, True),
    "tiny-qwen3": ("tiny-qwen3", 3, 6, 10, True),
    "tiny-qwen2": ("tiny-qwen2", 4, 4, 8, True),
    "smollm2-short": ("smollm2-135m", 20261201, 8, 8, True),
    "smollm2-135m": ("smollm2-135m", 20261201, 32, 256, False),
    "llama-160m-p0": ("llama-160m", 160, ("llama", 0), 128, False),
    "llama-160m-p1": ("llama-160m", 160, ("llama", 1), 128, False),
    "llama-160m-p2": ("llama-160m", 160, ("llama", 2), 128, False),
    # Qwen3-0.6B shape: 4096-token prompt, 256 generated tokens (positions 0..4351)
    "qwen3-0.6b-4096": ("qwen3-0.6b", 6, 4096, 256, False),
    # v0.4 tree reduction order (reference built with -DCIS2_REDUCTION_TREE)
    "tiny-llama-tree": ("tiny-llama", 1, 5, 12, True, True),
    "tiny-untied-tree": ("tiny-untied", 2, 7, 10, True, True),
    "tiny-qwen3-tree": ("tiny-qwen3", 3, 6, 10, True, True),
    "tiny-qwen2-tree": ("tiny-qwen2", 4, 4, 8, True, True),
    "tiny-wide-tree": ("tiny-wide", 77, 1180, 20, False, True),
    "smollm2-135m-tree": ("smollm2-135m", 20261201, 32, 256, False, True),
}


def llama_prompt(seed, idx, vocab):
    """Prompt idx of the llama-160m set: length U[8,64], ids U[0,vocab)."""
    n = int(artifacts.gen_uniform(seed, (1 << 41) + idx, 8, 64, 1)[0])
    return artifacts.gen_uniform(seed, (1 << 42) + idx, 0, vocab - 1, n)


def case_prompt(spec, seed, p):
    if isinstance(p, tuple):
        return [int(t) for t in llama_prompt(seed, p[1], spec.vocab)]
    return [int(t) for t in artifacts.prompt_ids(seed, spec.vocab, p)]


def run_case(name):
    spec_name, seed, p, gen, trace = CASES[name][:5]
    tree = len(CASES[name]) > 5 and CASES[name][5]
    spec = artifacts.SPECS[spec_name]
    prompt = case_prompt(spec, seed, p)
    w = artifacts.Weights(spec, seed)
    binary = os.path.join(REF, ("cis2_host_qwen3" if spec.qk_norm or spec.head_dim else "cis2_host")
                          + ("_tree" if tree else ""))
    with tempfile.TemporaryDirectory(prefix="cis2fx_") as d:
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
            raise RuntimeError("%s failed: %s" % (name, r.stderr[-2000:]))
        out = r.stdout
        rec = {"spec": spec_name, "seed": seed, "prompt": prompt, "gen_toks": gen,
               "reference_binary": os.path.basename(binary),
               "reduction": re.search(r"reduction_mode=(\w+)", out).group(1)}
        for key in ["weights_sha256", "tokenizer_sha256", "config_sha256", "table_digest",
                    "inv_freq_table_digest"]:
            rec[key] = re.search(key + r"=([0-9a-f]{64})", out).group(1)
        rec["witness"] = re.search(r"CIS2_REF digest=([0-9a-f]{64})", out).group(1)
        rec["argmax_digest"] = re.search(r"run1_argmax_digest=([0-9a-f]{64})", out).group(1)
        toks = re.search(r"run1_tokens=\[([0-9, ]*)\]", out).group(1)
        rec["tokens"] = [int(t) for t in toks.split(",")]
        if trace:
            data = open(tpath, "rb").read()
            rec["trace_sha256"] = hashlib.sha256(data).hexdigest()
            rec["trace_lines"] = data.count(b"\n")
            rec["layer_digests"] = layer_digest_lines(data.decode(), len(prompt) - 1)
        return name, rec


def layer_digest_lines(trace_text, pos):
    """The LAYER_DIGEST lines the reference CLI's --layer-digests prints for
    the forward pass at `pos` (code/cis2-fp/src/main.rs:382-384, 496-501,
    509-514, 525-527), from the same pass's trace lines: the embedding, each
    block's output (resid2), the final norm, the logits."""
    t = {}
    for line in trace_text.splitlines():
        m = re.match(r"pos=(-?\d+) layer=(-?\d+) op=(\S+) sha256=([0-9a-f]{64})$", line)
        if m and int(m.group(1)) == pos:
            t[(int(m.group(2)), m.group(3))] = m.group(4)
    out = ["LAYER_DIGEST embed %s" % t[(-1, "embedding")]]
    n_layers = len([k for k in t if k[1] == "resid2"])
    out += ["LAYER_DIGEST block_%d %s" % (li, t[(li, "resid2")]) for li in range(n_layers)]
    out += ["LAYER_DIGEST final_norm %s" % t[(-1, "final_norm")],
            "LAYER_DIGEST logits %s" % t[(-1, "logits")]]
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("cases", nargs="*")
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--out", default=OUT)
    a = ap.parse_args()
    names = a.cases or list(CASES)
    out = a.out
    doc = json.load(open(out)) if os.path.exists(out) else {}
    with ThreadPoolExecutor(a.jobs) as ex:
        for name, rec in ex.map(run_case, names):
            doc[name] = rec
            print(name, rec["witness"], flush=True)
            with open(out, "w") as f:
                json.dump(doc, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
