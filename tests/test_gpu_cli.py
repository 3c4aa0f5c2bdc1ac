"""The cis2_host CLI prints the reference driver's line protocol and writes a
byte-identical --trace file (gpu/Makefile:160-184 gate: digest equality and
`cmp` of the traces)."""
import hashlib
import os
import re
import subprocess

import pytest

from cis2amd import artifacts

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "cis2-lab-archive_amd", "bin", "cis2_host")


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen3", "tiny-untied", "tiny-qwen3-tree"])
def test_cli_matches_reference_lines_and_trace(name, model_fixtures, tmp_path):
    rec = model_fixtures[name]
    w = artifacts.Weights(artifacts.SPECS[rec["spec"]], rec["seed"])
    w.write_dir(str(tmp_path))
    ids = tmp_path / "ids.txt"
    ids.write_text("\n".join(str(t) for t in rec["prompt"]) + "\n")
    trace = tmp_path / "trace.txt"
    mode = rec.get("reduction", "sequential")
    r = subprocess.run([CLI, "--weights-dir", str(tmp_path), "--ids", str(ids), "--gen-toks",
                        str(rec["gen_toks"]), "--trace", str(trace), "--reduction", mode],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    out = r.stdout
    assert re.search(r"^CIS2_REF digest=%s prompt_idx=0 prompt_toks=%d gen_toks=%d dtype=fp32 "
                     r"reduction_mode=%s$" % (rec["witness"], len(rec["prompt"]),
                                              rec["gen_toks"], mode), out, re.M)
    assert "run1_argmax_digest=%s" % rec["argmax_digest"] in out
    assert "table_digest=%s" % rec["table_digest"] in out
    assert "inv_freq_table_digest=%s" % rec["inv_freq_table_digest"] in out
    assert "weights_sha256=%s" % rec["weights_sha256"] in out
    assert hashlib.sha256(trace.read_bytes()).hexdigest() == rec["trace_sha256"]


def test_cli_missing_tensor_exits_2(model_fixtures, tmp_path):
    rec = model_fixtures["tiny-llama"]
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    w.tensors = [t for t in w.tensors if t[0] != "model.norm.weight"]
    w.write_dir(str(tmp_path))
    ids = tmp_path / "ids.txt"
    ids.write_text("1 2 3\n")
    r = subprocess.run([CLI, "--weights-dir", str(tmp_path), "--ids", str(ids)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "FATAL: tensor model.norm.weight missing" in r.stderr
