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


def test_verify2_line_protocol(tmp_path):
    """`cis2-verify2` (the same driver under the verifier's name, no
    arguments, weights/ in the working directory) runs the section 13.1
    prompt (6403, 1980, 253, 655) for 16 tokens twice and prints the five
    lines the service's runner parses (code/cis2-llm/server/app/runner.py:
    25-31; verify2/src/main.rs:479-500), with the oracle's digests."""
    import _oracle as O
    spec = artifacts.SPECS["smollm2-135m"]
    w = artifacts.Weights(spec, 20261201)
    (tmp_path / "weights").mkdir()
    w.write_dir(str(tmp_path / "weights"))
    v2 = os.path.join(ROOT, "cis2-lab-archive_amd", "bin", "cis2-verify2")
    r = subprocess.run([v2], cwd=str(tmp_path), capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    pats = {
        "witness_digest": re.compile(r"^CIS2_VERIFY2 digest=([0-9a-f]+)"),
        "argmax_digest": re.compile(r"^argmax_digest=([0-9a-f]+)"),
        "table_digest": re.compile(r"^table_digest=([0-9a-f]+)"),
        "inv_freq_table_digest": re.compile(r"^inv_freq table_digest=([0-9a-f]+)"),
        "generated_token_ids": re.compile(r"^generated_token_ids=\[([0-9, ]+)\]"),
    }
    got = {}
    for line in r.stdout.splitlines():
        for k, p in pats.items():
            m = p.match(line)
            if m:
                got[k] = m.group(1)
    assert set(got) == set(pats), r.stdout
    assert len(r.stdout.splitlines()) == 5
    prompt = [6403, 1980, 253, 655]
    o = O.OracleModel(spec, w, max_pos=4 + 16)
    want = o.decode(prompt, 16)
    t, f = o.digests()
    assert got["witness_digest"] == want["witness"]
    assert got["argmax_digest"] == want["argmax_digest"]
    assert got["table_digest"] == t and got["inv_freq_table_digest"] == f
    assert [int(x) for x in got["generated_token_ids"].split(",")] == [int(v) for v in want["ids"][4:]]
    assert r.stdout.splitlines()[0].endswith(" prompt_toks=4 gen_toks=16 dtype=fp32")


def test_cli_head_dim_null_derives(model_fixtures, tmp_path):
    """A llama config.json with "head_dim": null passes the gate and runs
    with the derived head_dim (hidden / heads), as the reference driver
    derives it (code/cis2-fp/gpu/cis2_host.cpp:114): the tokens and the
    argmax digest equal the fixture's (the witness binds config.json's hash,
    which the null key changes)."""
    import json
    rec = model_fixtures["tiny-llama"]
    spec = artifacts.SPECS[rec["spec"]]
    artifacts.Weights(spec, rec["seed"]).write_dir(str(tmp_path))
    cfg = json.loads((tmp_path / "config.json").read_text())
    cfg["head_dim"] = None
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    ids = tmp_path / "ids.txt"
    ids.write_text("\n".join(str(t) for t in rec["prompt"]) + "\n")
    r = subprocess.run([CLI, "--weights-dir", str(tmp_path), "--ids", str(ids), "--gen-toks",
                        str(rec["gen_toks"])], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "run1_argmax_digest=%s" % rec["argmax_digest"] in r.stdout
    toks = re.search(r"run1_tokens=\[([0-9, ]*)\]", r.stdout).group(1)
    assert [int(t) for t in toks.split(",")] == rec["tokens"]


def test_second_process_decodes_beside_a_live_context(model_fixtures, tmp_path):
    """Two processes on one GPU: while this process holds a context that has
    run the persistent decode kernel, the CLI in a child process decodes the
    same case with the same digest (the kernel's launch must not need a
    per-device resource that the first process keeps)."""
    from cis2amd import Cis2Model
    rec = model_fixtures["tiny-llama"]
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    m = Cis2Model(spec, w, max_pos=len(rec["prompt"]) + rec["gen_toks"])
    try:
        assert m.decode(rec["prompt"], rec["gen_toks"])["witness"] == rec["witness"]
        w.write_dir(str(tmp_path))
        ids = tmp_path / "ids.txt"
        ids.write_text("\n".join(str(t) for t in rec["prompt"]) + "\n")
        r = subprocess.run([CLI, "--weights-dir", str(tmp_path), "--ids", str(ids), "--gen-toks",
                            str(rec["gen_toks"])], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr[-2000:]
        assert "CIS2_REF digest=%s" % rec["witness"] in r.stdout
        assert m.decode(rec["prompt"], rec["gen_toks"])["witness"] == rec["witness"]
    finally:
        m.close()


def test_cli_receipt_log(model_fixtures, tmp_path):
    """--receipt-log appends one hash-chained record per run (the service's
    log format, code/cis2-llm/server/app/receipts.py:31-97) holding the
    run's digests; --verify-chain and the Python mirror both accept the log,
    and a record altered afterwards is reported."""
    import json
    from cis2amd import receipts
    rec = model_fixtures["tiny-llama"]
    artifacts.Weights(artifacts.SPECS[rec["spec"]], rec["seed"]).write_dir(str(tmp_path))
    ids = tmp_path / "ids.txt"
    ids.write_text("\n".join(str(t) for t in rec["prompt"]) + "\n")
    log = tmp_path / "receipts.jsonl"
    for _ in range(2):
        r = subprocess.run([CLI, "--weights-dir", str(tmp_path), "--ids", str(ids), "--gen-toks",
                            str(rec["gen_toks"]), "--receipt-log", str(log)],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr[-2000:]
        assert "CIS2_REF digest=%s" % rec["witness"] in r.stdout
    L = receipts.ReceiptLog(log)
    assert L.verify_chain() == (True, "chain OK")
    recs = L.records()
    assert len(recs) == 2 and recs[0]["receipt_id"] != recs[1]["receipt_id"]
    for x in recs:
        assert x["witness_digest"] == rec["witness"]
        assert x["argmax_digest"] == rec["argmax_digest"]
        assert x["table_digest"] == rec["table_digest"]
        assert x["prompt_token_ids"] + x["generated_token_ids"] == rec["tokens"]
        assert x["cis2_version"] == "v0.3b" and x["backend"] == "gfx950"
    v = subprocess.run([CLI, "--verify-chain", str(log)], capture_output=True, text=True, timeout=60)
    assert v.returncode == 0 and "CIS2_CHAIN PASS records=2" in v.stdout
    lines = log.read_text().splitlines()
    bad = json.loads(lines[0])
    bad["generated_token_ids"][0] ^= 1
    log.write_text(json.dumps(bad, sort_keys=True) + "\n" + lines[1] + "\n")
    v = subprocess.run([CLI, "--verify-chain", str(log)], capture_output=True, text=True, timeout=60)
    assert v.returncode == 1 and "line 0: log_hash mismatch (tampered record)" in v.stdout


def _trace_lines(path):
    """{(pos, layer, op): sha} of a --trace file."""
    out = {}
    for line in path.read_text().splitlines():
        m = re.match(r"pos=(-?\d+) layer=(-?\d+) op=(\S+) sha256=([0-9a-f]{64})$", line)
        assert m, line
        out[(int(m.group(1)), int(m.group(2)), m.group(3))] = m.group(4)
    return out


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen3-tree", "smollm2-short"])
def test_cli_layer_digests_and_layer_dumps(name, model_fixtures, tmp_path):
    """--layer-digests (main.rs:743-751, 382-384, 496-501, 509-514, 525-527)
    prints LAYER_DIGEST lines for the last prompt position: the embedding,
    each block's output (the trace's resid2), the final norm and the
    logits; CIS2_DUMP_LAYERS prints CIS2_DUMP lines (main.rs:326-335) for
    that position and the first generated one.  Both are checked against
    the --trace file of the same run, which is itself byte-equal to the
    reference driver's trace (trace_sha256); the decode's digests are
    unchanged."""
    rec = model_fixtures[name]
    spec = artifacts.SPECS[rec["spec"]]
    artifacts.Weights(spec, rec["seed"]).write_dir(str(tmp_path))
    ids = tmp_path / "ids.txt"
    ids.write_text("\n".join(str(t) for t in rec["prompt"]) + "\n")
    trace = tmp_path / "trace.txt"
    mode = rec.get("reduction", "sequential")
    env = dict(os.environ, CIS2_DUMP_LAYERS="1")
    r = subprocess.run([CLI, "--weights-dir", str(tmp_path), "--ids", str(ids), "--gen-toks",
                        str(rec["gen_toks"]), "--trace", str(trace), "--reduction", mode,
                        "--layer-digests"], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stderr[-2000:]
    assert hashlib.sha256(trace.read_bytes()).hexdigest() == rec["trace_sha256"]
    assert "CIS2_REF digest=%s" % rec["witness"] in r.stdout
    t = _trace_lines(trace)
    last = len(rec["prompt"]) - 1
    want = ["LAYER_DIGEST embed %s" % t[(last, -1, "embedding")]]
    want += ["LAYER_DIGEST block_%d %s" % (li, t[(last, li, "resid2")])
             for li in range(spec.n_layers)]
    want += ["LAYER_DIGEST final_norm %s" % t[(last, -1, "final_norm")],
             "LAYER_DIGEST logits %s" % t[(last, -1, "logits")]]
    got = [l for l in r.stdout.splitlines() if l.startswith("LAYER_DIGEST")]
    assert got == want
    assert got == rec["layer_digests"]  # read from the reference driver's trace
    assert r.stdout.splitlines()[:len(want)] == want  # before every other stdout line
    dumps = [l for l in r.stderr.splitlines() if l.startswith("CIS2_DUMP ")]
    want_d = []
    for pos in (last, last + 1):
        want_d.append("CIS2_DUMP layer=embed field=token_embedding pos=%d digest=%s"
                      % (pos, t[(pos, -1, "embedding")]))
        for li in range(spec.n_layers):
            want_d.append("CIS2_DUMP layer=block%d field=post_attention_hidden pos=%d digest=%s"
                          % (li, pos, t[(pos, li, "resid1")]))
            want_d.append("CIS2_DUMP layer=block%d field=post_mlp_hidden pos=%d digest=%s"
                          % (li, pos, t[(pos, li, "resid2")]))
        want_d.append("CIS2_DUMP layer=final_norm field=final_norm_output pos=%d digest=%s"
                      % (pos, t[(pos, -1, "final_norm")]))
        want_d.append("CIS2_DUMP layer=logits field=pre_argmax_logits pos=%d digest=%s"
                      % (pos, t[(pos, -1, "logits")]))
    assert dumps == want_d


@pytest.mark.parametrize("name", ["tiny-qwen3", "smollm2-short"])
def test_cli_logit_dumps_match_oracle(name, model_fixtures, tmp_path):
    """CIS2_DUMP_STEP0_LOGITS / CIS2_DUMP_LASTSTEP_LOGITS (main.rs:1145-1160,
    1197-1212): raw little-endian fp32 files of step 0's logits and the
    final generated step's, bit-equal to the oracle's forward passes at
    those positions."""
    import numpy as np

    import _oracle as O
    rec = model_fixtures[name]
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    w.write_dir(str(tmp_path))
    ids = tmp_path / "ids.txt"
    ids.write_text("\n".join(str(t) for t in rec["prompt"]) + "\n")
    s0, sl = tmp_path / "step0.f32", tmp_path / "last.f32"
    env = dict(os.environ, CIS2_DUMP_STEP0_LOGITS=str(s0), CIS2_DUMP_LASTSTEP_LOGITS=str(sl))
    r = subprocess.run([CLI, "--weights-dir", str(tmp_path), "--ids", str(ids), "--gen-toks",
                        str(rec["gen_toks"])], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "CIS2_REF digest=%s" % rec["witness"] in r.stdout
    assert "[debug] wrote step-0 logits (%d f32 values) to %s" % (spec.vocab, s0) in r.stderr
    assert "[debug] wrote final-step logits (%d f32 values) to %s" % (spec.vocab, sl) in r.stderr
    toks = rec["tokens"]
    n = len(rec["prompt"])
    o = O.OracleModel(spec, w, max_pos=n + rec["gen_toks"])
    lg = None
    for p in range(n + rec["gen_toks"]):
        lg = o.forward(p, toks[p])
        if p == n - 1:
            assert s0.read_bytes() == lg.astype(np.float32).tobytes()
    assert sl.read_bytes() == lg.astype(np.float32).tobytes()
