"""The CLI's host readers on the CPU: strict JSON for config.json and the
safetensors header (every escape validated, UTF-8 decoded, grammar
enforced, no recursion), and the streaming safetensors reader's peak
memory: one tensor at a time, as the reference's per-tensor loader holds
(code/cis2-fp/src/stream_widen.rs:1-33)."""
import json
import os
import shutil
import struct
import subprocess

import pytest

from cis2amd import artifacts

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "cis2-lab-archive_amd", "bin", "cis2_host")
BASE = {"model_type": "llama", "torch_dtype": "bfloat16", "hidden_size": 576,
        "num_attention_heads": 9}


def run_cfg(text, tmp_path):
    if not os.path.exists(CLI):
        pytest.skip("cis2_host not built")
    d = tmp_path / "w"
    d.mkdir(exist_ok=True)
    (d / "config.json").write_bytes(text if isinstance(text, bytes) else text.encode())
    ids = tmp_path / "ids.txt"
    ids.write_text("1 2 3\n")
    return subprocess.run([CLI, "--weights-dir", str(d), "--ids", str(ids), "--gen-toks", "1"],
                          capture_output=True, text=True, timeout=60)


def base_with(raw_member):
    """config.json text: BASE plus one raw (unescaped-by-us) member."""
    body = json.dumps(BASE)[:-1]
    return body + ", " + raw_member + "}"


@pytest.mark.parametrize("raw,why", [
    ('"x": "a\\qb"', "unknown escape"),
    ('"x": "\\u00g1"', "non-hex digit"),
    ('"x": "\\u12"', "non-hex digit"),
    ('"x": "\\ud800"', "lone high surrogate"),
    ('"x": "\\ud800\\u0041"', "lone high surrogate"),
    ('"x": "\\udc00"', "lone low surrogate"),
    ('"x": "a\x01b"', "control character"),
    ('"x": 01', "expected ','"),
    ('"x": [1,]', "expected a value"),
    ('"x": 1.', "malformed number"),
    ('"x": -', "malformed number"),
    ('"x": 1e', "malformed number"),
    ('"x": tru', "unexpected character"),
    ('"x": "open', "unterminated string"),
    ('"model_type": "qwen2"', "duplicate key"),
    ('"x": ' + "[" * 65 + "]" * 65, "nesting deeper than 64"),
])
def test_config_json_strict(raw, why, tmp_path):
    r = run_cfg(base_with(raw), tmp_path)
    assert r.returncode == 2
    assert "CIS2_REF_UNSUPPORTED" not in r.stderr
    assert r.stderr.startswith("FATAL: JSON: ") and why in r.stderr, r.stderr


@pytest.mark.parametrize("text,why", [
    (json.dumps(BASE) + " x", "bytes after the document"),
    (json.dumps(BASE) + "{}", "bytes after the document"),
    ("", "unexpected end of input"),
    ("   ", "unexpected end of input"),
    ('{"a" 1}', "expected ':'"),
    ('{"a": 1 "b": 2}', "expected ',' or '}'"),
    ('{1: 2}', "expected a member name"),
    ('{"a": 1,}', "expected a member name"),
])
def test_config_json_grammar(text, why, tmp_path):
    r = run_cfg(text, tmp_path)
    assert r.returncode == 2
    assert r.stderr.startswith("FATAL: JSON: ") and why in r.stderr, r.stderr


def test_config_json_values_decoded(tmp_path):
    # every escape form and value kind parses; the gate then passes and the
    # driver stops at the missing weights
    raw = ('"x": [1, 2.5e3, -0, 0.5E-2, true, false, null, {}, [], '
           '{"b": "\\/\\"\\\\\\b\\f\\n\\r\\t\\u0041\\u00e9\\ud83d\\ude00"}]')
    r = run_cfg(base_with(raw), tmp_path)
    assert "CIS2_REF_UNSUPPORTED" not in r.stderr
    assert "FATAL: cannot open" in r.stderr and "model.safetensors" in r.stderr


def test_unicode_escape_decoded_in_refusal(tmp_path):
    # the refusal names the model_type as decoded text (serde's {:?} of the
    # string), not with replacement characters
    cfg = json.dumps(dict(BASE, model_type="lláma"), ensure_ascii=True)
    assert "\\u00e1" in cfg
    r = run_cfg(cfg, tmp_path)
    assert r.returncode == 2
    assert r.stderr.splitlines()[0].startswith('CIS2_REF_UNSUPPORTED reason=model_type="lláma"')


@pytest.fixture(scope="module")
def plain_harness(tmp_path_factory):
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("no g++")
    exe = tmp_path_factory.mktemp("h") / "st_harness"
    b = subprocess.run([gxx, "-std=c++17", "-O2", "-I" + os.path.join(ROOT, "cis2-lab-archive_amd",
                                                                      "csrc"),
                        "-o", str(exe), os.path.join(ROOT, "tests", "st_harness.cpp"),
                        os.path.join(ROOT, "cis2-lab-archive_amd", "csrc", "cis2_sha256.cpp")],
                       capture_output=True, text=True, timeout=300)
    assert b.returncode == 0, b.stderr[-2000:]
    return str(exe)


def test_streaming_reader_holds_one_tensor(plain_harness, tmp_path):
    """A Qwen3-0.6B-shape checkpoint (1.19 GB of BF16, data section sparse)
    read whole, tensor by tensor: the peak resident set is about the largest
    tensor (the 311 MB embedding) plus overhead, not the file."""
    spec = artifacts.SPECS["qwen3-0.6b"]
    hdr, off = {}, 0
    largest = 0
    for name, shape in artifacts.tensor_list(spec):
        nb = 2
        for d in shape:
            nb *= d
        hdr[name] = {"dtype": "BF16", "shape": list(shape), "data_offsets": [off, off + nb]}
        off += nb
        largest = max(largest, nb)
    h = json.dumps(hdr, separators=(",", ":")).encode()
    f = tmp_path / "model.safetensors"
    with open(f, "wb") as fp:
        fp.write(struct.pack("<Q", len(h)) + h)
        fp.truncate(8 + len(h) + off)
    total = 8 + len(h) + off
    r = subprocess.run([plain_harness, str(f), "--all"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr[-500:]
    fields = dict(kv.split("=") for kv in r.stdout.split() if "=" in kv)
    peak = int(fields["peak_rss_kb"]) * 1024
    assert int(fields["largest_bytes"]) == largest
    assert peak < largest + (96 << 20), (peak, largest, total)
    assert peak < total // 3
