"""The hash-chained receipt log (code/cis2-llm/server/app/receipts.py:31-97)
in both implementations, the CLI's (C++, tests/receipts_harness.cpp drives
it) and the Python mirror (cis2amd.receipts): logs written by either verify
with the other; the canonical form the hashes cover equals Python's
json.dumps(sort_keys=True, separators=(",", ":")) on arbitrary JSON
(property-based); tampering is caught at the right line with the service
verifier's messages; concurrent appends keep one linear chain; a broken
chain is never extended.  The CLI's --verify-chain runs without a GPU."""
import json
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from cis2amd import receipts

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "cis2-lab-archive_amd", "bin", "cis2_host")
INC = os.path.join(ROOT, "cis2-lab-archive_amd", "csrc")


@pytest.fixture(autouse=True)
def ieee_fpenv():
    """Canonical JSON of subnormal floats needs the default FP environment:
    an oracle test that ran earlier in this process left FTZ|DAZ pinned on
    the main thread."""
    import _oracle
    had = _oracle.fpenv_release()
    yield
    if had:
        _oracle.fpenv_repin()


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("no g++")
    exe = tmp_path_factory.mktemp("rh") / "receipts_harness"
    b = subprocess.run([gxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
                        "-fno-sanitize-recover=undefined", "-I" + INC, "-o", str(exe),
                        os.path.join(ROOT, "tests", "receipts_harness.cpp"),
                        os.path.join(INC, "cis2_sha256.cpp")],
                       capture_output=True, text=True, timeout=300)
    assert b.returncode == 0, b.stderr[-2000:]
    return str(exe)


def run(harness, *args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0")
    return subprocess.run([harness] + list(args), capture_output=True, text=True, timeout=60,
                          env=env)


def fields(i):
    return {"receipt_id": "r%02d" % i, "witness_digest": "%064x" % (i * 7919),
            "generated_token_ids": [i, i + 1, 49151], "note": "café ✓ #%d" % i,
            "score": 0.1 * i, "nested": {"b": [True, None], "a": -i}}


def cpp_append(harness, log, f, tmp_path):
    p = tmp_path / "fields.json"
    p.write_text(json.dumps(f))
    r = run(harness, "append", str(log), str(p))
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout.strip()


def cpp_verify(harness, log, upto=None):
    r = run(harness, "verify", str(log), *([upto] if upto else []))
    assert "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr
    return r.returncode == 0, r.stdout.strip()


def test_python_log_verifies_in_cpp(harness, tmp_path):
    log = tmp_path / "r.jsonl"
    L = receipts.ReceiptLog(log)
    recs = [L.append(fields(i)) for i in range(4)]
    assert L.verify_chain() == (True, "chain OK")
    assert cpp_verify(harness, log) == (True, "chain OK")
    assert recs[0]["prev_hash"] == receipts.GENESIS and recs[1]["prev_hash"] == recs[0]["log_hash"]
    assert cpp_verify(harness, log, "r02") == (True, "chain OK through line 2")
    assert cpp_verify(harness, log, "zz") == (False, "receipt_id zz not found")


def test_cpp_log_verifies_in_python(harness, tmp_path):
    log = tmp_path / "r.jsonl"
    hashes = [cpp_append(harness, log, fields(i), tmp_path) for i in range(4)]
    L = receipts.ReceiptLog(log)
    assert L.verify_chain() == (True, "chain OK")
    recs = L.records()
    assert [r["log_hash"] for r in recs] == hashes
    # the line text is json.dumps(record, sort_keys=True): the service's own form
    for line, rec in zip(log.read_text().splitlines(), recs):
        assert line == json.dumps(rec, sort_keys=True)
    # and mixed: a Python append continues a C++ chain and vice versa
    L.append(fields(9))
    cpp_append(harness, log, fields(10), tmp_path)
    assert L.verify_chain() == (True, "chain OK")
    assert cpp_verify(harness, log) == (True, "chain OK")


def tamper_cases(lines):
    edit = json.loads(lines[1])
    edit["witness_digest"] = "0" * 64
    t1 = list(lines)
    t1[1] = json.dumps(edit, sort_keys=True)
    t2 = lines[:1] + lines[2:]                         # a record removed
    t3 = [lines[0], lines[2], lines[1]] + lines[3:]     # two records swapped
    rec = json.loads(lines[2])
    t4 = list(lines)
    t4[2] = json.dumps(dict(reversed(list(rec.items()))))  # key order changed: still valid
    t5 = list(lines)
    t5[0] = lines[0].replace("r00", "r99")             # id of the first record changed
    return [(t1, False, "line 1: log_hash mismatch (tampered record)"),
            (t2, False, "line 1: prev_hash mismatch"),
            (t3, False, "line 1: prev_hash mismatch"),
            (t4, True, "chain OK"),
            (t5, False, "line 0: log_hash mismatch (tampered record)")]


def test_tampering_detected_by_both(harness, tmp_path):
    log = tmp_path / "r.jsonl"
    L = receipts.ReceiptLog(log)
    for i in range(4):
        L.append(fields(i))
    lines = log.read_text().splitlines()
    for k, (t, ok, msg) in enumerate(tamper_cases(lines)):
        p = tmp_path / ("t%d.jsonl" % k)
        p.write_text("\n".join(t) + "\n")
        assert receipts.ReceiptLog(p).verify_chain() == (ok, msg), k
        assert cpp_verify(harness, p) == (ok, msg), k


def test_broken_chain_not_extended(harness, tmp_path):
    log = tmp_path / "r.jsonl"
    L = receipts.ReceiptLog(log)
    for i in range(3):
        L.append(fields(i))
    lines = log.read_text().splitlines()
    log.write_text("\n".join(tamper_cases(lines)[0][0]) + "\n")
    before = log.read_text()
    with pytest.raises(RuntimeError):
        L.append(fields(5))
    p = tmp_path / "f.json"
    p.write_text(json.dumps(fields(6)))
    r = run(harness, "append", str(log), str(p))
    assert r.returncode == 1 and "existing log is broken" in r.stdout
    assert log.read_text() == before


def test_concurrent_appends_stay_linear(harness, tmp_path):
    log = tmp_path / "r.jsonl"

    def worker(w):
        for i in range(8):
            p = tmp_path / ("f%d_%d.json" % (w, i))
            p.write_text(json.dumps(dict(fields(i), receipt_id="w%d-%d" % (w, i))))
            r = run(harness, "append", str(log), str(p))
            assert r.returncode == 0, r.stdout + r.stderr
        for i in range(4):
            receipts.ReceiptLog(log).append(dict(fields(i), receipt_id="p%d-%d" % (w, i)))

    with ThreadPoolExecutor(4) as ex:
        list(ex.map(worker, range(4)))
    L = receipts.ReceiptLog(log)
    assert len(L.records()) == 48
    assert L.verify_chain() == (True, "chain OK")
    assert cpp_verify(harness, log) == (True, "chain OK")


json_values = st.recursive(
    st.none() | st.booleans() | st.integers(min_value=-(10 ** 30), max_value=10 ** 30) |
    st.floats(allow_nan=False, allow_infinity=False) | st.text(max_size=12),
    lambda inner: st.lists(inner, max_size=4) | st.dictionaries(st.text(max_size=6), inner,
                                                              max_size=4),
    max_leaves=12)


@settings(max_examples=120, deadline=None)
@given(json_values)
def test_canonical_form_equals_python(harness, tmp_path_factory, value):
    d = tmp_path_factory.mktemp("c")
    p = d / "v.json"
    p.write_text(json.dumps(value, ensure_ascii=False), encoding="utf-8")
    r = run(harness, "canon", str(p))
    assert r.returncode == 0, r.stderr
    assert r.stdout == receipts.canonical(value).decode()


def test_canonical_floats_at_power_of_two_boundaries(harness, tmp_path):
    """Below a power of two the neighbouring doubles are twice as close, so
    the correctly rounded n-digit decimal can fail to read back while the
    next one up does (2^-24: 5.960464477539063e-08, not ...0625e-08); every
    power of two, its neighbours and a few classic cases."""
    import math
    vals = []
    for k in range(-1074, 1024):
        v = math.ldexp(1.0, k)
        vals += [v, math.nextafter(v, 0.0), math.nextafter(v, math.inf), -v]
    vals += [0.1 + 0.2, 1e23, 9007199254740993.0, 5e-324, 2.2250738585072014e-308,
             1.7976931348623157e308, 1e16, 1e-4, 9.999999999999999e-5, 123456789012345678.0]
    p = tmp_path / "v.json"
    p.write_text(json.dumps(vals))
    r = run(harness, "canon", str(p))
    assert r.returncode == 0, r.stderr
    assert r.stdout == receipts.canonical(vals).decode()


def test_cli_verify_chain(harness, tmp_path):
    if not os.path.exists(CLI):
        pytest.skip("cis2_host not built")
    log = tmp_path / "r.jsonl"
    L = receipts.ReceiptLog(log)
    for i in range(3):
        L.append(fields(i))
    r = subprocess.run([CLI, "--verify-chain", str(log)], capture_output=True, text=True,
                       timeout=60)
    head = L.records()[-1]["log_hash"]
    assert r.returncode == 0
    assert r.stdout == "CIS2_CHAIN PASS records=3 head=%s message=chain OK\n" % head
    r = subprocess.run([CLI, "--verify-chain", str(log), "--receipt-id", "r01"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "message=chain OK through line 1" in r.stdout
    bad = tmp_path / "b.jsonl"
    tampered, _ok, _msg = tamper_cases(log.read_text().splitlines())[0]
    bad.write_text("\n".join(tampered) + "\n")
    r = subprocess.run([CLI, "--verify-chain", str(bad)], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 1 and "CIS2_CHAIN FAIL" in r.stdout and "line 1: log_hash mismatch" in r.stdout
