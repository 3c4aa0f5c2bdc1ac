"""Malformed weight files (the reference lab's loader-robustness study,
labs/rust-3/PREREG-from-ledger.md: seven structure-aware mutation operators
O1 header-length field, O2 JSON keys and values, O3 tensor offsets, O4
shapes including overflowing products, O5 dtype codes, O6 truncation at 100
cut points, O7 duplicate keys) against the CLI's safetensors reader.

Every mutant of a valid tiny model must be refused with a `FATAL:` line and
exit status 2 (never a crash, a hang or a digest), and every mutant whose
declared sizes or offsets disagree with the file must be refused by the
reader itself (the lab's "wrongly accepted" class).  The reader is also
built with AddressSanitizer and UBSan (host code) and run on every mutant.
The CLI checks the weights before it creates a device context, so all of
this runs without a GPU."""
import json
import os
import shutil
import struct
import subprocess

import pytest

from cis2amd import artifacts

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "cis2-lab-archive_amd", "bin", "cis2_host")
TARGET = "model.layers.0.self_attn.q_proj.weight"


def split(blob):
    n = struct.unpack("<Q", blob[:8])[0]
    return json.loads(blob[8:8 + n]), blob[8 + n:]


def join(header, data, raw_header=None):
    h = raw_header if raw_header is not None else json.dumps(header).encode()
    return struct.pack("<Q", len(h)) + h + data


def mutants(blob):
    """(operator, label, bytes, level): level "reader" = not a valid
    safetensors file (sizes, offsets or syntax disagree with the file),
    "model" = a valid file that does not hold this model's tensors, None = a
    valid file for the model."""
    hdr, data = split(blob)
    hlen = struct.unpack("<Q", blob[:8])[0]
    out = []
    # O1 header-length field
    for v in (0, 1, 2, hlen - 1, hlen + 1, len(blob) - 8, len(blob), 2**63, 2**64 - 1):
        out.append(("O1", "hlen=%d" % v, struct.pack("<Q", v) + blob[8:], "reader"))
    # O2 JSON keys and values
    def edit(fn):
        h = json.loads(json.dumps(hdr))
        fn(h)
        return join(h, data)
    out.append(("O2", "rename required", edit(lambda h: h.__setitem__("zz", h.pop(TARGET))), "model"))
    out.append(("O2", "entry is a list", edit(lambda h: h.__setitem__(TARGET, [1, 2])), "reader"))
    out.append(("O2", "drop dtype", edit(lambda h: h[TARGET].pop("dtype")), "reader"))
    out.append(("O2", "drop shape", edit(lambda h: h[TARGET].pop("shape")), "reader"))
    out.append(("O2", "drop offsets", edit(lambda h: h[TARGET].pop("data_offsets")), "reader"))
    out.append(("O2", "shape is a string", edit(lambda h: h[TARGET].__setitem__("shape", "64,64")), "reader"))
    out.append(("O2", "metadata not an object", edit(lambda h: h.__setitem__("__metadata__", 5)), "reader"))
    out.append(("O2", "header is a list", join(None, data, b"[1,2,3]"), "reader"))
    out.append(("O2", "broken JSON", join(None, data, json.dumps(hdr).encode()[:-7]), "reader"))
    out.append(("O2", "NUL bytes", join(None, data, b"{\"a\":\x00\x00}"), "reader"))
    out.append(("O2", "deep nesting", join(None, data, b"[" * 100000 + b"]" * 100000), "reader"))
    out.append(("O2", "metadata text", edit(lambda h: h.__setitem__("__metadata__", {"k": "v"})), None))
    # O3 tensor offsets
    b0, e0 = hdr[TARGET]["data_offsets"]
    for lab, offs in (("swap", [e0, b0]), ("past end", [b0, len(data) + 2]),
                      ("shift +2", [b0 + 2, e0 + 2]), ("shift -2", [b0 - 2, e0 - 2]),
                      ("negative", [-2, e0]), ("huge", [b0, 1e30]), ("fraction", [b0 + 0.5, e0]),
                      ("2^64", [b0, 18446744073709551616]), ("empty", [b0, b0]),
                      ("overlap next", [b0, e0 + 2]), ("strings", ["0", "8"]), ("three", [b0, e0, e0])):
        out.append(("O3", lab, edit(lambda h, o=offs: h[TARGET].__setitem__("data_offsets", o)), "reader"))
    # O4 shapes
    shp = hdr[TARGET]["shape"]
    for lab, sh in (("2^32 x 2^32", [2**32, 2**32]), ("overflow x 2", [2**62, 4]),
                    ("zero dim", [0, shp[1]]), ("negative", [-shp[0], shp[1]]),
                    ("extra dim", shp + [1]), ("transposed", shp[::-1] if shp[0] != shp[1] else [shp[0] * 2, shp[1] // 2]),
                    ("fraction", [shp[0] + 0.5, shp[1]]), ("double rows", [shp[0] * 2, shp[1]]),
                    ("scalar", []), ("2^53", [2**53, 1])):
        out.append(("O4", lab, edit(lambda h, s=sh: h[TARGET].__setitem__("shape", s)),
                    "model" if lab in ("transposed", "extra dim") else "reader"))
    # O5 dtype codes
    for dt in ("F32", "F16", "BF17", "", "bf16", 7):
        out.append(("O5", "dtype=%r" % (dt,), edit(lambda h, d=dt: h[TARGET].__setitem__("dtype", d)),
                    "model" if dt in ("F16",) else "reader"))
    # O6 truncation at 100 cut points
    for i in range(100):
        cut = max(1, (len(blob) - 1) * i // 100)
        out.append(("O6", "cut=%d" % cut, blob[:cut], "reader"))
    # O7 duplicate keys
    raw = json.dumps(hdr).encode()
    ent = json.dumps({TARGET: hdr[TARGET]})[1:-1].encode()
    out.append(("O7", "duplicate target", join(None, data, raw[:-1] + b"," + ent + b"}"), "reader"))
    ent2 = json.dumps({TARGET: dict(hdr[TARGET], data_offsets=[0, e0 - b0])})[1:-1].encode()
    out.append(("O7", "duplicate, other offsets", join(None, data, raw[:-1] + b"," + ent2 + b"}"), "reader"))
    out.append(("O7", "duplicate metadata", join(None, data, b'{"__metadata__":{},' + raw[1:-1] +
                                                b',"__metadata__":{}}'), "reader"))
    return out


@pytest.fixture(scope="module")
def model_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("tiny")
    artifacts.Weights(artifacts.SPECS["tiny-llama"], 1).write_dir(str(d))
    (d / "ids.txt").write_text("1 2 3\n")
    return d


def test_operators_cover_the_lab_set(model_dir):
    ops = {m[0] for m in mutants((model_dir / "model.safetensors").read_bytes())}
    assert ops == {"O1", "O2", "O3", "O4", "O5", "O6", "O7"}


def test_cli_refuses_every_mutant(model_dir, tmp_path):
    if not os.path.exists(CLI):
        pytest.skip("cis2_host not built")
    blob = (model_dir / "model.safetensors").read_bytes()
    w = tmp_path / "w"
    w.mkdir()
    for f in ("config.json", "tokenizer.json"):
        shutil.copy(model_dir / f, w / f)
    # the unmutated file passes the reader (and stops at the device here or runs)
    (w / "model.safetensors").write_bytes(blob)
    r = subprocess.run([CLI, "--weights-dir", str(w), "--ids", str(model_dir / "ids.txt"),
                        "--gen-toks", "1"], capture_output=True, text=True, timeout=60)
    assert "FATAL: tensor" not in r.stderr and "FATAL: safetensors" not in r.stderr
    for op, lab, data, level in mutants(blob):
        (w / "model.safetensors").write_bytes(data)
        r = subprocess.run([CLI, "--weights-dir", str(w), "--ids", str(model_dir / "ids.txt"),
                            "--gen-toks", "1"], capture_output=True, text=True, timeout=30)
        what = "%s %s: rc=%d %s" % (op, lab, r.returncode, r.stderr[-300:])
        assert "CIS2_REF digest=" not in r.stdout, what
        if level:
            assert r.returncode == 2, what
            assert "FATAL:" in r.stderr and "cis2_ctx_create" not in r.stderr, what
        else:
            assert "FATAL: tensor" not in r.stderr, what


def test_reader_under_sanitizers(model_dir, tmp_path):
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("no g++")
    exe = tmp_path / "st_harness"
    src = os.path.join(ROOT, "tests", "st_harness.cpp")
    inc = os.path.join(ROOT, "cis2-lab-archive_amd", "csrc")
    b = subprocess.run([gxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
                        "-fno-sanitize-recover=undefined", "-I" + inc, "-o", str(exe), src,
                        os.path.join(inc, "cis2_sha256.cpp")],
                       capture_output=True, text=True, timeout=300)
    assert b.returncode == 0, b.stderr[-2000:]
    blob = (model_dir / "model.safetensors").read_bytes()
    f = tmp_path / "m.safetensors"
    f.write_bytes(blob)
    r = subprocess.run([str(exe), str(f)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.startswith("accepted"), r.stderr[-500:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:exitcode=99",
               UBSAN_OPTIONS="exitcode=98")
    for op, lab, data, level in mutants(blob):
        f.write_bytes(data)
        r = subprocess.run([str(exe), str(f)], capture_output=True, text=True, timeout=30, env=env)
        what = "%s %s: rc=%d %s" % (op, lab, r.returncode, r.stderr[-600:])
        assert "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, what
        assert r.returncode in (0, 2), what
        if level == "reader":
            assert r.returncode == 2 and "FATAL:" in r.stderr, what
        else:
            assert r.returncode == 0, what


def test_cli_refuses_oversized_header_before_reading_it(model_dir, tmp_path):
    """A (sparse) file whose header-length field claims 150 MiB, which the
    file does hold: refused by the 100 MiB cap before the header is
    allocated or read, not after a 150 MiB allocation."""
    if not os.path.exists(CLI):
        pytest.skip("cis2_host not built")
    w = tmp_path / "w"
    w.mkdir()
    for f in ("config.json", "tokenizer.json"):
        shutil.copy(model_dir / f, w / f)
    hlen = 150 << 20
    with open(w / "model.safetensors", "wb") as f:
        f.write(struct.pack("<Q", hlen) + b"{")
        f.truncate(8 + hlen + 64)  # sparse: no disk blocks behind the claim
    r = subprocess.run([CLI, "--weights-dir", str(w), "--ids", str(model_dir / "ids.txt"),
                        "--gen-toks", "1"], capture_output=True, text=True, timeout=30)
    assert r.returncode == 2, r.stderr[-300:]
    assert "FATAL: safetensors: header length above the 100 MiB limit" in r.stderr
