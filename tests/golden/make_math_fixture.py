"""Generate tests/golden/math_chunk_hashes.json.

For each pinned function (exp, sin, cos, ln, silu, rsqrt, sqrt) the 2^32
binary32 inputs are split into 256 chunks of 2^24 consecutive bit patterns.
Each chunk is summarised by an order-free 64-bit hash
    sum_i mix64(bits(f(x_i)) ^ (bits(x_i) * 0x9E3779B97F4A7C15))  (mod 2^64)
computed with the repository oracle (oracle/liboracle.so) AND, when the
reference archive is present, with the reference's own cis2_math.h compiled
in oracle/_ref/libref_math.so.  The two must agree on every chunk; the
fixture then pins the device kernels, which compute the same hash.

Usage: python tests/golden/make_math_fixture.py [--procs 8]
"""
import argparse
import ctypes
import json
import os
import sys
from multiprocessing import Pool

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
FNS = ["exp", "sin", "cos", "ln", "silu", "rsqrt", "sqrt"]
CHUNK = 1 << 24


def _libs():
    o = ctypes.CDLL(os.path.join(ROOT, "oracle", "liboracle.so"))
    o.orc_math_chunk_hash.restype = ctypes.c_uint64
    o.orc_math_chunk_hash.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32]
    r = None
    rp = os.path.join(ROOT, "oracle", "_ref", "libref_math.so")
    if os.path.exists(rp):
        r = ctypes.CDLL(rp)
        r.ref_math_chunk_hash.restype = ctypes.c_uint64
        r.ref_math_chunk_hash.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32]
    return o, r


def work(args):
    fn, chunk = args
    o, r = _libs()
    h = o.orc_math_chunk_hash(fn, chunk * CHUNK, CHUNK)
    hr = r.ref_math_chunk_hash(fn, chunk * CHUNK, CHUNK) if r is not None else None
    return fn, chunk, h, hr


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--procs", type=int, default=8)
    ap.add_argument("--out", default=os.path.join(ROOT, "tests", "golden", "math_chunk_hashes.json"))
    a = ap.parse_args()
    jobs = [(f, c) for f in range(len(FNS)) for c in range(256)]
    res = {n: [None] * 256 for n in FNS}
    mism = []
    with Pool(a.procs) as p:
        for fn, chunk, h, hr in p.imap_unordered(work, jobs, chunksize=4):
            res[FNS[fn]][chunk] = "%016x" % h
            if hr is not None and hr != h:
                mism.append((FNS[fn], chunk))
    if mism:
        print("MISMATCH oracle vs reference:", mism[:20], file=sys.stderr)
        sys.exit(1)
    _, r = _libs()
    doc = {"chunk_bits": 24, "hash": "sum mix64(out_bits ^ in_bits*0x9E3779B97F4A7C15)",
           "checked_against_reference": r is not None, "chunks": res}
    with open(a.out, "w") as f:
        json.dump(doc, f, indent=0)
    print("wrote", a.out, "reference-checked:", r is not None)


if __name__ == "__main__":
    main()
