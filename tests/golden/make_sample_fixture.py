"""Generate tests/golden/sample_fixture.json: sampled decodes (CIS-2 v0.4
draft section 14) of the SmolLM2-135M-shape synthetic model computed by the
oracle (oracle/liboracle.so, pinned by the draft's known answers), for the
bench's workload: seed-20261201 weights, the 32-token prompt, 256 drawn
tokens, under two parameter sets:
  draft: seed 1, T 0.8, top_k 40, top_p 0.95 (the draft's model-vector settings)
  full_top_p: seed 7, T 0.8, top_k 0, top_p 0.95 (top-p over the whole vocabulary)

The reference's own sampler source is not archived (only its digests on the
real weights, which are not available offline); these values pin the device
path to the oracle at the full workload size.

Usage: python tests/golden/make_sample_fixture.py
"""
import json
import os
import struct
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "cis2-lab-archive_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import _oracle as O  # noqa: E402
from cis2amd import artifacts  # noqa: E402

SEED = 20261201
SETS = {
    "draft": {"seed": 1, "temperature_bits": 0x3F4CCCCD, "top_k": 40, "top_p_bits": 0x3F733333},
    "full_top_p": {"seed": 7, "temperature_bits": 0x3F4CCCCD, "top_k": 0, "top_p_bits": 0x3F733333},
}


def f32(bits):
    return struct.unpack("<f", struct.pack("<I", bits))[0]


def main():
    spec = artifacts.SPECS["smollm2-135m"]
    w = artifacts.Weights(spec, SEED)
    prompt = artifacts.prompt_ids(SEED, spec.vocab, 32)
    gen = 256
    o = O.OracleModel(spec, w, max_pos=32 + gen, threads=8)
    doc = {"spec": "smollm2-135m", "weights_seed": SEED, "prompt": [int(t) for t in prompt],
           "gen_toks": gen, "cases": {}}
    for name, p in SETS.items():
        r = o.decode_sampled(prompt, gen, p["seed"], f32(p["temperature_bits"]), p["top_k"],
                             f32(p["top_p_bits"]))
        doc["cases"][name] = dict(p, witness=r["witness"], argmax_digest=r["argmax_digest"],
                                  ids=[int(t) for t in r["ids"][32:]])
        print(name, r["witness"], flush=True)
    out = os.path.join(ROOT, "tests", "golden", "sample_fixture.json")
    with open(out, "w") as f:
        json.dump(doc, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
