"""Seeded sampling on the device (CIS-2 v0.4 draft section 14,
code/patches/cis2-spec__seeded-sampling.patch:57-196) against the oracle:
single draws over every parameter regime and vocabulary sizes up to
Qwen3's, and whole sampled decodes (ids, witness with the CIS2-SAMPLE-1
header, argmax digest, per-step logit digests)."""
import struct

import numpy as np
import pytest

import _oracle as O
from cis2amd import Cis2Error, Cis2Model, artifacts

pytestmark = pytest.mark.gpu


def f32(bits):
    return struct.unpack("<f", struct.pack("<I", bits))[0]


def tiny_with_vocab(V):
    return artifacts.ModelSpec("tiny-v%d" % V, 64, 128, 1, 4, 2, V, 1e-5, 10000.0, True)


@pytest.fixture(scope="module")
def ctx_by_vocab():
    made = {}

    def get(V):
        if V not in made:
            spec = tiny_with_vocab(V)
            made[V] = Cis2Model(spec, artifacts.Weights(spec, 5), max_pos=8)
        return made[V]
    yield get
    for m in made.values():
        m.close()


def rows(rng, V, n):
    out = []
    for t in range(n):
        kind = t % 4
        if kind == 0:
            lg = rng.standard_normal(V).astype(np.float32)
        elif kind == 1:  # ties and signed zeros
            lg = rng.integers(-3, 4, V).astype(np.float32) * np.float32(0.25)
            lg[rng.random(V) < 0.2] = np.float32(-0.0)
        elif kind == 2:  # wide spread: most exp terms underflow
            lg = (rng.standard_normal(V) * 40).astype(np.float32)
        else:  # near-flat, like random-init logits: top-p keeps most of the vocabulary
            lg = (rng.standard_normal(V) * 0.01).astype(np.float32)
        out.append(lg)
    return out


PARAMS = [  # (T, top_k, top_p)
    (1.0, 0, 1.0),            # nothing cut: no sort
    (0.8, 40, 0.95),          # the draft's model-vector settings
    (0.8, 0, 0.95),           # top-p over the whole vocabulary
    (f32(0x3F4CCCCD), 1, 1.0),  # top-1
    (2.5, 1000, 0.5),
    (0.05, 0, 1e-6),          # top-p keeps rank 0 only
    (1.0, 5, 1.0),
]


@pytest.mark.parametrize("V", [256, 4096, 4097, 49152, 151936])
def test_draws_match_oracle(V, ctx_by_vocab):
    m = ctx_by_vocab(V)
    rng = np.random.default_rng(V)
    lgs = rows(rng, V, 4)
    for T, k, p in PARAMS:
        for seed in (1, 0xFFFFFFFFFFFFFFFF, int(rng.integers(0, 2**63))):
            m.set_sampling(seed, T, k, p)
            steps = [0, 1, 7, int(rng.integers(0, 2**32))]
            ids, nk = m.sample_logits(np.stack(lgs), steps)
            for lg, st, i, n in zip(lgs, steps, ids, nk):
                want, _, wk = O.sample(lg, seed, st, T, k, p)
                assert (int(i), int(n)) == (want, wk), (V, T, k, p, seed, st)
    m.set_sampling(None)


def test_top_k_at_and_beyond_vocab_is_disabled(ctx_by_vocab):
    V = 512
    m = ctx_by_vocab(V)
    lg = np.random.default_rng(2).standard_normal(V).astype(np.float32)
    got = []
    for k in (0, V, V + 1, 2**32 - 1):
        m.set_sampling(9, 1.0, k, 1.0)
        got.append(int(m.sample_logits(lg[None], [3])[0][0]))
    assert len(set(got)) == 1
    assert got[0] == O.sample(lg, 9, 3, 1.0, 0, 1.0)[0]
    m.set_sampling(None)


def test_invalid_parameters_and_nan(ctx_by_vocab):
    m = ctx_by_vocab(256)
    for T, p in ((0.0, 1.0), (-1.0, 1.0), (float("inf"), 1.0), (float("nan"), 1.0),
                 (1.0, 0.0), (1.0, 1.5), (1.0, float("nan"))):
        with pytest.raises(Cis2Error) as e:
            m.set_sampling(1, T, 0, p)
        assert e.value.code == -1
    for k, p in ((0, 1.0), (10, 0.9)):
        m.set_sampling(1, 1.0, k, p)
        lg = np.zeros(256, np.float32)
        lg[17] = np.nan
        with pytest.raises(Cis2Error) as e:
            m.sample_logits(lg[None], [0])
        assert e.value.code == -10
    # the context works again afterwards
    lg = np.linspace(-1, 1, 256, dtype=np.float32)
    m.set_sampling(4, 1.0, 0, 1.0)
    assert int(m.sample_logits(lg[None], [0])[0][0]) == O.sample(lg, 4, 0, 1.0, 0, 1.0)[0]
    m.set_sampling(None)


@pytest.mark.parametrize("name,n_prompt,gen,params", [
    ("tiny-llama", 5, 24, (1, 0.8, 40, 0.95)),
    ("tiny-qwen3", 3, 16, (77, 1.3, 0, 0.9)),
    ("tiny-untied", 4, 16, (2**64 - 1, 0.5, 3, 1.0)),
    ("smollm2-135m", 32, 32, (1, f32(0x3F4CCCCD), 40, f32(0x3F733333))),
    ("smollm2-135m", 8, 16, (5, 1.0, 0, 1.0)),
])
def test_sampled_decode_matches_oracle(name, n_prompt, gen, params):
    spec = artifacts.SPECS[name]
    w = artifacts.Weights(spec, 20261201)
    prompt = artifacts.prompt_ids(20261201, spec.vocab, n_prompt)
    seed, T, k, p = params
    m = Cis2Model(spec, w, max_pos=n_prompt + gen)
    m.set_sampling(seed, T, k, p)
    got = m.decode(prompt, gen)
    # greedy again on the same context: unchanged receipts
    m.set_sampling(None)
    greedy = m.decode(prompt, gen)
    m.close()
    o = O.OracleModel(spec, w, max_pos=n_prompt + gen)
    want = o.decode_sampled(prompt, gen, seed, T, k, p)
    want_greedy = o.decode(prompt, gen)
    assert list(got["ids"]) == list(want["ids"])
    assert got["witness"] == want["witness"]
    assert got["argmax_digest"] == want["argmax_digest"]
    assert got["step_digests"] == want["step_digests"]
    assert greedy["witness"] == want_greedy["witness"]
    assert got["witness"] != want_greedy["witness"]


def test_sampled_stepwise_session_equals_one_call():
    spec = artifacts.SPECS["tiny-llama"]
    w = artifacts.Weights(spec, 3)
    prompt = artifacts.prompt_ids(3, spec.vocab, 6)
    m = Cis2Model(spec, w, max_pos=6 + 20)
    m.set_sampling(123, 0.7, 16, 0.8)
    one = m.decode(prompt, 20)
    m.begin(prompt, 20)
    m.steps(7)
    m.steps(13)
    parts = m.end(20)
    assert parts["witness"] == one["witness"] and list(parts["ids"]) == list(one["ids"])
    # greedy-only paths refuse sampling mode
    with pytest.raises(Cis2Error) as e:
        m.decode_batch([prompt], 4)
    assert e.value.code == -2
    m.close()


def test_cli_sample_flag(tmp_path):
    """cis2_host --sample SEED,T,K,P (the lab driver's flag): the CIS2_REF
    digest is the sampled witness, one `step N next_id=ID` line per step,
    T and P parsed as f32 by correct rounding ("0.8" -> 3f4ccccd)."""
    import os
    import re
    import subprocess
    cli = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                       "cis2-lab-archive_amd", "bin", "cis2_host")
    spec = artifacts.SPECS["tiny-llama"]
    w = artifacts.Weights(spec, 8)
    w.write_dir(str(tmp_path))
    prompt = artifacts.prompt_ids(8, spec.vocab, 4)
    ids = tmp_path / "ids.txt"
    ids.write_text("\n".join(str(t) for t in prompt) + "\n")
    r = subprocess.run([cli, "--weights-dir", str(tmp_path), "--ids", str(ids), "--gen-toks", "12",
                        "--sample", "1,0.8,40,0.95"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    o = O.OracleModel(spec, w, max_pos=4 + 12)
    want = o.decode_sampled(prompt, 12, 1, f32(0x3F4CCCCD), 40, f32(0x3F733333))
    assert re.search(r"^CIS2_REF digest=%s prompt_idx=0 prompt_toks=4 gen_toks=12 dtype=fp32 "
                     r"reduction_mode=sequential$" % want["witness"], r.stdout, re.M)
    steps = re.findall(r"^step (\d+) next_id=(\d+)$", r.stdout, re.M)
    assert [int(i) for _, i in steps] == [int(v) for v in want["ids"][4:]]
    assert "temperature=3f4ccccd top_k=40 top_p=3f733333" in r.stdout
    for bad in ("1,0,40,0.95", "1,0.8,40,0", "1,0.8,40,1.5", "1,0.8,40", "x,0.8,1,1", "1,nan,1,1"):
        r = subprocess.run([cli, "--weights-dir", str(tmp_path), "--ids", str(ids), "--sample", bad],
                           capture_output=True, text=True, timeout=60)
        assert r.returncode == 2 and "FATAL: --sample" in r.stderr, bad


def test_smollm2_256_sampled_tokens_match_fixture():
    """The bench workload (SmolLM2-135M shape, 32-token prompt, 256 drawn
    tokens) under both fixture parameter sets, against the oracle's
    witnesses (tests/golden/sample_fixture.json)."""
    import json
    import os
    doc = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                      "sample_fixture.json")))
    spec = artifacts.SPECS[doc["spec"]]
    w = artifacts.Weights(spec, doc["weights_seed"])
    prompt = np.array(doc["prompt"], dtype=np.uint32)
    m = Cis2Model(spec, w, max_pos=prompt.size + doc["gen_toks"])
    for name, c in doc["cases"].items():
        m.set_sampling(c["seed"], f32(c["temperature_bits"]), c["top_k"], f32(c["top_p_bits"]))
        r = m.decode(prompt, doc["gen_toks"])
        assert r["witness"] == c["witness"], name
        assert [int(v) for v in r["ids"][prompt.size:]] == c["ids"], name
    m.close()
