"""Sharing the GPU with the persistent decode kernel.

Its grid (one workgroup per CU) must be resident at once; every phase wait
is bounded by a spin cap.  These tests force the bounded waits to give up
from the host (a one-sleep cap set at context creation, CIS2_SPIN_CAP) so
that every launch still ends normally, and check that each affected step is
recomputed on the per-op path with the reference bits (decode sessions,
sampled decodes, single forward passes).  Two CLI processes then decode the
headline case at the same time: with the per-GPU session lock (the default)
and without it (where a grid that finds CUs held by the other process's
grid gives up at a short cap and recovers); both digests must equal the
reference driver's."""
import os
import subprocess
import sys

import numpy as np
import pytest

from cis2amd import Cis2Model, artifacts

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "cis2-lab-archive_amd", "bin", "cis2_host")


def model_with_env(spec, w, max_pos, **env):
    old = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    try:
        return Cis2Model(spec, w, max_pos=max_pos)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen3", "smollm2-short"])
def test_decode_recovers_when_waits_give_up(model_fixtures, name):
    rec = model_fixtures[name]
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    m = model_with_env(spec, w, len(rec["prompt"]) + rec["gen_toks"], CIS2_SPIN_CAP=1)
    try:
        r = m.decode(rec["prompt"], rec["gen_toks"])
        assert m.recoveries() >= 1, "the one-sleep cap never made a wait give up"
        assert r["witness"] == rec["witness"]
        assert [int(t) for t in r["ids"]] == rec["tokens"]
        # the context stays usable: a second session recovers again
        n0 = m.recoveries()
        r2 = m.decode(rec["prompt"], rec["gen_toks"])
        assert r2["witness"] == rec["witness"] and m.recoveries() > n0
    finally:
        m.close()


def test_session_split_and_sampled_recovery(model_fixtures):
    """Steps enqueued across several cis2_decode_steps calls (the recovery
    can fall on a call's last pass) and a sampled decode, both against the
    same model without the forced cap."""
    rec = model_fixtures["tiny-llama"]
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    n = len(rec["prompt"]) + rec["gen_toks"]
    ref = Cis2Model(spec, w, max_pos=n)
    m = model_with_env(spec, w, n, CIS2_SPIN_CAP=1)
    try:
        m.begin(rec["prompt"], rec["gen_toks"])
        for k in (1, 2, 3, rec["gen_toks"] - 6):
            m.steps(k)
        r = m.end(rec["gen_toks"])
        assert r["witness"] == rec["witness"] and m.recoveries() >= 1
        for mm in (ref, m):
            mm.set_sampling(1234, 0.8, 40, 0.95)
        want = ref.decode(rec["prompt"], rec["gen_toks"])
        got = m.decode(rec["prompt"], rec["gen_toks"])
        assert got["witness"] == want["witness"]
        assert list(got["ids"]) == list(want["ids"])
    finally:
        ref.close()
        m.close()


def test_forward_recovers_when_waits_give_up(model_fixtures):
    rec = model_fixtures["tiny-qwen3"]
    spec = artifacts.SPECS[rec["spec"]]
    w = artifacts.Weights(spec, rec["seed"])
    ref = Cis2Model(spec, w, max_pos=16)
    m = model_with_env(spec, w, 16, CIS2_SPIN_CAP=1)
    try:
        for p, t in enumerate(rec["prompt"]):
            lr, ar = ref.forward_token(p, t)
            lg, ag = m.forward_token(p, t)
            assert lg.tobytes() == lr.tobytes() and ag == ar, p
        assert m.recoveries() >= 1
    finally:
        ref.close()
        m.close()


def _cli_case(model_fixtures, tmp_path):
    rec = model_fixtures["smollm2-135m"]
    spec = artifacts.SPECS[rec["spec"]]
    artifacts.Weights(spec, rec["seed"]).write_dir(str(tmp_path))
    ids = tmp_path / "ids.txt"
    ids.write_text("\n".join(str(t) for t in rec["prompt"]) + "\n")
    return rec, [CLI, "--weights-dir", str(tmp_path), "--ids", str(ids), "--gen-toks",
                 str(rec["gen_toks"])]


@pytest.mark.parametrize("lock", ["1", "0"])
def test_two_processes_decode_at_the_same_time(model_fixtures, tmp_path, lock):
    if not os.path.exists(CLI):
        pytest.skip("cis2_host not built")
    rec, cmd = _cli_case(model_fixtures, tmp_path)
    env = dict(os.environ, CIS2_LOCK_DIR=str(tmp_path), CIS2_DECODE_LOCK=lock)
    if lock == "0":
        env["CIS2_SPIN_CAP"] = str(1 << 16)  # a few ms: a grid short of CUs gives up soon
    print("starting two decoding processes, lock=%s" % lock, flush=True)
    procs = [subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                              env=env) for _ in range(2)]
    outs = [p.communicate(timeout=180) for p in procs]
    for p, (out, err) in zip(procs, outs):
        assert p.returncode == 0, err[-2000:]
        assert "CIS2_REF digest=%s" % rec["witness"] in out, out[-500:]
