#!/usr/bin/env python3
"""Benchmark: bit-exact fp32 greedy decode, SmolLM2-135M shape, bs=1, on one
MI355X, plus the strict-order GEMV roofline and the CPU baseline.

A step is one greedy decode step of the hot path: device argmax of the logits
already computed, their witness fold on the host, and the forward pass of the
chosen token (30 layers + LM head).  The workload is the 32-token prompt plus
256 generated tokens of the SmolLM2-135M-shape synthetic model (seeded BF16
weights ~N(0,0.02)).  Every run decodes all 256 steps: `--warmup` steps run
first, then `--steps` are timed, then the rest run untimed, and the run's
witness digest and tokens are checked against the reference driver's for the
same inputs (tests/golden).  vs_baseline is value / cpu_baseline.value, the
same workload on the host CPU in the same run.

The roofline object is the persistent decode kernel's (one launch computes one
position: all layers, LM head, argmax): algorithmic bytes per launch are the
fp32 GEMV weights, the norm weights and the K/V rows read at that position,
divided by the launch's device time from HIP events on the library's own
stream (cis2_profile), summed over the timed steps.  `traffic` is the HBM
bytes per launch from the committed rocprofv3 counter summary, when present.

Beside the headline line, the same JSON object carries the other
measured workloads: the same decode with seeded sampling in place of the
argmax (sampled_decode) and in the v0.4-candidate tree order (tree_decode),
the strict-order GEMV at 1536x576, one per launch and
128 per launch (gemv_config1), the batched decode of the batch-stress
sequences at B = 1, 8, 32, 64 (batch_decode), the llama-160m set of 300
prompts decoded as one batch (llama160m_set), the Qwen3-0.6B-shape
4096-token prefill + 256-step decode (qwen3_4096), and the CPU baseline
(the oracle decoding the same 256 steps after an untimed prefill, witness
checked) both single-thread (cpu_baseline, the reference protocol) and
row-parallel over up to 16 host threads (cpu_baseline_parallel).

Prints ONE JSON line on stdout.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "cis2-lab-archive_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

METRIC = "bit-exact fp32 decode tok/s (SmolLM2-135M shape, bs=1); GEMV HBM GB/s % peak"
HBM_PEAK_GBS = 8000.0
# the reference's published C decode rate, SmolLM2-135M, 1 thread
# (labs/rust-1/reports/rust-1/RESULT.md:26)
CPU_REF_TOKS = 5.189
SEED = 20261201
GEN = 256  # generated tokens of the workload (positions 32..287)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# Algorithmic bytes of one SmolLM2-135M decode launch at position p: fp32 GEMV
# weights (30 layers x 3,538,944 + LM head 49152 x 576 floats), 61 norm vectors
# of 576 floats, and the cached K and V rows of positions 0..p (2 x 192 floats
# per layer per position).
GEMV_WEIGHT_BYTES = 4 * (30 * 3538944 + 49152 * 576)
NORM_BYTES = 4 * 61 * 576
KV_BYTES_PER_POS = 4 * 2 * 192 * 30
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_decode_smollm2_pmc.txt")
GEMV_STREAM_FILE = os.path.join(ROOT, "profiles", "k_gemv_many_1536x576_stream.txt")
LM_HEAD_FILE = os.path.join(ROOT, "profiles", "k_gemv_lm_head_49152x576.txt")
GEMV_ONE_FILE = os.path.join(ROOT, "profiles", "k_gemv_pipe_1536x576.txt")
QWEN3_FILE = os.path.join(ROOT, "profiles", "k_decode_qwen3_4096.txt")


def decode_bytes(pos):
    return GEMV_WEIGHT_BYTES + NORM_BYTES + KV_BYTES_PER_POS * (int(pos) + 1)


def spec_bytes(spec):
    """(weight bytes, KV bytes per cached position) of one decode row of a
    model: the fp32 GEMV weights of every layer and the LM head, the norm
    weights (two per layer, the QK norms, the final norm), and the K and V
    rows one position adds to the cache."""
    H, I, L = spec.hidden, spec.inter, spec.n_layers
    qd, kvd = spec.qd, spec.kvd
    gemv = L * (H * qd + 2 * H * kvd + qd * H + 3 * H * I) + spec.vocab * H
    norms = L * (2 * H + (2 * spec.hd if spec.qk_norm else 0)) + H
    return 4 * (gemv + norms), 4 * 2 * kvd * L


def roofline_obj(algo_bytes, seconds, kernel, **extra):
    achieved = algo_bytes / seconds / 1e9
    r = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": kernel}
    r.update(extra)
    return r


def measured_traffic(path=TRAFFIC_FILE):
    """HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, copy-calibrated) from a
    committed counter summary, or None."""
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch="):
                return int(line.split("=", 1)[1].split()[0])
    except OSError:
        pass
    return None


def gemv_roofline(M=1536, K=576, copies=128, iters=4096):
    """Strict-order GEMV at the config-1 shape, W rotated through `copies`
    replicas (copies*3.5 MB > the 256 MB Infinity Cache), timed with HIP
    events on the kernel's own stream."""
    from cis2amd import GemvPlan, artifacts
    W = artifacts.gen_f32(SEED, 1, M * K, 0.02).reshape(M, K)
    plan = GemvPlan(W, copies=copies)
    plan.time(256)
    ms = plan.time(iters)
    algo_bytes = 4 * M * K + 4 * K + 4 * M
    achieved = algo_bytes / (ms * 1e-3) / 1e9
    # a stream of `copies` GEMVs per launch (each on its own replica and x)
    plan.time_batch(copies, 4)
    ms_b = plan.time_batch(copies, 32)
    achieved_b = copies * algo_bytes / (ms_b * 1e-3) / 1e9
    plan.close()
    lm = lm_head_roofline(K=K)
    return {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(GEMV_ONE_FILE) if (M, K) == (1536, 576) else None,
            "kernel": "k_gemv_pipe<16, %d>: one %dx%d GEMV per launch" % (K, M, K),
            "us_per_launch": round(ms * 1e3, 3),
            "algorithmic_bytes": algo_bytes,
            "stream": {"gemvs_per_launch": copies, "us_per_launch": round(ms_b * 1e3, 2),
                       "achieved": round(achieved_b, 2), "frac": round(achieved_b / HBM_PEAK_GBS, 4),
                       "traffic": measured_traffic(GEMV_STREAM_FILE) if copies == 128 else None,
                       "kernel": "k_gemv_many: %d independent %dx%d GEMVs per launch"
                                 % (copies, M, K)},
            "lm_head": lm}


def lm_head_roofline(M=49152, K=576, copies=6, iters=66):
    """The one bs=1 GEMV wide enough to stream at HBM rate: the SmolLM2-135M
    LM head, 49152x576 strict order (113 MB of fp32 weights), one GEMV per
    launch, rotating through `copies` replicas (680 MB: each replica is read
    again only after 566 MB of other replicas, more than twice the 256 MB
    Infinity Cache, so its reads come from HBM), timed with HIP events on
    the plan's stream."""
    from cis2amd import GemvPlan, artifacts
    W = artifacts.gen_f32(SEED, 3, M * K, 0.02).reshape(M, K)
    plan = GemvPlan(W, copies=copies)
    plan.time(8)
    ms = plan.time(iters)
    plan.close()
    algo = 4 * M * K + 4 * K + 4 * M
    achieved = algo / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(LM_HEAD_FILE),
            "kernel": "k_gemv_many<16, 576> (one %dx%d GEMV per launch, %d row blocks)"
                      % (M, K, (M + 15) // 16),
            "us_per_launch": round(ms * 1e3, 3), "algorithmic_bytes": algo,
            "replicas": copies, "bytes_between_rereads": algo * (copies - 1)}


def host_cpu():
    """(model name, logical CPUs this process may use) of the host."""
    name = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return name, n


def cpu_decode(spec, weights, prompt, gen, threads, fixture):
    """The headline workload on the host CPU with the oracle (this
    repository's CPU restatement, pinned bit-identical to the reference
    driver): the 32-token prompt prefilled untimed, then `gen` greedy steps
    timed as the reference protocol times them (argmax, witness fold of the
    logits and the id, forward of the id; labs/rust-1/reports/rust-1/
    RESULT.md:13).  The witness of the run is checked against the fixture."""
    import hashlib
    import struct

    import numpy as np

    import _oracle as O
    n = len(prompt)
    m = O.OracleModel(spec, weights, max_pos=n + gen, threads=threads)
    table, invf = (bytes.fromhex(h) for h in m.digests())
    logits = np.empty(spec.vocab, np.float32)
    L = O.lib()
    for p, t in enumerate(prompt):
        L.orc_forward(m.m, p, int(t), O.ptr(logits, O.c_fp), O.TRACE_FN(), None)
    w = hashlib.sha256(weights.header_digests() + table + invf)
    w.update(b"".join(struct.pack("<I", int(t)) for t in prompt))
    ids = []
    t0 = time.perf_counter()
    for s in range(gen):
        nid = int(L.orc_argmax(O.ptr(logits, O.c_fp), spec.vocab))
        w.update(logits.tobytes())
        w.update(struct.pack("<I", nid))
        ids.append(nid)
        L.orc_forward(m.m, n + s, nid, O.ptr(logits, O.c_fp), O.TRACE_FN(), None)
    dt = time.perf_counter() - t0
    ok = None
    if fixture is not None:
        ok = (w.hexdigest() == fixture["witness"] and
              [int(v) for v in prompt] + ids == fixture["tokens"])
    return gen / dt, dt, ok


def cpu_baseline(spec, weights, prompt, gen, fixture, threads=1):
    """cpu_baseline: the whole 256-step decode (positions 32..287) on `threads`
    host threads (1: the reference's single-thread protocol; more: the oracle's
    GEMV rows split over threads, same bits since rows are independent)."""
    tok_s, dt, ok = cpu_decode(spec, weights, prompt, gen, threads, fixture)
    model, ncpu = host_cpu()
    return {"value": round(tok_s, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": "the full workload: %d greedy steps (positions %d..%d) after an untimed "
                      "%d-token prefill, %d thread(s), %.1f s" % (
                          gen, len(prompt), len(prompt) + gen - 1, len(prompt), threads, dt),
            "witness_bit_exact": ok, "cpu_model": model, "host_cpus": ncpu}


def batch_decode(spec, weights, sizes=(1, 8, 32, 64)):
    """Config 4: batched greedy decode of the batch-stress sequences (prompts of
    16..512 tokens, 256 generated each) through cis2_decode_batch: one
    row-batched prefill, then one row per sequence per step.  tok/s counts
    generated tokens over the decode steps (total time minus the prefill-only
    run).  The B=64 digests are checked against the reference's."""
    from cis2amd import Cis2Model, artifacts
    pset = artifacts.BATCH_SET
    prompts = artifacts.set_prompts(pset)
    gen = pset["gen_toks"]
    m = Cis2Model(spec, weights, max_pos=pset["hi"] + gen, max_seqs=max(sizes))
    m.decode_batch(prompts[:2], 4)
    out = {}
    for B in sizes:
        P = prompts[:B]
        t = time.perf_counter()
        m.decode_batch(P, 0)
        tp = time.perf_counter() - t
        t = time.perf_counter()
        rows = m.decode_batch(P, gen)
        tt = time.perf_counter() - t
        rec = {"tok_s": round(B * gen / (tt - tp), 1), "prefill_rows": sum(len(p) for p in P),
               "prefill_s": round(tp, 4), "total_s": round(tt, 4)}
        if B == max(sizes):
            # decode steps only: weights once per step for all B rows, each
            # row's cached K/V at its own position (prompt length + step)
            wb, kvb = spec_bytes(spec)
            algo = sum(wb + sum(kvb * (len(p) + st + 1) for p in P) for st in range(gen))
            rec["roofline"] = roofline_obj(
                algo, tt - tp, "batched decode step (row GEMMs, row attention, argmax; "
                "timed by wall clock over the %d decode steps)" % gen,
                algorithmic_bytes_per_step=int(round(algo / gen)))
        fx = os.path.join(ROOT, "tests", "golden", "batch_set.json")
        if os.path.exists(fx):
            doc = json.load(open(fx))
            if doc.get("set") == pset:
                rec["digests_bit_exact"] = all(
                    [r["witness"], r["argmax_digest"]] == doc["cases"][str(i)]
                    for i, r in enumerate(rows))
        out["B=%d" % B] = rec
        log("batch decode B=%d:" % B, rec)
    m.close()
    return out


def llama_set():
    """Config 3: llama-160m shape, the 300 seeded prompts of 8..64 tokens with
    128 greedy tokens each, all through one cis2_decode_batch call (300
    KV-cache slots): tok/s over the whole call, and whether every
    sequence's digests equal the reference's."""
    from cis2amd import Cis2Model, artifacts
    pset = artifacts.LLAMA_SET
    spec = artifacts.SPECS[pset["spec"]]
    w = artifacts.Weights(spec, pset["seed"])
    prompts = artifacts.set_prompts(pset)
    gen = pset["gen_toks"]
    m = Cis2Model(spec, w, max_pos=pset["hi"] + gen, max_seqs=len(prompts))
    m.decode_batch(prompts[:2], 4)
    t = time.perf_counter()
    m.decode_batch(prompts, 0)
    tp = time.perf_counter() - t
    t = time.perf_counter()
    rows = m.decode_batch(prompts, gen)
    tt = time.perf_counter() - t
    wb, kvb = spec_bytes(spec)
    algo = sum(wb + sum(kvb * (len(p) + st + 1) for p in prompts) for st in range(gen))
    rec = {"sequences": len(prompts), "gen_toks": gen, "total_s": round(tt, 4),
           "tok_s": round(len(prompts) * gen / tt, 1), "prefill_s": round(tp, 4),
           "roofline": roofline_obj(
               algo, tt - tp, "batched decode step over all %d sequences (wall clock over the "
               "%d decode steps, the prefill-only call's time subtracted)" % (len(prompts), gen),
               algorithmic_bytes_per_step=int(round(algo / gen)))}
    fx = os.path.join(ROOT, "tests", "golden", "llama160m_set.json")
    if os.path.exists(fx):
        doc = json.load(open(fx))
        if doc.get("set") == pset and len(doc["cases"]) >= len(prompts):
            rec["digests_bit_exact"] = all(
                [r["witness"], r["argmax_digest"]] == doc["cases"][str(i)]
                for i, r in enumerate(rows))
    m.close()
    log("llama-160m set:", rec)
    return rec


def qwen3_long(gen=256, n_prompt=4096, seed=6):
    """Config 5: Qwen3-0.6B shape, 4096-token prompt (one row-batched prefill
    pass) then 256 greedy steps of the persistent kernel with streamed
    attention (positions 4096..4351)."""
    from cis2amd import Cis2Model, artifacts
    spec = artifacts.SPECS["qwen3-0.6b"]
    w = artifacts.Weights(spec, seed)
    prompt = artifacts.prompt_ids(seed, spec.vocab, n_prompt)
    m = Cis2Model(spec, w, max_pos=n_prompt + gen)
    t = time.perf_counter()
    m.begin(prompt, gen)
    tp = time.perf_counter() - t
    m.profile(True)
    t = time.perf_counter()
    m.steps(gen)
    td = time.perf_counter() - t
    m.profile(False)
    launches, kernel_ms, positions = m.profile_read()
    r = m.end(gen)
    m.close()
    rec = {"prefill_s": round(tp, 4), "prefill_rows_s": round(n_prompt / tp, 1),
           "decode_tok_s": round(gen / td, 2), "witness": r["witness"]}
    if launches:
        wb, kvb = spec_bytes(spec)
        algo = sum(wb + kvb * (int(p) + 1) for p in positions)
        rec["roofline"] = roofline_obj(
            algo, kernel_ms * 1e-3, "k_decode (persistent, split attention; HIP events per launch)",
            traffic=measured_traffic(QWEN3_FILE), launches=launches, us_per_launch=round(kernel_ms * 1e3 / launches, 2),
            algorithmic_bytes_per_launch=int(round(algo / launches)),
            positions=[int(positions[0]), int(positions[-1])])
    fx = os.path.join(ROOT, "tests", "golden", "qwen3_fixture.json")
    if os.path.exists(fx):
        ref = json.load(open(fx)).get("qwen3-0.6b-4096")
        if ref and ref["prompt"] == [int(v) for v in prompt]:
            rec["witness_bit_exact"] = r["witness"] == ref["witness"]
    log("qwen3 4096+256:", rec)
    return rec


def sampled_decode(spec, weights, prompt):
    """Seeded sampling (v0.4 draft section 14) in place of the argmax: the
    same 32 + 256 workload under the fixture's two parameter sets (the
    draft's T 0.8 / top-k 40 / top-p 0.95, and top-p 0.95 over the whole
    vocabulary, which sorts all 49,152 logits and runs two rank-order chains
    over most of them per step).  tok/s over the 256 steps (prefill
    excluded); witness and ids against the oracle's fixture."""
    import struct
    from cis2amd import Cis2Model
    fx = os.path.join(ROOT, "tests", "golden", "sample_fixture.json")
    if not os.path.exists(fx):
        return None
    doc = json.load(open(fx))
    if doc["prompt"] != [int(v) for v in prompt]:
        return None
    gen = doc["gen_toks"]
    m = Cis2Model(spec, weights, max_pos=len(prompt) + gen)
    out = {}
    for name, c in doc["cases"].items():
        T = struct.unpack("<f", struct.pack("<I", c["temperature_bits"]))[0]
        P = struct.unpack("<f", struct.pack("<I", c["top_p_bits"]))[0]
        m.set_sampling(c["seed"], T, c["top_k"], P)
        m.begin(prompt, gen)
        t = time.perf_counter()
        m.steps(gen)
        dt = time.perf_counter() - t
        r = m.end(gen)
        out[name] = {"tok_s": round(gen / dt, 1), "top_k": c["top_k"], "top_p": round(P, 6),
                     "witness_bit_exact": r["witness"] == c["witness"] and
                     [int(v) for v in r["ids"][len(prompt):]] == c["ids"]}
        log("sampled decode %s:" % name, out[name])
    m.close()
    return out


def tree_decode(spec, weights, prompt, gen=256):
    """The same greedy workload in the v0.4-candidate tree reduction order
    (reduction_mode 1, the reference's -DCIS2_REDUCTION_TREE build): tok/s
    over steps 17..256, the kernel time per launch (HIP events around each
    launch on its stream) and the witness against the reference driver's
    tree-order fixture."""
    from cis2amd import Cis2Model
    m = Cis2Model(spec, weights, max_pos=len(prompt) + gen, reduction_mode=1)
    m.begin(prompt, gen)
    m.steps(16)
    m.profile(True)
    t = time.perf_counter()
    m.steps(gen - 16)
    dt = time.perf_counter() - t
    m.profile(False)
    launches, kernel_ms, _ = m.profile_read()
    r = m.end(gen)
    m.close()
    rec = {"tok_s": round((gen - 16) / dt, 1), "witness": r["witness"]}
    if launches:
        rec["us_per_launch"] = round(kernel_ms * 1e3 / launches, 2)
    fx = os.path.join(ROOT, "tests", "golden", "model_fixtures.json")
    if os.path.exists(fx):
        ref = json.load(open(fx)).get("smollm2-135m-tree")
        if ref and list(ref["prompt"]) == [int(v) for v in prompt] and ref["gen_toks"] == gen:
            rec["witness_bit_exact"] = r["witness"] == ref["witness"]
    log("tree-order decode:", rec)
    return rec


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-roofline", action="store_true")
    ap.add_argument("--no-batch", action="store_true", help="skip the batched-decode sizes")
    ap.add_argument("--no-qwen3", action="store_true", help="skip the Qwen3 4096+256 run")
    ap.add_argument("--only", choices=["qwen3", "batch", "llama"], default=None,
                    help="run one side workload alone and print its JSON (profiling)")
    ap.add_argument("--batch-sizes", default="1,8,32,64",
                    help="batch sizes of the batched decode (comma-separated)")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only the strict-order GEMV rooflines (config 1, the stream, the LM head)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 512 MiB device-to-device copy (counter calibration)")
    a = ap.parse_args()
    if a.copy_calibration:
        import torch
        n = 128 << 20  # floats: 512 MiB per buffer
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copied 3 x %d bytes" % (4 * n))
        print(json.dumps({"copy_bytes": 4 * n, "copies": 3}), flush=True)
        return
    if a.only:
        from cis2amd import artifacts
        spec = artifacts.SPECS["smollm2-135m"]
        if a.only == "qwen3":
            out = {"qwen3_4096": qwen3_long()}
        elif a.only == "llama":
            out = {"llama160m_set": llama_set()}
        else:
            out = {"batch_decode": batch_decode(spec, artifacts.Weights(spec, SEED),
                                                sizes=tuple(int(v) for v in a.batch_sizes.split(",")))}
        print(json.dumps(out), flush=True)
        return
    if a.gemv_only:
        print(json.dumps({"gemv_config1": gemv_roofline()}), flush=True)
        return
    if a.gpus != 1:
        print("bench.py: one GPU only (the pinned-order decode is not sharded across GPUs); "
              "use --gpus 1", file=sys.stderr)
        sys.exit(2)
    from cis2amd import Cis2Model, artifacts
    spec = artifacts.SPECS["smollm2-135m"]
    if a.warmup < 0 or a.steps < 1 or a.warmup + a.steps > GEN:
        print("bench.py: --warmup + --steps must be within the workload's %d decode steps "
              "(1 <= steps, warmup >= 0)" % GEN, file=sys.stderr)
        sys.exit(2)
    t = time.perf_counter()
    weights = artifacts.Weights(spec, SEED)
    prompt = artifacts.prompt_ids(SEED, spec.vocab, 32)
    log("weights generated in %.1fs" % (time.perf_counter() - t))
    fixture = None
    fx_path = os.path.join(ROOT, "tests", "golden", "model_fixtures.json")
    if os.path.exists(fx_path):
        rec = json.load(open(fx_path)).get("smollm2-135m")
        if rec and list(rec["prompt"]) == [int(v) for v in prompt] and rec["gen_toks"] == GEN:
            fixture = rec
    # the whole workload every run: prefill, `warmup` steps, `steps` timed
    # steps, the rest of the 256 untimed; the witness covers all 256
    model = Cis2Model(spec, weights, max_pos=len(prompt) + GEN)
    # a short session first, so that loading the kernels' code objects and
    # the first launches' one-time work fall outside the measured workload
    model.begin(prompt[:8], 8)
    model.steps(8)
    model.end(8)
    # the per-launch timing events are created here, outside every timed
    # window (the first cis2_profile(1) creates them)
    model.profile(True)
    model.profile(False)
    t = time.perf_counter()
    model.begin(prompt, GEN)
    prefill_s = time.perf_counter() - t
    ta = time.perf_counter()
    model.steps(a.warmup)  # returns with the stream drained
    model.profile(True)
    t0 = time.perf_counter()
    model.steps(a.steps)   # blocks until every step is folded and the stream drained
    t1 = time.perf_counter()
    model.profile(False)
    rest = GEN - a.warmup - a.steps
    if rest:
        model.steps(rest)
    tb = time.perf_counter()
    launches, kernel_ms, positions = model.profile_read()
    res = model.end(GEN)
    dt = t1 - t0
    value = a.steps / dt
    witness_ok = None
    if fixture is not None:
        witness_ok = (res["witness"] == fixture["witness"] and
                      [int(v) for v in res["ids"]] == fixture["tokens"])
    log("decode: %d timed steps (steps %d..%d of %d) in %.3fs -> %.1f tok/s; prefill 32 tokens "
        "%.3fs; witness_ok=%s" % (a.steps, a.warmup, a.warmup + a.steps - 1, GEN, dt, value,
                                  prefill_s, witness_ok))
    roof = None
    if launches:
        algo = sum(decode_bytes(p) for p in positions)
        achieved = algo / (kernel_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(),
                "kernel": "k_decode (persistent: 30 layers + LM head + argmax per launch)",
                "launches": launches, "us_per_launch": round(kernel_ms * 1e3 / launches, 2),
                "algorithmic_bytes_per_launch": int(round(algo / launches)),
                "positions": [int(positions[0]), int(positions[-1])]}
        log("decode kernel roofline:", roof)
    model.close()
    cpu = None
    if not a.no_cpu_baseline:
        cpu = cpu_baseline(spec, weights, prompt, GEN, fixture, threads=1)
        log("cpu baseline:", cpu)
    out = {
        "metric": METRIC, "value": round(value, 3), "unit": "tok/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(dt * 1e3 / a.steps, 4),
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(value / cpu["value"], 2) if cpu else None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "SmolLM2-135M-shape fp32 greedy decode, bs=1, 32-token prompt "
                               "+ 256 generated tokens, seeded BF16 weights ~N(0,0.02)",
                   "global_batch": 1, "seq_len": len(prompt) + GEN, "parallelism": "none",
                   "timed_steps": [a.warmup, a.warmup + a.steps - 1]},
        "witness_bit_exact": witness_ok, "witness": res["witness"],
        "vs_published_cpu": round(value / CPU_REF_TOKS, 2),
        # every decode step of the workload (positions 32..287, the warmup
        # and untimed steps included; the prefill excluded), wall clock
        "all_steps": {"steps": GEN, "tok_s": round(GEN / (tb - ta), 3),
                      "ms_per_step": round((tb - ta) * 1e3 / GEN, 4)},
    }
    if cpu is not None:
        out["cpu_baseline"] = cpu
    if roof is not None:
        out["roofline"] = roof
    sd = sampled_decode(spec, weights, prompt)
    if sd is not None:
        out["sampled_decode"] = sd
    out["tree_decode"] = tree_decode(spec, weights, prompt)
    if not a.no_roofline:
        out["gemv_config1"] = gemv_roofline()
        log("standalone GEMV 1536x576:", out["gemv_config1"])
    if not a.no_batch:
        out["batch_decode"] = batch_decode(spec, weights,
                                           sizes=tuple(int(v) for v in a.batch_sizes.split(",")))
        out["llama160m_set"] = llama_set()
    if not a.no_qwen3:
        out["qwen3_4096"] = qwen3_long()
    if not a.no_cpu_baseline:
        _model, ncpu = host_cpu()
        out["cpu_baseline_parallel"] = cpu_baseline(spec, weights, prompt, GEN, fixture,
                                                    threads=max(1, min(16, ncpu)))
        log("cpu baseline (row-parallel):", out["cpu_baseline_parallel"])
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
