"""Per-phase timeline of the persistent decode kernel (a profiling tool).

With CIS2_TIMELINE=<file> set before a context is created, every launch of
the persistent decode kernel records four device timestamps (s_memrealtime,
100 MHz) per (layer, phase, task): 0 task start, 1 inputs gathered, 3 the
middle of the task (after the norm / before the GEMV chain; for the
attention task after the softmax), 2 done (outputs published).  The LM
phase records 0 start, 1 final norm input gathered, 2 its blocks done, and
3 on the workgroup that reduced the argmax candidates.

This module records a greedy decode that way and summarises, per phase of a
layer (medians over the middle layers and the recorded launches):
  handover   earliest task's inputs-ready minus the predecessor phase's last
             done (the latency of the tagged-word hand-over)
  ready      median / slowest task's inputs-ready, from the same origin
  norm/soft  median task's ready -> mid (RMSNorm, or scores + softmax)
  chain      median task's mid -> done (GEMV product pass + strict chains,
             or the V mix, and the publish)
  done       median / slowest task's done, from the same origin
  phase      the critical path: slowest done minus the predecessor's
             slowest done; the phases sum to the layer time.

Usage:
  python -m cis2amd.timeline [--spec smollm2-135m] [--reduction 0|1]
      [--prompt 32] [--steps 24] [--from-pos 40] [--max-pos N] [--file PATH]
"""
import argparse
import os
import struct
import sys
import tempfile

import numpy as np

PHASES = ["QKV", "ATT", "O", "GU", "D"]
TICK_US = 0.01  # s_memrealtime: 100 MHz


def record(spec_name, reduction, n_prompt, steps, path, seed=20261201, max_pos=None):
    """Decodes `steps` greedy tokens after an `n_prompt`-token prompt with
    the timeline on; max_pos (default prompt + steps) sizes the context as a
    longer decode would (the attention plan depends on it)."""
    os.environ["CIS2_TIMELINE"] = path
    from . import Cis2Model, artifacts
    spec = artifacts.SPECS[spec_name]
    w = artifacts.Weights(spec, seed)
    prompt = artifacts.prompt_ids(seed, spec.vocab, n_prompt)
    m = Cis2Model(spec, w, max_pos=max(max_pos or 0, n_prompt + steps), reduction_mode=reduction)
    try:
        m.begin(prompt, steps)
        m.steps(steps)
        r = m.end(steps)
    finally:
        m.close()
        os.environ.pop("CIS2_TIMELINE", None)
    return r


def load(path):
    """[(position, stamps[L][6][T][4] int64, want_logits)]"""
    data = open(path, "rb").read()
    off, out = 0, []
    while off < len(data):
        pos, L, T, wl = struct.unpack_from("<4I", data, off)
        off += 16
        n = L * 6 * T * 4
        a = np.frombuffer(data, np.uint64, n, off).reshape(L, 6, T, 4).astype(np.int64)
        off += n * 8
        out.append((pos, a, wl))
    return out


def summarize(recs, from_pos=0):
    rows = {ph: [] for ph in range(5)}
    lm, layer_t = [], []
    for pos, a, wl in recs:
        if pos < from_pos:
            continue
        L = a.shape[0]
        for l in range(1, L - 1):
            prev_done = None
            for ph in range(5):
                if ph == 0:
                    pd = a[l - 1, 4]
                else:
                    pd = a[l, ph - 1]
                pd = pd[pd[:, 2] > 0]
                cur = a[l, ph]
                cur = cur[cur[:, 2] > 0]
                if len(pd) == 0 or len(cur) == 0:
                    continue
                t0 = pd[:, 2].max()
                rd, md, dn = cur[:, 1] - t0, cur[:, 3] - t0, cur[:, 2] - t0
                rows[ph].append([rd.min(), np.median(rd), rd.max(),
                                 np.median(cur[:, 3] - cur[:, 1]),
                                 np.median(cur[:, 2] - cur[:, 3]),
                                 np.median(dn), dn.max()])
                prev_done = t0
            d_prev = a[l - 1, 4]
            d_cur = a[l, 4]
            d_prev = d_prev[d_prev[:, 2] > 0]
            d_cur = d_cur[d_cur[:, 2] > 0]
            if len(d_prev) and len(d_cur):
                layer_t.append(d_cur[:, 2].max() - d_prev[:, 2].max())
        if wl:
            d_last = a[L - 1, 4]
            d_last = d_last[d_last[:, 2] > 0]
            s = a[L - 1, 5]
            fin = s[s[:, 3] > 0]
            blk = s[s[:, 2] > 0]
            if len(d_last) and len(fin) and len(blk):
                t0 = d_last[:, 2].max()
                lm.append([np.median(blk[:, 1] - t0), np.median(blk[:, 2] - t0),
                           blk[:, 2].max() - t0, fin[:, 3].max() - t0])
    lines = ["times in us; origin: the predecessor phase's slowest task done; "
             "medians over layers 1..L-2 of the launches at positions >= %d" % from_pos,
             "%-4s %9s %15s %9s %9s %15s %8s" % ("", "handover", "ready med/max", "norm/soft",
                                                "chain", "done med/max", "phase")]
    total = 0.0
    for ph in range(5):
        if not rows[ph]:
            continue
        r = np.median(np.array(rows[ph], dtype=np.float64), axis=0) * TICK_US
        total += r[6]
        lines.append("%-4s %9.2f %7.2f/%7.2f %9.2f %9.2f %7.2f/%7.2f %8.2f" % (
            PHASES[ph], r[0], r[1], r[2], r[3], r[4], r[5], r[6], r[6]))
    lines.append("sum of phases %.2f us; layer time (slowest D to slowest D) median %.2f us" % (
        total, np.median(layer_t) * TICK_US if layer_t else float("nan")))
    if lm:
        m = np.median(np.array(lm, dtype=np.float64), axis=0) * TICK_US
        lines.append("LM   norm input ready %.2f, blocks done med %.2f / max %.2f, argmax "
                     "reduced %.2f (from the last layer's slowest D)" % tuple(m))
    return "\n".join(lines)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--spec", default="smollm2-135m")
    ap.add_argument("--reduction", type=int, default=0)
    ap.add_argument("--prompt", type=int, default=32)
    ap.add_argument("--steps", type=int, default=24)
    ap.add_argument("--from-pos", type=int, default=40)
    ap.add_argument("--max-pos", type=int, default=None,
                    help="context size (default prompt + steps)")
    ap.add_argument("--file", default=None, help="timeline file (default: a temporary file)")
    a = ap.parse_args(argv)
    path = a.file or os.path.join(tempfile.mkdtemp(prefix="cis2tl_"), "timeline.bin")
    r = record(a.spec, a.reduction, a.prompt, a.steps, path, max_pos=a.max_pos)
    print("%s reduction=%d prompt=%d steps=%d witness=%s" % (
        a.spec, a.reduction, a.prompt, a.steps, r["witness"]))
    print(summarize(load(path), a.from_pos))
    if not a.file:
        os.remove(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
