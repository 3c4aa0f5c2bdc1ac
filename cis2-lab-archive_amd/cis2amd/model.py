"""Host-side mirror of the reference forward-pass interface.

Reference interface (code/cis2-fp/gpu/cis2_model.h:635-774,
code/cis2-fp/gpu/cis2_host.cpp:61-249):
  Cis2Workspace::alloc(model, max_positions)   -> Cis2Model(spec, ..., max_pos)
  cis2_forward_token(model, ws, pos, tok, trace) + cis2_download(logits)
                                                -> Cis2Model.forward_token(pos, tok)
  the cis2_host greedy/witness loop              -> Cis2Model.decode(prompt, gen_toks)
  Cis2Trace (--trace)                            -> Cis2Model.trace(prompt, gen_toks)
  the seeded-sampling driver (--sample seed,T,K,P; v0.4 draft section 14,
  code/patches/cis2-spec__seeded-sampling.patch:57-196)
                                                -> Cis2Model.set_sampling(...), then decode
Errors surface as Cis2Error (the reference exits with status 2 instead).
"""
import ctypes

import numpy as np

from . import _lib
from ._lib import check


def _u8buf(n):
    return (ctypes.c_uint8 * n)()


def _ptr(arr, ctype):
    return arr.ctypes.data_as(ctype)


class Cis2Model:
    def __init__(self, spec, weights, max_pos, max_seqs=1, reduction_mode=0):
        """reduction_mode 0: sequential order (v0.3b); 1: the v0.4-candidate
        tree order (code/cis2-fp/src/math.rs:60-125, CIS2_REDUCTION_TREE)."""
        L = _lib.lib()
        self.spec = spec
        self.weights = weights
        cfg = _lib.Cis2Config(
            hidden=spec.hidden, inter=spec.inter, n_layers=spec.n_layers,
            n_heads=spec.n_heads, n_kv_heads=spec.n_kv_heads, head_dim=spec.hd,
            vocab=spec.vocab, tied=1 if spec.tied else 0, max_pos=max_pos,
            max_seqs=max_seqs, reduction_mode=reduction_mode, eps=spec.eps, rope_theta=spec.rope_theta)
        h = ctypes.c_void_p()
        check(L.cis2_ctx_create(ctypes.byref(cfg), ctypes.byref(h)))
        self.ctx = h
        self.max_pos = max_pos
        self.max_seqs = max_seqs
        self.reduction_mode = reduction_mode
        for name, _shape, arr in weights.tensors:
            arr = np.ascontiguousarray(arr, dtype=np.uint16)
            check(L.cis2_upload_bf16(self.ctx, name.encode(), _ptr(arr, _lib.c_u16p), arr.size),
                  self.ctx)
        check(L.cis2_check_ready(self.ctx), self.ctx)
        self.hdr = weights.header_digests()

    def close(self):
        if getattr(self, "ctx", None):
            _lib.lib().cis2_ctx_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        self.close()

    def digests(self):
        t, f = _u8buf(32), _u8buf(32)
        check(_lib.lib().cis2_digests(self.ctx, t, f), self.ctx)
        return bytes(t), bytes(f)

    def reset(self, seq=0):
        check(_lib.lib().cis2_reset_seq(self.ctx, seq), self.ctx)

    def profile(self, on):
        """Starts (clearing the record) or stops event timing of every
        persistent-decode kernel launch (cis2_profile)."""
        check(_lib.lib().cis2_profile(self.ctx, 1 if on else 0), self.ctx)

    def profile_read(self, cap=65536):
        """(launches, summed device ms, positions computed) since profile(True)."""
        n = (ctypes.c_uint64 * 1)()
        ms = (ctypes.c_double * 1)()
        pos = np.zeros(cap, dtype=np.uint32)
        check(_lib.lib().cis2_profile_read(self.ctx, n, ms, _ptr(pos, _lib.c_u32p), cap), self.ctx)
        k = int(n[0])
        return k, float(ms[0]), pos[:min(k, cap)].copy()

    def recoveries(self):
        """Steps whose persistent launch hit its bounded wait and were
        recomputed on the per-op path (cis2_recoveries)."""
        n = np.zeros(1, dtype=np.uint32)
        check(_lib.lib().cis2_recoveries(self.ctx, _ptr(n, _lib.c_u32p)), self.ctx)
        return int(n[0])

    def forward_token(self, pos, tok, seq=0):
        """One forward pass; returns (logits float32[vocab], argmax id)."""
        V = self.spec.vocab
        logits = np.empty(V, dtype=np.float32)
        am = np.zeros(1, dtype=np.uint32)
        s = np.array([seq], dtype=np.uint32)
        p = np.array([pos], dtype=np.uint32)
        t = np.array([tok], dtype=np.uint32)
        check(_lib.lib().cis2_forward(self.ctx, 1, _ptr(s, _lib.c_u32p), _ptr(p, _lib.c_u32p),
                                      _ptr(t, _lib.c_u32p), _ptr(logits, _lib.c_fp),
                                      _ptr(am, _lib.c_u32p)), self.ctx)
        return logits, int(am[0])

    def set_sampling(self, seed=None, temperature=1.0, top_k=0, top_p=1.0):
        """Seeded sampling for the following decodes (seed None: greedy).
        temperature and top_p are narrowed to f32 as given (pass the f32
        value, e.g. np.float32(0.8)); invalid values raise Cis2Error."""
        if seed is None:
            sp = _lib.Cis2Sampling(mode=0)
        else:
            sp = _lib.Cis2Sampling(mode=1, top_k=int(top_k), seed=int(seed),
                                   temperature=float(np.float32(temperature)),
                                   top_p=float(np.float32(top_p)))
        check(_lib.lib().cis2_set_sampling(self.ctx, ctypes.byref(sp)), self.ctx)

    def sample_logits(self, logits, steps):
        """Draws with the current sampling parameters from host logit rows
        (float32 [n, vocab]) at the given generation steps; returns (ids,
        kept-set sizes)."""
        lg = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1, self.spec.vocab)
        n = lg.shape[0]
        st = np.ascontiguousarray(steps, dtype=np.uint32).reshape(n)
        ids = np.zeros(n, dtype=np.uint32)
        nk = np.zeros(n, dtype=np.uint32)
        check(_lib.lib().cis2_sample_logits(self.ctx, _ptr(lg, _lib.c_fp), n, _ptr(st, _lib.c_u32p),
                                            _ptr(ids, _lib.c_u32p), _ptr(nk, _lib.c_u32p)),
              self.ctx)
        return ids, nk

    def decode(self, prompt, gen_toks, seq=0, step_digests=True):
        """Greedy (or, after set_sampling, sampled) decode with the witness
        fold; returns a dict with ids, witness, argmax_digest and the
        per-step logit digests."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        n = prompt.size
        ids = np.zeros(n + gen_toks, dtype=np.uint32)
        wit, adg = _u8buf(32), _u8buf(32)
        steps = _u8buf(32 * max(gen_toks, 1)) if step_digests else None
        hdr = (ctypes.c_uint8 * 96).from_buffer_copy(self.hdr)
        check(_lib.lib().cis2_decode(self.ctx, seq, _ptr(prompt, _lib.c_u32p), n, gen_toks, hdr,
                                     _ptr(ids, _lib.c_u32p), wit, adg, steps), self.ctx)
        out = {"ids": ids, "witness": bytes(wit).hex(), "argmax_digest": bytes(adg).hex()}
        if step_digests:
            sb = bytes(steps)
            out["step_digests"] = [sb[32 * i:32 * i + 32].hex() for i in range(gen_toks)]
        return out

    def begin(self, prompt, max_steps, seq=0):
        """Starts a step-wise decode: witness header + prefill."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        self._sess = (prompt.size, max_steps)
        hdr = (ctypes.c_uint8 * 96).from_buffer_copy(self.hdr)
        check(_lib.lib().cis2_decode_begin(self.ctx, seq, _ptr(prompt, _lib.c_u32p), prompt.size,
                                           max_steps, hdr), self.ctx)

    def steps(self, n):
        """n complete greedy steps (argmax, witness fold, forward); blocks."""
        check(_lib.lib().cis2_decode_steps(self.ctx, n), self.ctx)

    def end(self, nsteps):
        n_prompt, _ = self._sess
        ids = np.zeros(n_prompt + nsteps, dtype=np.uint32)
        wit, adg, steps = _u8buf(32), _u8buf(32), _u8buf(32 * max(nsteps, 1))
        check(_lib.lib().cis2_decode_end(self.ctx, _ptr(ids, _lib.c_u32p), wit, adg, steps),
              self.ctx)
        sb = bytes(steps)
        return {"ids": ids, "witness": bytes(wit).hex(), "argmax_digest": bytes(adg).hex(),
                "step_digests": [sb[32 * i:32 * i + 32].hex() for i in range(nsteps)]}

    def decode_batch(self, prompts, gen_toks):
        lens = np.array([len(p) for p in prompts], dtype=np.uint32)
        flat = np.ascontiguousarray(np.concatenate(prompts).astype(np.uint32))
        total = int(lens.sum()) + gen_toks * len(prompts)
        ids = np.zeros(total, dtype=np.uint32)
        wit, adg = _u8buf(32 * len(prompts)), _u8buf(32 * len(prompts))
        hdr = (ctypes.c_uint8 * 96).from_buffer_copy(self.hdr)
        check(_lib.lib().cis2_decode_batch(self.ctx, len(prompts), _ptr(flat, _lib.c_u32p),
                                           _ptr(lens, _lib.c_u32p), gen_toks, hdr,
                                           _ptr(ids, _lib.c_u32p), wit, adg), self.ctx)
        rows, off = [], 0
        wb, ab = bytes(wit), bytes(adg)
        for i, n in enumerate(lens):
            rows.append({"ids": ids[off:off + n + gen_toks].copy(),
                         "witness": wb[32 * i:32 * i + 32].hex(),
                         "argmax_digest": ab[32 * i:32 * i + 32].hex()})
            off += int(n) + gen_toks
        return rows

    def forward_rows(self, seq, pos, tok, want_logits=True):
        """One row-batched pass over rows (seq[i], pos[i], tok[i]); returns
        (logits float32[n][vocab] or None, argmax ids uint32[n])."""
        seq = np.ascontiguousarray(seq, dtype=np.uint32)
        pos = np.ascontiguousarray(pos, dtype=np.uint32)
        tok = np.ascontiguousarray(tok, dtype=np.uint32)
        n = seq.size
        logits = np.empty((n, self.spec.vocab), dtype=np.float32) if want_logits else None
        am = np.zeros(n, dtype=np.uint32)
        check(_lib.lib().cis2_forward(self.ctx, n, _ptr(seq, _lib.c_u32p), _ptr(pos, _lib.c_u32p),
                                      _ptr(tok, _lib.c_u32p),
                                      _ptr(logits, _lib.c_fp) if want_logits else None,
                                      _ptr(am, _lib.c_u32p)), self.ctx)
        return logits, am

    def verify_prefill(self, prompt, claimed, seq=0, want_logits=False):
        """Teacher-forced check of a claimed continuation in one pass
        (cis2_verify_prefill): ids argmax'd at each claimed position, the
        witness / argmax digest they give, and the first mismatch (-1)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        claimed = np.ascontiguousarray(claimed, dtype=np.uint32)
        n_gen = claimed.size
        gen = np.zeros(max(n_gen, 1), dtype=np.uint32)
        wit, adg = _u8buf(32), _u8buf(32)
        fm = ctypes.c_int64()
        logits = np.empty((n_gen, self.spec.vocab), dtype=np.float32) if want_logits else None
        hdr = (ctypes.c_uint8 * 96).from_buffer_copy(self.hdr)
        check(_lib.lib().cis2_verify_prefill(
            self.ctx, seq, _ptr(prompt, _lib.c_u32p), prompt.size, _ptr(claimed, _lib.c_u32p),
            n_gen, hdr, _ptr(gen, _lib.c_u32p), wit, adg, ctypes.byref(fm),
            _ptr(logits, _lib.c_fp) if want_logits else None), self.ctx)
        out = {"generated": gen[:n_gen].copy(), "witness": bytes(wit).hex(),
               "argmax_digest": bytes(adg).hex(), "first_mismatch": int(fm.value)}
        if want_logits:
            out["logits"] = logits
        return out

    def trace(self, prompt, gen_toks):
        """Decode with per-op tracing; returns (decode result, trace lines in
        the reference's `pos=.. layer=.. op=.. sha256=..` format)."""
        lines = []

        def cb(pos, layer, op, sha, _user):
            lines.append("pos=%d layer=%d op=%s sha256=%s" % (
                pos, layer, op.decode(), bytes(sha[:32]).hex()))

        fn = _lib.TRACE_FN(cb)
        check(_lib.lib().cis2_trace_enable(self.ctx, fn, None), self.ctx)
        try:
            res = self.decode(prompt, gen_toks)
        finally:
            _lib.lib().cis2_trace_enable(self.ctx, _lib.TRACE_FN(), None)
        return res, lines


class GemvPlan:
    """Standalone pinned-order GEMV y = W x on the device (the 4-row
    interleaved reference kernel of labs/rust-5; bits of dot_seq)."""

    def __init__(self, W, copies=1):
        W = np.ascontiguousarray(W, dtype=np.float32)
        self.M, self.K = W.shape
        h = ctypes.c_void_p()
        check(_lib.lib().cis2_gemv_plan_create(self.M, self.K, copies, _ptr(W, _lib.c_fp),
                                               ctypes.byref(h)))
        self.plan = h
        self.copies = copies

    def __call__(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(self.M, dtype=np.float32)
        check(_lib.lib().cis2_gemv_plan_run(self.plan, _ptr(x, _lib.c_fp), _ptr(y, _lib.c_fp)))
        return y

    def time(self, iters):
        ms = ctypes.c_float()
        check(_lib.lib().cis2_gemv_plan_time(self.plan, iters, ctypes.byref(ms)))
        return ms.value

    def run_batch(self, X):
        """n independent GEMVs in one launch: row i of the result is
        W_(i mod copies) X[i]."""
        X = np.ascontiguousarray(X, dtype=np.float32)
        n = X.shape[0]
        assert X.shape == (n, self.K)
        Y = np.empty((n, self.M), dtype=np.float32)
        check(_lib.lib().cis2_gemv_plan_run_batch(self.plan, n, _ptr(X, _lib.c_fp),
                                                  _ptr(Y, _lib.c_fp)))
        return Y

    def time_batch(self, n, iters):
        """Mean ms per launch of n GEMVs (device-resident inputs)."""
        ms = ctypes.c_float()
        check(_lib.lib().cis2_gemv_plan_time_batch(self.plan, n, iters, ctypes.byref(ms)))
        return ms.value

    def close(self):
        if getattr(self, "plan", None):
            _lib.lib().cis2_gemv_plan_destroy(self.plan)
            self.plan = None

    def __del__(self):
        self.close()


FN_IDS = {"exp": 0, "sin": 1, "cos": 2, "ln": 3, "silu": 4, "rsqrt": 5, "sqrt": 6}


def device_math(fn, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    check(_lib.lib().cis2_math_map(FN_IDS[fn], _ptr(x, _lib.c_fp), _ptr(out, _lib.c_fp), x.size))
    return out


def device_div(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty_like(a)
    check(_lib.lib().cis2_div_map(_ptr(a, _lib.c_fp), _ptr(b, _lib.c_fp), _ptr(out, _lib.c_fp),
                                  a.size))
    return out


def device_math_chunk_hashes(fn, c0=0, nchunks=256):
    out = np.zeros(nchunks, dtype=np.uint64)
    check(_lib.lib().cis2_math_chunk_hashes(FN_IDS[fn], c0, nchunks, _ptr(out, _lib.c_u64p)))
    return out


def fpenv_probe():
    out = np.zeros(2, dtype=np.uint32)
    check(_lib.lib().cis2_fpenv_probe(_ptr(out, _lib.c_u32p)))
    return int(out[0]), int(out[1])


def wait_probe():
    """(wrong registers after 128 vector loads and one vmcnt(0) wait, wrong
    words after 40 LDS reads and one lgkmcnt(0) wait): cis2_wait_probe."""
    out = np.zeros(2, dtype=np.uint32)
    check(_lib.lib().cis2_wait_probe(_ptr(out, _lib.c_u32p)))
    return int(out[0]), int(out[1])


def sha256(data):
    buf = bytes(data)
    out = _u8buf(32)
    _lib.lib().cis2_sha256(buf, len(buf), out)
    return bytes(out)
