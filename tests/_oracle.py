"""ctypes wrapper of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE: the oracle produces the expected bits.  Only tests/,
the smoke() entry point and bench.py's cpu_baseline leg load it.
"""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
REF_MATH_PATH = os.path.join(ROOT, "oracle", "_ref", "libref_math.so")

c_u8p = ctypes.POINTER(ctypes.c_uint8)
c_u16p = ctypes.POINTER(ctypes.c_uint16)
c_u32p = ctypes.POINTER(ctypes.c_uint32)
c_fp = ctypes.POINTER(ctypes.c_float)

FN_IDS = {"exp": 0, "sin": 1, "cos": 2, "ln": 3, "silu": 4, "rsqrt": 5, "sqrt": 6}


class OrcConfig(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("inter", ctypes.c_int), ("n_layers", ctypes.c_int),
                ("n_heads", ctypes.c_int), ("n_kv_heads", ctypes.c_int),
                ("head_dim", ctypes.c_int), ("vocab", ctypes.c_int), ("tied", ctypes.c_int),
                ("max_pos", ctypes.c_int), ("reduction", ctypes.c_int),
                ("threads", ctypes.c_int), ("eps", ctypes.c_float),
                ("rope_theta", ctypes.c_double)]


TRACE_FN = ctypes.CFUNCTYPE(None, ctypes.c_int, ctypes.c_int, ctypes.c_char_p, c_u8p,
                            ctypes.c_void_p)

_o = None


def lib():
    global _o
    if _o is None:
        if not os.path.exists(ORACLE_PATH):
            raise RuntimeError("oracle not built: make -C oracle")
        L = ctypes.CDLL(ORACLE_PATH)
        for n in ["orc_exp", "orc_sin", "orc_cos", "orc_ln", "orc_silu", "orc_rsqrt", "orc_sqrt"]:
            getattr(L, n).restype = ctypes.c_float
            getattr(L, n).argtypes = [ctypes.c_float]
        L.orc_math_map.argtypes = [ctypes.c_int, c_fp, c_fp, ctypes.c_size_t]
        L.orc_div_map.argtypes = [c_fp, c_fp, c_fp, ctypes.c_size_t]
        L.orc_math_chunk_hash.restype = ctypes.c_uint64
        L.orc_math_chunk_hash.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32]
        for n in ["orc_dot_seq", "orc_dot_tree"]:
            getattr(L, n).restype = ctypes.c_float
            getattr(L, n).argtypes = [c_fp, c_fp, ctypes.c_int]
        for n in ["orc_sum_seq", "orc_sum_tree"]:
            getattr(L, n).restype = ctypes.c_float
            getattr(L, n).argtypes = [c_fp, ctypes.c_int]
        L.orc_gemv.argtypes = [c_fp, c_fp, c_fp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                               ctypes.c_int]
        L.orc_softmax.argtypes = [c_fp, ctypes.c_int, ctypes.c_int]
        L.orc_argmax.restype = ctypes.c_uint32
        L.orc_argmax.argtypes = [c_fp, ctypes.c_int]
        L.orc_sha256.argtypes = [ctypes.c_void_p, ctypes.c_size_t, c_u8p]
        L.orc_table_digest.argtypes = [c_u8p]
        L.orc_inv_freq.argtypes = [ctypes.c_double, ctypes.c_int, c_fp, c_u8p]
        L.orc_model_create.restype = ctypes.c_void_p
        L.orc_model_create.argtypes = [ctypes.POINTER(OrcConfig)]
        L.orc_model_destroy.argtypes = [ctypes.c_void_p]
        L.orc_model_set_bf16.argtypes = [ctypes.c_void_p, ctypes.c_char_p, c_u16p, ctypes.c_size_t]
        L.orc_model_digests.argtypes = [ctypes.c_void_p, c_u8p, c_u8p]
        L.orc_forward.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, c_fp,
                                  TRACE_FN, ctypes.c_void_p]
        L.orc_murmur3_32.restype = ctypes.c_uint32
        L.orc_murmur3_32.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32]
        L.orc_sample_noise.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, c_u32p,
                                       c_fp, c_fp]
        L.orc_sample_params_ok.argtypes = [ctypes.c_float, ctypes.c_uint32, ctypes.c_float]
        L.orc_sample.restype = ctypes.c_uint32
        L.orc_sample.argtypes = [c_fp, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint32,
                                 ctypes.c_float, ctypes.c_uint32, ctypes.c_float, c_fp, c_u32p]
        L.orc_decode_sampled.argtypes = [ctypes.c_void_p, c_u32p, ctypes.c_int, ctypes.c_int, c_u8p,
                                         ctypes.c_uint64, ctypes.c_float, ctypes.c_uint32,
                                         ctypes.c_float, c_u32p, c_u8p, c_u8p, c_u8p]
        L.orc_decode.argtypes = [ctypes.c_void_p, c_u32p, ctypes.c_int, ctypes.c_int, c_u8p,
                                 c_u32p, c_u8p, c_u8p, c_u8p, TRACE_FN, ctypes.c_void_p]
        L.orc_fpenv_pin.restype = ctypes.c_int
        L.orc_model_hidden.argtypes = [ctypes.c_void_p, c_fp]
        L.orc_set_mutation.argtypes = [ctypes.c_int]
        _o = L
        if L.orc_fpenv_pin() != 0:
            raise RuntimeError("oracle FTZ/DAZ pin failed")
    return _o


def fpenv_release():
    """Give the calling thread back the default FP environment (subnormals
    kept) if the oracle pinned FTZ|DAZ on it; returns whether it had."""
    if _o is None:
        return False
    _o.orc_fpenv_release()
    return True


def fpenv_repin():
    if _o is not None and _o.orc_fpenv_pin() != 0:
        raise RuntimeError("oracle FTZ/DAZ pin failed")


def ref_math():
    """The reference's own cis2_math.h compiled here (None if not built)."""
    if not os.path.exists(REF_MATH_PATH):
        return None
    R = ctypes.CDLL(REF_MATH_PATH)
    R.ref_math_map.argtypes = [ctypes.c_int, c_fp, c_fp, ctypes.c_size_t]
    R.ref_math_chunk_hash.restype = ctypes.c_uint64
    R.ref_math_chunk_hash.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32]
    for n in ["ref_dot_seq", "ref_dot_tree"]:
        getattr(R, n).restype = ctypes.c_float
        getattr(R, n).argtypes = [c_fp, c_fp, ctypes.c_int]
    R.ref_sum_tree.restype = ctypes.c_float
    R.ref_sum_tree.argtypes = [c_fp, ctypes.c_int]
    R.ref_softmax.argtypes = [c_fp, ctypes.c_int, ctypes.c_int]
    return R


def ptr(a, t):
    return a.ctypes.data_as(t)


def math_map(fn, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_math_map(FN_IDS[fn], ptr(x, c_fp), ptr(out, c_fp), x.size)
    return out


def div_map(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty_like(a)
    lib().orc_div_map(ptr(a, c_fp), ptr(b, c_fp), ptr(out, c_fp), a.size)
    return out


def gemv(W, x, mode=0, threads=8):
    W = np.ascontiguousarray(W, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = W.shape
    y = np.empty(M, dtype=np.float32)
    lib().orc_gemv(ptr(W, c_fp), ptr(x, c_fp), ptr(y, c_fp), M, K, mode, threads)
    return y


def table_digest():
    b = (ctypes.c_uint8 * 32)()
    lib().orc_table_digest(b)
    return bytes(b).hex()


def inv_freq(theta, hd):
    out = np.empty(hd // 2, dtype=np.float32)
    d = (ctypes.c_uint8 * 32)()
    lib().orc_inv_freq(theta, hd, ptr(out, c_fp), d)
    return out, bytes(d).hex()


class OracleModel:
    """The oracle's forward/decode over the same seeded weights."""

    def __init__(self, spec, weights, max_pos, threads=8, reduction=0):
        L = lib()
        cfg = OrcConfig(hidden=spec.hidden, inter=spec.inter, n_layers=spec.n_layers,
                        n_heads=spec.n_heads, n_kv_heads=spec.n_kv_heads, head_dim=spec.hd,
                        vocab=spec.vocab, tied=1 if spec.tied else 0, max_pos=max_pos,
                        reduction=reduction, threads=threads, eps=spec.eps,
                        rope_theta=spec.rope_theta)
        self.m = L.orc_model_create(ctypes.byref(cfg))
        self.spec = spec
        for name, _shape, arr in weights.tensors:
            rc = L.orc_model_set_bf16(self.m, name.encode(), ptr(arr, c_u16p), arr.size)
            if rc != 0:
                raise RuntimeError("oracle rejected %s (%d)" % (name, rc))
        self.hdr = weights.header_digests()

    def __del__(self):
        if getattr(self, "m", None):
            lib().orc_model_destroy(self.m)
            self.m = None

    def digests(self):
        t, f = (ctypes.c_uint8 * 32)(), (ctypes.c_uint8 * 32)()
        lib().orc_model_digests(self.m, t, f)
        return bytes(t).hex(), bytes(f).hex()

    def forward(self, pos, tok):
        """One forward pass at `pos` (positions are filled in order by the
        caller); returns the logits."""
        logits = np.empty(self.spec.vocab, dtype=np.float32)
        rc = lib().orc_forward(self.m, int(pos), int(tok), ptr(logits, c_fp), TRACE_FN(), None)
        if rc != 0:
            raise RuntimeError("oracle forward failed (%d)" % rc)
        return logits

    def hidden(self):
        """The final-norm output of the last forward (the LM head's input)."""
        out = np.empty(self.spec.hidden, dtype=np.float32)
        if lib().orc_model_hidden(self.m, ptr(out, c_fp)) != 0:
            raise RuntimeError("no forward has run")
        return out

    def decode_sampled(self, prompt, gen_toks, seed, temperature, top_k, top_p):
        """The sampled decode of draft section 14 (orc_decode_sampled)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        ids = np.zeros(prompt.size + gen_toks, dtype=np.uint32)
        wit, adg = (ctypes.c_uint8 * 32)(), (ctypes.c_uint8 * 32)()
        steps = (ctypes.c_uint8 * (32 * max(gen_toks, 1)))()
        hdr = (ctypes.c_uint8 * 96).from_buffer_copy(self.hdr)
        rc = lib().orc_decode_sampled(self.m, ptr(prompt, c_u32p), prompt.size, gen_toks, hdr,
                                      int(seed), float(np.float32(temperature)), int(top_k),
                                      float(np.float32(top_p)), ptr(ids, c_u32p), wit, adg, steps)
        if rc != 0:
            raise RuntimeError("oracle sampled decode failed (%d)" % rc)
        sb = bytes(steps)
        return {"ids": ids, "witness": bytes(wit).hex(), "argmax_digest": bytes(adg).hex(),
                "step_digests": [sb[32 * i:32 * i + 32].hex() for i in range(gen_toks)]}

    def decode(self, prompt, gen_toks, trace=None):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        ids = np.zeros(prompt.size + gen_toks, dtype=np.uint32)
        wit, adg = (ctypes.c_uint8 * 32)(), (ctypes.c_uint8 * 32)()
        steps = (ctypes.c_uint8 * (32 * max(gen_toks, 1)))()
        hdr = (ctypes.c_uint8 * 96).from_buffer_copy(self.hdr)
        cb = TRACE_FN()
        if trace is not None:
            def _cb(pos, layer, op, sha, _u):
                trace.append("pos=%d layer=%d op=%s sha256=%s" % (
                    pos, layer, op.decode(), bytes(sha[:32]).hex()))
            cb = TRACE_FN(_cb)
        rc = lib().orc_decode(self.m, ptr(prompt, c_u32p), prompt.size, gen_toks, hdr,
                              ptr(ids, c_u32p), wit, adg, steps, cb, None)
        if rc != 0:
            raise RuntimeError("oracle decode failed (%d)" % rc)
        sb = bytes(steps)
        return {"ids": ids, "witness": bytes(wit).hex(), "argmax_digest": bytes(adg).hex(),
                "step_digests": [sb[32 * i:32 * i + 32].hex() for i in range(gen_toks)]}


MUT_ARGMAX_GE = 1  # greedy argmax with >= (the last maximum wins)
MUT_NO_FTZ = 2     # FTZ/DAZ left off


class mutation:
    """Context manager: runs the oracle with a planted mistake (a test that
    shows a fixture detects it), and restores the specified oracle after."""

    def __init__(self, m):
        self.m = m

    def __enter__(self):
        lib().orc_set_mutation(self.m)
        return self

    def __exit__(self, *exc):
        lib().orc_set_mutation(0)
        if lib().orc_fpenv_pin() != 0:
            raise RuntimeError("oracle FTZ/DAZ pin failed")
        return False


def sample_noise(seed, step, index):
    """(hash, u, g) of draft 14.2 from the oracle."""
    h = (ctypes.c_uint32 * 1)()
    u = (ctypes.c_float * 1)()
    g = (ctypes.c_float * 1)()
    lib().orc_sample_noise(int(seed), int(step), int(index), h, u, g)
    return int(h[0]), float(u[0]), float(g[0])


def sample(logits, seed, step, temperature, top_k, top_p):
    """(next_id, z[V], kept-set size) of draft 14.3-14.4 from the oracle;
    next_id is None for invalid parameters or NaN scaled logits."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    z = np.empty(lg.size, dtype=np.float32)
    nk = (ctypes.c_uint32 * 1)()
    r = lib().orc_sample(ptr(lg, c_fp), lg.size, int(seed), int(step),
                         float(np.float32(temperature)), int(top_k), float(np.float32(top_p)),
                         ptr(z, c_fp), nk)
    return (None if r == 0xFFFFFFFF else int(r)), z, int(nk[0])
