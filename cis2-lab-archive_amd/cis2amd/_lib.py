"""ctypes bindings of include/cis2_amd.h (lib/libcis2amd.so) and of the
synthetic-artifact generator (lib/libcis2synth.so).

The HIP library is the product: there is no CPU fallback.  If the shared
library is missing, loading fails with an error that says how to build it.
"""
import ctypes
import os

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libcis2amd.so")
SYNTH_PATH = os.path.join(LIB_DIR, "libcis2synth.so")

c_u8p = ctypes.POINTER(ctypes.c_uint8)
c_u16p = ctypes.POINTER(ctypes.c_uint16)
c_u32p = ctypes.POINTER(ctypes.c_uint32)
c_u64p = ctypes.POINTER(ctypes.c_uint64)
c_fp = ctypes.POINTER(ctypes.c_float)

CIS2_OK = 0
ERRORS = {
    -1: "CIS2_E_ARG", -2: "CIS2_E_UNSUPPORTED", -3: "CIS2_E_MISSING_TENSOR",
    -4: "CIS2_E_SHAPE", -5: "CIS2_E_NAME", -6: "CIS2_E_FPENV", -7: "CIS2_E_DEVICE",
    -8: "CIS2_E_OOM", -9: "CIS2_E_RANGE", -10: "CIS2_E_NUMERIC",
}


class Cis2Config(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_uint32), ("inter", ctypes.c_uint32),
        ("n_layers", ctypes.c_uint32), ("n_heads", ctypes.c_uint32),
        ("n_kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
        ("vocab", ctypes.c_uint32), ("tied", ctypes.c_uint32),
        ("max_pos", ctypes.c_uint32), ("max_seqs", ctypes.c_uint32),
        ("reduction_mode", ctypes.c_uint32), ("eps", ctypes.c_float),
        ("rope_theta", ctypes.c_double),
    ]


class Cis2Sampling(ctypes.Structure):
    _fields_ = [
        ("mode", ctypes.c_uint32), ("top_k", ctypes.c_uint32), ("seed", ctypes.c_uint64),
        ("temperature", ctypes.c_float), ("top_p", ctypes.c_float),
    ]


TRACE_FN = ctypes.CFUNCTYPE(None, ctypes.c_int, ctypes.c_int, ctypes.c_char_p, c_u8p,
                            ctypes.c_void_p)

# name -> (restype, argtypes); every symbol declared in include/cis2_amd.h
SIGNATURES = {
    "cis2_ctx_create": (ctypes.c_int, [ctypes.POINTER(Cis2Config), ctypes.POINTER(ctypes.c_void_p)]),
    "cis2_ctx_destroy": (None, [ctypes.c_void_p]),
    "cis2_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "cis2_last_error": (ctypes.c_char_p, [ctypes.c_void_p]),
    "cis2_upload_bf16": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, c_u16p, ctypes.c_uint64]),
    "cis2_check_ready": (ctypes.c_int, [ctypes.c_void_p]),
    "cis2_digests": (ctypes.c_int, [ctypes.c_void_p, c_u8p, c_u8p]),
    "cis2_reset_seq": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32]),
    "cis2_forward": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, c_u32p, c_u32p, c_u32p,
                                    c_fp, c_u32p]),
    "cis2_decode": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, c_u32p, ctypes.c_uint32,
                                   ctypes.c_uint32, c_u8p, c_u32p, c_u8p, c_u8p, c_u8p]),
    "cis2_decode_begin": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, c_u32p, ctypes.c_uint32,
                                         ctypes.c_uint32, c_u8p]),
    "cis2_decode_steps": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32]),
    "cis2_decode_end": (ctypes.c_int, [ctypes.c_void_p, c_u32p, c_u8p, c_u8p, c_u8p]),
    "cis2_decode_batch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, c_u32p, c_u32p,
                                         ctypes.c_uint32, c_u8p, c_u32p, c_u8p, c_u8p]),
    "cis2_verify_prefill": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, c_u32p, ctypes.c_uint32,
                                           c_u32p, ctypes.c_uint32, c_u8p, c_u32p, c_u8p, c_u8p,
                                           ctypes.POINTER(ctypes.c_int64), c_fp]),
    "cis2_set_sampling": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(Cis2Sampling)]),
    "cis2_sample_logits": (ctypes.c_int, [ctypes.c_void_p, c_fp, ctypes.c_uint32, c_u32p, c_u32p,
                                          c_u32p]),
    "cis2_sample_logits_noalloc": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32,
                                                  c_u32p, ctypes.c_void_p, ctypes.c_void_p]),
    "cis2_trace_enable": (ctypes.c_int, [ctypes.c_void_p, TRACE_FN, ctypes.c_void_p]),
    "cis2_profile": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "cis2_profile_read": (ctypes.c_int, [ctypes.c_void_p, c_u64p, ctypes.POINTER(ctypes.c_double),
                                         c_u32p, ctypes.c_uint64]),
    "cis2_recoveries": (ctypes.c_int, [ctypes.c_void_p, c_u32p]),
    "cis2_gemv_plan_create": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                             c_fp, ctypes.POINTER(ctypes.c_void_p)]),
    "cis2_gemv_plan_run": (ctypes.c_int, [ctypes.c_void_p, c_fp, c_fp]),
    "cis2_gemv_plan_time": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, c_fp]),
    "cis2_gemv_plan_run_batch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, c_fp, c_fp]),
    "cis2_gemv_plan_time_batch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32,
                                                 ctypes.c_uint32, c_fp]),
    "cis2_gemv_plan_destroy": (None, [ctypes.c_void_p]),
    "cis2_sha256": (None, [ctypes.c_void_p, ctypes.c_uint64, c_u8p]),
    "cis2_math_map": (ctypes.c_int, [ctypes.c_int, c_fp, c_fp, ctypes.c_uint64]),
    "cis2_math_chunk_hashes": (ctypes.c_int, [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32, c_u64p]),
    "cis2_div_map": (ctypes.c_int, [c_fp, c_fp, c_fp, ctypes.c_uint64]),
    "cis2_fpenv_probe": (ctypes.c_int, [c_u32p]),
    "cis2_wait_probe": (ctypes.c_int, [c_u32p]),
}

_lib = None
_synth = None


class Cis2Error(RuntimeError):
    def __init__(self, code, msg=""):
        self.code = code
        super().__init__("%s (%d)%s" % (ERRORS.get(code, "CIS2_E_?"), code,
                                         (": " + msg) if msg else ""))


def lib():
    """Loads lib/libcis2amd.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("libcis2amd.so not built: run `make -C cis2-lab-archive_amd` "
                               "(or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def synth():
    global _synth
    if _synth is None:
        if not os.path.exists(SYNTH_PATH):
            raise RuntimeError("libcis2synth.so not built: run `make -C cis2-lab-archive_amd`")
        S = ctypes.CDLL(SYNTH_PATH)
        S.cis2_synth_bf16.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double, c_u16p, ctypes.c_uint64]
        S.cis2_synth_f32.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double, c_fp, ctypes.c_uint64]
        S.cis2_synth_uniform.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32,
                                         ctypes.c_uint32, c_u32p, ctypes.c_uint64]
        S.cis2_synth_mix64.restype = ctypes.c_uint64
        S.cis2_synth_mix64.argtypes = [ctypes.c_uint64]
        _synth = S
    return _synth


def check(code, ctx=None):
    if code != CIS2_OK:
        msg = ""
        if ctx:
            m = lib().cis2_last_error(ctx)
            msg = m.decode() if m else ""
        raise Cis2Error(code, msg)
