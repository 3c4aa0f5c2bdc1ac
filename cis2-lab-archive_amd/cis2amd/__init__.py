"""cis2amd — host-side mirror of the CIS-2 forward-pass interface over the
gfx950 C ABI (include/cis2_amd.h, lib/libcis2amd.so).

The Python layer is plumbing for tests and benchmarks: every forward pass,
GEMV and pinned-math evaluation runs in the HIP library.
"""
from . import _lib
from ._lib import Cis2Error
from .artifacts import SPECS, ModelSpec, Weights, prompt_ids, tensor_list
from .model import Cis2Model, GemvPlan, device_math, device_math_chunk_hashes, fpenv_probe, sha256

__all__ = ["Cis2Error", "Cis2Model", "GemvPlan", "ModelSpec", "SPECS", "Weights",
           "device_math", "device_math_chunk_hashes", "fpenv_probe", "prompt_ids", "sha256",
           "tensor_list", "_lib"]
