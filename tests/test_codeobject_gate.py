"""Numerics gate on the gfx950 code objects built here (the CIS-2 build
contract, code/cis2-fp/gpu/Makefile:252-313: no FMA on the arithmetic path,
no hardware transcendentals; spec 1.4-1.6).  The device code of every
library object is unbundled and disassembled with the ROCm LLVM tools, and
each kernel is checked:

  - no hardware transcendental or approximate op: v_exp/v_log/v_sin/v_cos,
    their legacy forms, v_sqrt_f32, legacy rcp/rsq;
  - no packed or mixed FP32 arithmetic (v_pk_add/mul/fma_f32, v_fma_mix*),
    no non-IEEE multiply-add (v_mad_f32, v_mac_f32, legacy fma), no dot ops;
  - every f32 FMA belongs to a correctly rounded divide (v_div_scale x2,
    v_rcp, 5 FMAs, v_div_fmas, v_div_fixup) or square root (v_rsq + 5
    FMAs), every f64 FMA to an f64 divide (5 FMAs) -- counted exactly;
    the only others allowed are the compiler's integer sequences (64-bit
    unsigned division's float estimate, corrected in integers: a v_mul by
    0x5f7ffffc, FMAs with a +-2^32 literal or a zero multiplicand; the f64 ->
    integer split with a -2^32 literal), which carry no float data;
  - the pure reduction kernels (the standalone GEMVs, the per-op GEMV, the
    row GEMMs without norm or gate) contain no FMA and no divide at all;
  - no scalar-cache writes of any kind (stores, atomics, write-back).

The per-kernel FMA accounting is printed (pytest -s)."""
import collections
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OBJ = os.path.join(ROOT, "cis2-lab-archive_amd", "obj")
LLVM = "/opt/rocm/llvm/bin"
OBJECTS = ["cis2_kernels", "cis2_decode", "cis2_rows", "cis2_sample"]

FORBIDDEN = re.compile(
    r"^(v_(exp|log|sin|cos)(_legacy)?_f(16|32|64)|v_sqrt_f(16|32|64)|v_rcp_legacy_f32|"
    r"v_rsq_legacy_f32|v_pk_(add|mul|fma)_f32|v_fma_mix\w*|v_mad_f32|v_mac_f32|"
    r"v_mad_legacy_f32|v_fma_legacy_f32|v_fmac_legacy_f32|v_dot\w*|"
    r"s_(buffer_)?store\w*|s_scratch_store\w*|s_(buffer_)?atomic\w*|s_dcache_wb\w*|"
    r"s_dcache_discard\w*)$")
FMA32 = re.compile(r"^v_fma(c|ak|mk)?_f32$")
FMA64 = re.compile(r"^v_fma(c)?_f64$")
# integer sequences: +-2^32 as an f32 literal, or as the high word of an f64
INT_LIT32 = re.compile(r"0x[4c]f800000\b")
INT_LIT64 = re.compile(r"0x[4c]1f00000\b")
STRICT_ZERO = re.compile(r"(k_gemv_blk|k_gemv_pipe|k_gemv_many|4cis26k_gemvE|k_bgemmILb0ELb0E|k_bgemm16ILb0ELb0E)")


def tools():
    for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump"):
        if not os.path.exists(os.path.join(LLVM, t)):
            pytest.skip("ROCm LLVM tools not found")


def disassemble(name, tmp):
    src = os.path.join(OBJ, name + ".o")
    if not os.path.exists(src):
        pytest.skip("library not built")
    fat, host, co = (os.path.join(tmp, name + s) for s in (".fat", ".host", ".co"))
    subprocess.run([os.path.join(LLVM, "llvm-objcopy"), "--dump-section", ".hip_fatbin=" + fat,
                    src, host], check=True, capture_output=True)
    subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o",
                    "--input=" + fat, "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    "--output=" + co], check=True, capture_output=True)
    r = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--mcpu=gfx950", co],
                       check=True, capture_output=True, text=True)
    return r.stdout


def kernels(asm):
    """{function: [(mnemonic without encoding suffix, operand text)]}"""
    out = collections.defaultdict(list)
    fn = None
    for line in asm.splitlines():
        m = re.match(r"^[0-9a-f]+ <(.*)>:$", line)
        if m:
            fn = m.group(1)
            continue
        t = line.split("//")[0].strip()
        if not t or fn is None:
            continue
        op, _, rest = t.partition(" ")
        out[fn].append((re.sub(r"_(e32|e64|sdwa|dpp)$", "", op), rest))
    return out


def account(ins):
    c = collections.Counter(op for op, _ in ins)
    fma32 = [(op, a) for op, a in ins if FMA32.match(op)]
    fma64 = [(op, a) for op, a in ins if FMA64.match(op)]
    int32 = sum(1 for _, a in fma32 if INT_LIT32.search(a) or re.search(r",\s*0,", a + ","))
    int64 = sum(1 for _, a in fma64 if INT_LIT64.search(a))
    udiv = sum(1 for op, a in ins if op == "v_mul_f32" and "0x5f7ffffc" in a)
    return {
        "fma32": len(fma32), "fma64": len(fma64), "int_fma32": int32, "int_fma64": int64,
        "div32": c["v_div_fixup_f32"], "sqrt32": c["v_rsq_f32"], "div64": c["v_div_fixup_f64"],
        "rcp32": c["v_rcp_f32"], "rcp64": c["v_rcp_f64"], "udiv64": udiv,
        "div_scale32": c["v_div_scale_f32"], "div_fmas32": c["v_div_fmas_f32"],
        "forbidden": sorted({op for op in c if FORBIDDEN.match(op)}),
    }


@pytest.fixture(scope="module")
def code(tmp_path_factory):
    tools()
    tmp = str(tmp_path_factory.mktemp("co"))
    return {name: kernels(disassemble(name, tmp)) for name in OBJECTS}


def test_every_object_has_kernels(code):
    for name in OBJECTS:
        assert code[name], name
    assert any("k_decode" in f for f in code["cis2_decode"])


def test_no_forbidden_instructions(code):
    bad = {f: account(ins)["forbidden"] for obj in code.values() for f, ins in obj.items()}
    bad = {f: v for f, v in bad.items() if v}
    assert not bad, bad


def test_fma_only_in_divide_and_sqrt_expansions(code):
    lines, bad = [], []
    for name in OBJECTS:
        for f, ins in sorted(code[name].items()):
            a = account(ins)
            expect32 = 5 * a["div32"] + 5 * a["sqrt32"] + a["int_fma32"]
            expect64 = 5 * a["div64"] + a["int_fma64"]
            ok = (a["fma32"] == expect32 and a["fma64"] == expect64 and
                  a["rcp32"] == a["div32"] + a["udiv64"] and a["rcp64"] == a["div64"] and
                  a["div_scale32"] == 2 * a["div32"] and a["div_fmas32"] == a["div32"])
            if a["fma32"] or a["fma64"]:
                lines.append("%-70s f32 FMA %3d = 5 x %d div + 5 x %d sqrt + %d int; "
                             "f64 FMA %2d = 5 x %d div + %d int" % (
                                 f[:70], a["fma32"], a["div32"], a["sqrt32"], a["int_fma32"],
                                 a["fma64"], a["div64"], a["int_fma64"]))
            if not ok:
                bad.append((f, a))
    print("\n".join(lines))
    assert not bad, bad


def test_no_kernel_spills_vector_registers(tmp_path):
    """Every kernel keeps its values in registers: no VGPR spills to scratch
    (code-object metadata .vgpr_spill_count).  Spill code is where this
    compiler was caught reloading a partly spilled register tuple into the
    wrong register, and a chain kernel fully unrolled under register
    pressure is what spills."""
    tools()
    bad = []
    for name in OBJECTS:
        disassemble(name, str(tmp_path))  # unbundles <name>.co into tmp_path
        co = os.path.join(str(tmp_path), name + ".co")
        r = subprocess.run([os.path.join(LLVM, "llvm-readelf"), "--notes", co], check=True,
                           capture_output=True, text=True)
        kern = None
        for line in r.stdout.splitlines():
            m = re.match(r"\s*\.name:\s+(\S+)", line)
            if m:
                kern = m.group(1)
            m = re.match(r"\s*\.vgpr_spill_count:\s+(\d+)", line)
            if m and int(m.group(1)) != 0:
                bad.append((name, kern, int(m.group(1))))
    assert not bad, bad


def test_wait_probes_issue_every_load_before_one_wait(code):
    """The wait-counter probes (cis2_wait_probe) test the hardware only if
    the built code issues all 128 vector loads (40 LDS reads) back to back,
    waits once, and never copies or spills a destination register before
    that wait (such a copy would read the register before its load lands)."""
    fns = code["cis2_kernels"]
    for tag, load, wait, n in (("k_probe_vm", "global_load_dword", "vmcnt(0)", 128),
                               ("k_probe_lds", "ds_read_b128", "lgkmcnt(0)", 40)):
        name = [f for f in fns if tag in f]
        assert len(name) == 1, tag
        ins = fns[name[0]]
        first = next(i for i, (op, _) in enumerate(ins) if op == load)
        end = next(i for i, (op, a) in enumerate(ins) if i > first and op == "s_waitcnt")
        assert wait in ins[end][1], (tag, ins[end])
        between = ins[first:end]
        assert [op for op, _ in between].count(load) == n, tag

        def regs(text):
            out = set()
            for a, b in re.findall(r"\bv\[(\d+):(\d+)\]", text):
                out.update(range(int(a), int(b) + 1))
            out.update(int(r) for r in re.findall(r"\bv(\d+)\b", text))
            return out

        dest = set()
        for op, a in between:
            if op == load:
                dest |= regs(a.split(",")[0])
        for op, a in between:
            if op != load:  # nothing reads, copies or overwrites a register in flight
                assert not (regs(a) & dest), (tag, op, a)
        assert not any(op.startswith(("scratch_", "v_accvgpr")) for op, _ in ins), tag


def test_pure_reduction_kernels_have_no_fma(code):
    seen = 0
    for obj in code.values():
        for f, ins in obj.items():
            if STRICT_ZERO.search(f):
                seen += 1
                a = account(ins)
                assert a["fma32"] == a["fma64"] == 0 and a["div32"] == a["div64"] == 0, (f, a)
    assert seen >= 6


PROBE = r"""
#include <hip/hip_runtime.h>
__global__ void probe_dot(const float* w, const float* x, float* y, int n) {
  float acc = 0.0f;
  for (int k = 0; k < n; ++k) acc = acc + w[threadIdx.x * n + k] * x[k];
  y[threadIdx.x] = acc;
}
"""


@pytest.mark.parametrize("contract,flagged", [("off", False), ("fast", True)])
def test_gate_catches_contraction(contract, flagged, tmp_path):
    """A strict dot product compiled with -ffp-contract=fast (a plausible
    build mistake) has FMAs the gate rejects; with =off it passes."""
    tools()
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("no hipcc")
    src = tmp_path / "probe.hip"
    src.write_text(PROBE)
    obj = tmp_path / "probe.o"
    r = subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-ffp-contract=" + contract,
                        "-c", "-o", str(obj), str(src)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-1000:]
    fat, host, co = (str(tmp_path / ("p" + s)) for s in (".fat", ".host", ".co"))
    subprocess.run([os.path.join(LLVM, "llvm-objcopy"), "--dump-section", ".hip_fatbin=" + fat,
                    str(obj), host], check=True, capture_output=True)
    subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o",
                    "--input=" + fat, "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    "--output=" + co], check=True, capture_output=True)
    asm = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--mcpu=gfx950", co],
                         check=True, capture_output=True, text=True).stdout
    k = kernels(asm)
    f = [n for n in k if "probe_dot" in n][0]
    a = account(k[f])
    extra = a["fma32"] - (5 * a["div32"] + 5 * a["sqrt32"] + a["int_fma32"])
    assert (extra > 0) == flagged, a
