"""The CLI's architecture gate (code/cis2-fp/src/main.rs:545-644, run at
:817-823 on config.json alone): every checkpoint outside the specified
subset is refused by name with exit status 2, a `CIS2_REF_UNSUPPORTED
reason=...` line and no digest, before any weights file is opened.  The
configs are the reference's own refusal fixtures
(code/cis2-fp/tests/fixtures/refusal*/, copied as data to
tests/golden/refusal/); the expected reasons are the reference gate's
format strings.  One deliberate difference: model_type "qwen3" is in this
build's subset (the archived Qwen3 port), so qwen3-0.6b-base passes the
gate and stops at its missing weights, as qwen25-1.5b does in the
reference suite (run_refusal_suite.sh:15-18).  The gate runs before any
GPU call, so these tests need no GPU."""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "cis2-lab-archive_amd", "bin", "cis2_host")
FIX = os.path.join(ROOT, "tests", "golden", "refusal")
SUBSET = ' is not in the CIS-2 specified subset ["llama", "qwen2", "qwen3"]'
MULT = ("is set; this implementation hardcodes rsqrt(head_dim) attention scaling and no logit "
        "scaling, so the result would be silently wrong")

EXPECTED = {
    "deepseek-v3": 'model_type="deepseek_v3"' + SUBSET,
    "gpt-oss-20b": 'model_type="gpt_oss"' + SUBSET,
    "granite-3.3-2b": 'model_type="granite"' + SUBSET,
    "mistral-7b-v03": 'model_type="mistral"' + SUBSET,
    "olmo2-1b": 'model_type="olmo2"' + SUBSET,
    "phi-4-mini": 'model_type="phi3"' + SUBSET,
    "smollm3-3b": 'model_type="smollm3"' + SUBSET,
    "granite-disguised-as-llama": "attention_multiplier " + MULT,
    "olmo2-disguised-as-llama": 'torch_dtype="float32"; CIS-2 pins bf16-on-disk weights (§3.5)',
    "qwen3-disguised-as-qwen2": ("config declares head_dim=128 but this implementation derives "
                                 "hidden_size/num_attention_heads=64; the decode path uses the "
                                 "derived value, so the explicit one would be silently ignored"),
    "qwen25-1.5b": None,      # in the subset: passes the gate, no weights here
    "qwen3-0.6b-base": None,  # in this build's subset (Qwen3 port)
}


def run(wdir, tmp_path):
    if not os.path.exists(CLI):
        pytest.skip("cis2_host not built")
    ids = tmp_path / "ids.txt"
    ids.write_text("1 2 3\n")
    return subprocess.run([CLI, "--weights-dir", str(wdir), "--ids", str(ids), "--gen-toks", "1"],
                          capture_output=True, text=True, timeout=60)


@pytest.mark.parametrize("name", sorted(EXPECTED))
def test_reference_refusal_fixtures(name, tmp_path):
    r = run(os.path.join(FIX, name), tmp_path)
    assert r.returncode == 2
    assert "CIS2_REF digest=" not in r.stdout
    want = EXPECTED[name]
    if want is None:
        assert "CIS2_REF_UNSUPPORTED" not in r.stderr
        assert "FATAL: cannot open" in r.stderr and "model.safetensors" in r.stderr
    else:
        lines = r.stderr.splitlines()
        assert lines[0] == "CIS2_REF_UNSUPPORTED reason=" + want
        assert lines[1] == "This checkpoint is outside the CIS-2 specified subset; no digest emitted."


BASE = {"model_type": "llama", "torch_dtype": "bfloat16", "hidden_size": 576,
        "num_attention_heads": 9, "rope_scaling": None}


@pytest.mark.parametrize("extra,reason", [
    ({"num_attention_heads": 0}, "num_attention_heads=0"),
    ({"hidden_size": 27, "num_attention_heads": 3}, "derived head_dim=9 is odd; RoPE pairs require even"),
    ({"model_type": "qwen3", "head_dim": 7}, "head_dim=7 is odd; RoPE pairs require even"),
    ({"partial_rotary_factor": 0.5}, "partial_rotary_factor=0.5; only full rotary is specified"),
    ({"rope_scaling": {"type": "linear", "factor": 2.0}},
     "rope_scaling is set; only unscaled RoPE is specified"),
    ({"use_sliding_window": True}, "use_sliding_window=true; only full causal attention is specified"),
    ({"quantization_config": {"bits": 4}},
     "quantization_config is present; CIS-2 reads unquantized bf16 weights"),
    ({"final_logit_softcapping": 30.0}, "final_logit_softcapping " + MULT),
    ({"num_experts": 8}, "num_experts is set; MoE routing is not specified"),
    ({"model_type": "qwen2", "head_dim": 32},
     "config declares head_dim=32 but this implementation derives hidden_size/num_attention_heads"
     "=64; the decode path uses the derived value, so the explicit one would be silently ignored"),
])
def test_gate_checks(extra, reason, tmp_path):
    d = tmp_path / "w"
    d.mkdir()
    cfg = dict(BASE)
    cfg.update(extra)
    (d / "config.json").write_text(json.dumps(cfg))
    r = run(d, tmp_path)
    assert r.returncode == 2
    assert r.stderr.splitlines()[0] == "CIS2_REF_UNSUPPORTED reason=" + reason


@pytest.mark.parametrize("extra", [
    {}, {"partial_rotary_factor": 1.0}, {"use_sliding_window": False}, {"head_dim": 64},
    {"model_type": "qwen3", "head_dim": 128}, {"model_type": "qwen2"},
    {"head_dim": None}, {"model_type": "qwen3", "head_dim": None},
])
def test_gate_accepts(extra, tmp_path):
    d = tmp_path / "w"
    d.mkdir()
    cfg = dict(BASE)
    cfg.update(extra)
    (d / "config.json").write_text(json.dumps(cfg))
    r = run(d, tmp_path)
    assert "CIS2_REF_UNSUPPORTED" not in r.stderr
    assert "FATAL: cannot open" in r.stderr
