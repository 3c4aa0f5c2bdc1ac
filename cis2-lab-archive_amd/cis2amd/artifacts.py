"""Synthetic CIS-2 artifacts: model configs, seeded BF16 weights, the
weights/config/tokenizer files the reference driver reads, and prompts.

The model shapes restate the workloads the CIS-2 evidence uses (SmolLM2-135M,
llama-160m, Qwen3-0.6B) plus small shapes for fast checks.  Weights come from
the deterministic generator in csrc/cis2_synth.c (integer PRNG, exact
transform), so every host regenerates identical bytes and identical
sha256(model.safetensors).
"""
import hashlib
import json
import os
from dataclasses import dataclass, field

import numpy as np

from . import _lib


@dataclass
class ModelSpec:
    name: str
    hidden: int
    inter: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    vocab: int
    eps: float
    rope_theta: float
    tied: bool
    head_dim: int = 0          # 0: hidden // n_heads (no head_dim key)
    qk_norm: bool = False      # Qwen3 per-head q_norm / k_norm tensors
    qkv_bias: bool = False     # Qwen2 q/k/v biases
    sigma: float = 0.02
    extra: dict = field(default_factory=dict)

    @property
    def hd(self):
        return self.head_dim or self.hidden // self.n_heads

    @property
    def qd(self):
        return self.n_heads * self.hd

    @property
    def kvd(self):
        return self.n_kv_heads * self.hd

    def config_json(self):
        """config.json text; keys as the reference driver reads them
        (code/cis2-fp/gpu/cis2_host.cpp:97-117), rendered the way HF writes them."""
        d = {
            "architectures": ["Qwen3ForCausalLM" if self.qk_norm else "LlamaForCausalLM"],
            "hidden_act": "silu",
            "hidden_size": self.hidden,
            "intermediate_size": self.inter,
            "model_type": "qwen3" if self.qk_norm else "llama",
            "num_attention_heads": self.n_heads,
            "num_hidden_layers": self.n_layers,
            "num_key_value_heads": self.n_kv_heads,
            "rms_norm_eps": self.eps,
            "rope_theta": self.rope_theta,
            "tie_word_embeddings": self.tied,
            "torch_dtype": "bfloat16",
            "vocab_size": self.vocab,
        }
        if self.head_dim:
            d["head_dim"] = self.head_dim
        d.update(self.extra)
        return json.dumps(d, indent=2, sort_keys=True) + "\n"


SPECS = {
    # SmolLM2-135M architecture (code/cis2-fp/weights/config.json).
    "smollm2-135m": ModelSpec("smollm2-135m", 576, 1536, 30, 9, 3, 49152, 1e-5, 100000.0, True),
    # JackFram/llama-160m shape; eps 1e-6 as that model's config records.
    "llama-160m": ModelSpec("llama-160m", 768, 3072, 12, 12, 12, 32000, 1e-6, 10000.0, False),
    # Qwen3-0.6B shape: head_dim 128 independent of hidden/heads, QK-norm.
    "qwen3-0.6b": ModelSpec("qwen3-0.6b", 1024, 3072, 28, 16, 8, 151936, 1e-6, 1000000.0, True,
                            head_dim=128, qk_norm=True),
    # small shapes for quick parity runs
    "tiny-llama": ModelSpec("tiny-llama", 64, 128, 2, 4, 2, 512, 1e-5, 10000.0, True),
    "tiny-untied": ModelSpec("tiny-untied", 96, 160, 3, 6, 3, 300, 1e-6, 500000.0, False),
    "tiny-qwen3": ModelSpec("tiny-qwen3", 64, 96, 2, 4, 2, 384, 1e-6, 1000000.0, True,
                            head_dim=32, qk_norm=True),
    "tiny-qwen2": ModelSpec("tiny-qwen2", 64, 128, 2, 4, 1, 256, 1e-6, 1000000.0, True,
                            qkv_bias=True),
    "smollm2-4l": ModelSpec("smollm2-4l", 576, 1536, 4, 9, 3, 49152, 1e-5, 100000.0, True),
    # Qwen3-style head geometry (head_dim 128, QK-norm, GQA 2:1) at a small
    # size: long prompts run the streamed-attention path in few seconds.
    "tiny-wide": ModelSpec("tiny-wide", 256, 256, 2, 2, 1, 512, 1e-6, 1000000.0, True,
                           head_dim=128, qk_norm=True),
}

TOKENIZER_JSON = (json.dumps({"version": "1.0", "model": {"type": "synthetic-ids"},
                              "note": "token ids are supplied directly"}, sort_keys=True)
                  + "\n")


def tensor_list(spec):
    """(name, shape) in a fixed order; the order is also the generator ordinal
    and the safetensors data order."""
    H, I, V, QD, KV, HD = spec.hidden, spec.inter, spec.vocab, spec.qd, spec.kvd, spec.hd
    out = [("model.embed_tokens.weight", (V, H))]
    for i in range(spec.n_layers):
        p = "model.layers.%d." % i
        out += [
            (p + "input_layernorm.weight", (H,)),
            (p + "post_attention_layernorm.weight", (H,)),
            (p + "self_attn.q_proj.weight", (QD, H)),
            (p + "self_attn.k_proj.weight", (KV, H)),
            (p + "self_attn.v_proj.weight", (KV, H)),
            (p + "self_attn.o_proj.weight", (H, QD)),
            (p + "mlp.gate_proj.weight", (I, H)),
            (p + "mlp.up_proj.weight", (I, H)),
            (p + "mlp.down_proj.weight", (H, I)),
        ]
        if spec.qkv_bias:
            out += [(p + "self_attn.q_proj.bias", (QD,)), (p + "self_attn.k_proj.bias", (KV,)),
                    (p + "self_attn.v_proj.bias", (KV,))]
        if spec.qk_norm:
            out += [(p + "self_attn.q_norm.weight", (HD,)), (p + "self_attn.k_norm.weight", (HD,))]
    out.append(("model.norm.weight", (H,)))
    if not spec.tied:
        out.append(("lm_head.weight", (V, H)))
    return out


def gen_bf16(seed, ordinal, n, sigma):
    out = np.empty(n, dtype=np.uint16)
    _lib.synth().cis2_synth_bf16(seed, ordinal, sigma,
                                 out.ctypes.data_as(_lib.c_u16p), n)
    return out


def gen_f32(seed, ordinal, n, sigma):
    out = np.empty(n, dtype=np.float32)
    _lib.synth().cis2_synth_f32(seed, ordinal, sigma, out.ctypes.data_as(_lib.c_fp), n)
    return out


def gen_uniform(seed, ordinal, lo, hi, n):
    out = np.empty(n, dtype=np.uint32)
    _lib.synth().cis2_synth_uniform(seed, ordinal, lo, hi, out.ctypes.data_as(_lib.c_u32p), n)
    return out


class Weights:
    """All tensors of a spec as BF16 arrays (generated once, kept in memory)."""

    def __init__(self, spec, seed):
        self.spec = spec
        self.seed = seed
        self.tensors = []
        for i, (name, shape) in enumerate(tensor_list(spec)):
            n = int(np.prod(shape))
            self.tensors.append((name, shape, gen_bf16(seed, i, n, spec.sigma)))

    def safetensors_bytes(self):
        """The model.safetensors byte image: 8-byte LE header length, JSON
        header (dtype BF16, shape, data_offsets), then the raw data."""
        hdr = {}
        off = 0
        for name, shape, arr in self.tensors:
            nb = arr.nbytes
            hdr[name] = {"dtype": "BF16", "shape": list(shape), "data_offsets": [off, off + nb]}
            off += nb
        hj = json.dumps(hdr, separators=(",", ":")).encode()
        hj += b" " * ((8 - len(hj) % 8) % 8)
        return len(hj).to_bytes(8, "little") + hj, off

    def file_sha256(self):
        head, _ = self.safetensors_bytes()
        h = hashlib.sha256(head)
        for _, _, arr in self.tensors:
            h.update(arr.tobytes())
        return h.digest()

    def write_dir(self, path):
        """Writes model.safetensors, config.json and tokenizer.json."""
        os.makedirs(path, exist_ok=True)
        head, _ = self.safetensors_bytes()
        with open(os.path.join(path, "model.safetensors"), "wb") as f:
            f.write(head)
            for _, _, arr in self.tensors:
                f.write(arr.tobytes())
        with open(os.path.join(path, "config.json"), "w") as f:
            f.write(self.spec.config_json())
        with open(os.path.join(path, "tokenizer.json"), "w") as f:
            f.write(TOKENIZER_JSON)

    def header_digests(self):
        """96 bytes: sha256 of model.safetensors, tokenizer.json, config.json."""
        return (self.file_sha256() + hashlib.sha256(TOKENIZER_JSON.encode()).digest() +
                hashlib.sha256(self.spec.config_json().encode()).digest())


def prompt_ids(seed, vocab, n, ordinal=1 << 40):
    """n prompt ids uniform in [0, vocab)."""
    return gen_uniform(seed, ordinal, 0, vocab - 1, n)


def set_prompt(seed, idx, vocab, lo, hi, stream):
    """Prompt idx of a seeded prompt set: length uniform in [lo, hi], ids
    uniform in [0, vocab).  stream separates sets drawn from one seed."""
    n = int(gen_uniform(seed, (stream << 40) + (1 << 39) + idx, lo, hi, 1)[0])
    return gen_uniform(seed, (stream << 40) + idx, 0, vocab - 1, n)


# The llama-160m prompt set: 300 prompts of 8..64 tokens, 128 generated each.
LLAMA_SET = {"spec": "llama-160m", "seed": 160, "count": 300, "lo": 8, "hi": 64,
             "stream": 3, "gen_toks": 128}
# The batch-stress set on the SmolLM2-135M shape: 64 sequences with prompts of
# 16..512 tokens, 256 generated each; a batch of B uses sequences 0..B-1.
BATCH_SET = {"spec": "smollm2-135m", "seed": 20261201, "count": 64, "lo": 16, "hi": 512,
             "stream": 4, "gen_toks": 256}


def set_prompts(pset):
    spec = SPECS[pset["spec"]]
    return [set_prompt(pset["seed"], i, spec.vocab, pset["lo"], pset["hi"], pset["stream"])
            for i in range(pset["count"])]
