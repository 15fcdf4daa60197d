"""Seeded synthetic workloads of the Qwen3-30B-A3B MoE shapes (numpy, host side).

Distributions (one layer, MLX affine format, group 64):
  packed 4-bit / 8-bit words: uniform random bits (nibbles / bytes U{0..2^bits-1});
  scales bf16(|N(0, 0.02)|); biases bf16(N(0, 0.01)); activations bf16(N(0, 1)).
Prefill routing: Gumbel-top-k over log Zipf(s) weights of a seeded expert
permutation (exact sampling of k distinct experts without replacement with
probability proportional to rank^-s); routing weights are the softmax of the
perturbed scores over the selected experts.
"""
from __future__ import annotations

from typing import Dict, Tuple

import numpy as np


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_normal(rng: np.random.Generator, shape, std: float = 1.0, absval: bool = False) -> np.ndarray:
    v = rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std)
    if absval:
        v = np.abs(v)
    return f32_to_bf16_bits(v)


def quant_tensor(rng: np.random.Generator, rows: int, cols: int, bits: int = 4, group: int = 64,
                 scale_std: float = 0.02, bias_std: float = 0.01) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(weight uint32 [rows, cols*bits/32], scales bf16 [rows, cols/group], biases bf16)."""
    w = rng.integers(0, 2**32, size=(rows, cols * bits // 32), dtype=np.uint64).astype(np.uint32)
    s = bf16_normal(rng, (rows, cols // group), scale_std, absval=True)
    b = bf16_normal(rng, (rows, cols // group), bias_std)
    return w, s, b


def moe_layer(seed: int, n_exp: int = 128, hidden: int = 2048, inter: int = 768, group: int = 64
              ) -> Dict[str, np.ndarray]:
    """Stacked switch_mlp tensors of one layer + 8-bit router gate."""
    rng = np.random.default_rng(seed)
    out: Dict[str, np.ndarray] = {}
    for proj, (r, c) in (("gate", (inter, hidden)), ("up", (inter, hidden)), ("down", (hidden, inter))):
        w, s, b = quant_tensor(rng, n_exp * r, c, 4, group)
        out[f"{proj}_w"] = w.reshape(n_exp, r, c // 8)
        out[f"{proj}_s"] = s.reshape(n_exp, r, c // group)
        out[f"{proj}_b"] = b.reshape(n_exp, r, c // group)
    w, s, b = quant_tensor(rng, n_exp, hidden, 8, group)
    out["router_w"], out["router_s"], out["router_b"] = w, s, b
    return out


def zipf_routing(T: int, n_exp: int = 128, k: int = 8, s: float = 1.1, seed: int = 0
                 ) -> Tuple[np.ndarray, np.ndarray]:
    """ids int32 [T, k] (distinct per token), weights fp32 [T, k] summing to 1."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(n_exp)
    logw = np.empty(n_exp)
    logw[perm] = -s * np.log(np.arange(1, n_exp + 1))
    score = logw[None, :] + rng.gumbel(size=(T, n_exp))
    ids = np.argsort(-score, axis=1, kind="stable")[:, :k]
    sel = np.take_along_axis(score, ids, axis=1)
    w = np.exp(sel - sel.max(axis=1, keepdims=True))
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids.astype(np.int32), w


def bytes_per_expert(hidden: int = 2048, inter: int = 768, group: int = 64) -> int:
    """Packed weights + bf16 scales + bf16 biases of gate, up and down."""
    per_proj = inter * hidden // 2 + 2 * 2 * (inter * hidden // group)
    return 3 * per_proj


def router_bytes(n_exp: int = 128, hidden: int = 2048, group: int = 64) -> int:
    return n_exp * hidden + 2 * 2 * (n_exp * hidden // group)


# Checkpoint tensor names of one layer's MoE block (MLX Qwen3-MoE checkpoints;
# the split files of tools/split_experts.py:9-19 use e{N}.{proj}.{kind}).
CKPT_NAMES = {
    "gate_w": "mlp.switch_mlp.gate_proj.weight", "gate_s": "mlp.switch_mlp.gate_proj.scales",
    "gate_b": "mlp.switch_mlp.gate_proj.biases", "up_w": "mlp.switch_mlp.up_proj.weight",
    "up_s": "mlp.switch_mlp.up_proj.scales", "up_b": "mlp.switch_mlp.up_proj.biases",
    "down_w": "mlp.switch_mlp.down_proj.weight", "down_s": "mlp.switch_mlp.down_proj.scales",
    "down_b": "mlp.switch_mlp.down_proj.biases", "router_w": "mlp.gate.weight",
    "router_s": "mlp.gate.scales", "router_b": "mlp.gate.biases",
    "norm_w": "post_attention_layernorm.weight",
}
BF16_KEYS = ("gate_s", "gate_b", "up_s", "up_b", "down_s", "down_b", "router_s", "router_b", "norm_w")


def hf_config(n_layers: int, n_exp: int = 128, top_k: int = 8, hidden: int = 2048, inter: int = 768,
              group: int = 64, norm_topk: bool = True, rms_eps: float = 1e-6) -> dict:
    """A Qwen3-MoE config.json (the fields of Qwen3MoeConfig, src/model.rs:9-22,
    plus MLX's quantization block)."""
    return {
        "architectures": ["Qwen3MoeForCausalLM"], "model_type": "qwen3_moe",
        "num_hidden_layers": n_layers, "hidden_size": hidden, "num_attention_heads": 32,
        "num_key_value_heads": 4, "head_dim": 128, "num_experts": n_exp, "num_experts_per_tok": top_k,
        "moe_intermediate_size": inter, "rms_norm_eps": rms_eps, "rope_theta": 10000000.0,
        "vocab_size": 151936, "norm_topk_prob": norm_topk,
        "quantization": {"group_size": group, "bits": 4},
    }


def write_checkpoint(model_dir: str, layers: Dict[int, Dict[str, np.ndarray]], config: dict,
                     layout: str = "sharded", shards: int = 2) -> None:
    """Writes `layers` ({layer: MoeLayer-keyed arrays}) as a safetensors model
    directory with the `safetensors` package (an independent writer).

    layout "single": one model.safetensors; "sharded": `shards` files listed in
    model.safetensors.index.json, a layer's tensors spread over all of them;
    "split": expert tensors in splitted_moe/layer_{l}_experts.safetensors as
    e{N}.{proj}.{kind} with scales and biases cast to float16 (as
    tools/split_experts.py:72-75 does), the rest in model.safetensors."""
    import json
    import os

    import torch
    from safetensors.torch import save_file

    def tt(key: str, a: np.ndarray):
        t = torch.from_numpy(np.array(a, copy=True))  # the writer refuses tensors sharing memory
        return t.view(torch.bfloat16) if key in BF16_KEYS and a.dtype == np.uint16 else t

    os.makedirs(model_dir, exist_ok=True)
    with open(os.path.join(model_dir, "config.json"), "w") as f:
        json.dump(config, f, indent=2)
    named = {}
    split = {}
    for il, t in sorted(layers.items()):
        for key, a in t.items():
            if a is None:
                continue
            name = f"model.layers.{il}.{CKPT_NAMES[key]}"
            if layout == "split" and key[:-2] in ("gate", "up", "down"):
                proj, kind = CKPT_NAMES[key].split(".")[-2:]
                for e in range(a.shape[0]):
                    x = a[e]
                    if key in BF16_KEYS and x.dtype == np.uint16:  # bf16 bits; float16 arrays go as given
                        x = bf16_bits_to_f32(x).astype(np.float16)
                    split.setdefault(il, {})[f"e{e}.{proj}.{kind}"] = torch.from_numpy(np.ascontiguousarray(x))
            else:
                named[name] = tt(key, a)
    meta = {"format": "mlx"}
    if layout in ("single", "split"):
        save_file(named, os.path.join(model_dir, "model.safetensors"), metadata=meta)
    elif layout == "sharded":
        files = [f"model-{i + 1:05d}-of-{shards:05d}.safetensors" for i in range(shards)]
        parts = [{} for _ in range(shards)]
        weight_map = {}
        for i, (name, t) in enumerate(sorted(named.items())):
            parts[i % shards][name] = t
            weight_map[name] = files[i % shards]
        for fn, p in zip(files, parts):
            save_file(p, os.path.join(model_dir, fn), metadata=meta)
        with open(os.path.join(model_dir, "model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {"total_size": sum(t.numel() * t.element_size() for t in named.values())},
                       "weight_map": weight_map}, f, indent=2)
    else:
        raise ValueError(f"unknown layout {layout!r}")
    if layout == "split":
        d = os.path.join(model_dir, "splitted_moe")
        os.makedirs(d, exist_ok=True)
        for il, t in split.items():
            save_file(t, os.path.join(d, f"layer_{il}_experts.safetensors"))


def centered_quant(rng: np.random.Generator, rows: int, cols: int, group: int = 64,
                   scale_std: float = 0.02) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """4-bit matrix whose dequantized values are centred on zero, as MLX
    quantisation of real weights makes them (bias ~ -7.5 * scale, the group
    minimum): scales bf16(|N(0, scale_std)|), biases bf16(-7.5 s + N(0, s/8))."""
    w = rng.integers(0, 2**32, size=(rows, cols // 8), dtype=np.uint64).astype(np.uint32)
    s = bf16_normal(rng, (rows, cols // group), scale_std, absval=True)
    sf = bf16_bits_to_f32(s)
    b = f32_to_bf16_bits(-7.5 * sf + rng.standard_normal(sf.shape).astype(np.float32) * sf / 8)
    return w, s, b


def norm_weight(rng: np.random.Generator, n: int) -> np.ndarray:
    """RMSNorm weight around 1: bf16(1 + N(0, 0.1))."""
    return f32_to_bf16_bits(1.0 + 0.1 * rng.standard_normal(n).astype(np.float32))


def decoder_weights(seed: int, n_layers: int, hidden: int, n_heads: int, n_kv: int, head_dim: int, n_exp: int,
                    inter: int, vocab: int, group: int = 64):
    """Seeded random weights of a Qwen3-MoE decoder (host arrays): per layer the
    attention tensors (centred 4-bit q/k/v/o, norm weights), the router of
    moe_layer() and centred expert tables; globally the embedding, final norm
    and lm_head.

    The experts are centred too: moe_layer()'s all-positive tables give every
    expert output one common direction, which the residual stream accumulates
    until the SwiGLU intermediates leave the f16 range the kernels carry them
    in (|h| > 65504 within six tokens of two layers), where a trained model's
    stay small."""
    rng = np.random.default_rng(seed)
    layers = []
    qd, kvd = n_heads * head_dim, n_kv * head_dim
    for il in range(n_layers):
        t = moe_layer(seed * 1000 + il, n_exp, hidden, inter, group)
        for proj, (r, c), sd in (("gate", (inter, hidden), 0.02), ("up", (inter, hidden), 0.02),
                                 ("down", (hidden, inter), 0.01)):
            w, s, b = centered_quant(rng, n_exp * r, c, group, sd)
            t[f"{proj}_w"] = w.reshape(n_exp, r, c // 8)
            t[f"{proj}_s"] = s.reshape(n_exp, r, c // group)
            t[f"{proj}_b"] = b.reshape(n_exp, r, c // group)
        for name, (r, c) in (("q", (qd, hidden)), ("k", (kvd, hidden)), ("v", (kvd, hidden)), ("o", (hidden, qd))):
            t[name + "_w"], t[name + "_s"], t[name + "_b"] = centered_quant(rng, r, c, group)
        t["in_norm"] = norm_weight(rng, hidden)
        t["post_norm"] = norm_weight(rng, hidden)
        t["q_norm"] = norm_weight(rng, head_dim)
        t["k_norm"] = norm_weight(rng, head_dim)
        layers.append(t)
    glob = {"final_norm": norm_weight(rng, hidden)}
    glob["embed_w"], glob["embed_s"], glob["embed_b"] = centered_quant(rng, vocab, hidden, group, 0.05)
    glob["lm_w"], glob["lm_s"], glob["lm_b"] = centered_quant(rng, vocab, hidden, group)
    return layers, glob
