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
