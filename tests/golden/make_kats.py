#!/usr/bin/env python3
"""Writes tests/golden/kats.json: known-answer vectors for the MoE expert path,
derived from closed forms only (no call into the oracle or the library).

The reference ships no test vectors (its only known answer needs the 17 GB
checkpoint), so every expected value here follows from the mathematics of the
format and of the operators:

* dequant (MLX affine, tools/split_experts.py:9-19, fused_dequant_matvec_4bit.metal:39-42,
  dequant_matvec_8bit.metal:26-27): element c of a row is field c % 8 (4-bit) or
  c % 4 (8-bit) of word c // per_word, low bits first; w = q*s + b. With bf16
  s and b, q*s is exact in fp32, so the fp32 result is the exact sum rounded
  once; float64 holds that sum exactly for the values below, and one
  float64 -> float32 conversion rounds it.
* mat-vec with one-hot x (fused_dequant_matvec_4bit.metal:14-53): y[o] = W[o, j]
  exactly (every other product is an exact zero).
* top-k routing (moe_routing_topk.metal:31-56): ids are the k largest logits,
  ties to the lower id; the renormalised weight of a chosen id is
  exp(l_i - m) / sum over the chosen exp(l_j - m) (the full-softmax
  denominator cancels), computed in float64. A -inf logit has p = 0 and is
  still chosen, after every positive p (strict > against a -inf start,
  :44-46). A NaN logit makes the softmax sum NaN (:33-39: max skips it, exp
  does not), so every p is NaN, no comparison succeeds and no id is chosen:
  ids -1 (weights 0 here; the shader writes -inf halves and indexes out of
  range, :48-51).
* SwiGLU (ops.metal:18-22): g / (1 + exp(-g)) * u in float64.

Run:  python3 tests/golden/make_kats.py   (rewrites kats.json deterministically)
"""
import json
import math
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f32_bits(v: float) -> int:
    return struct.unpack("<I", struct.pack("<f", v))[0]


def bf16_bits_exact(v: float) -> int:
    """bf16 pattern of a value that bf16 represents exactly (asserted)."""
    b = f32_bits(v)
    assert b & 0xFFFF == 0, v
    return b >> 16


def bf16_value(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", bits << 16))[0]


def rne_f32_to_bf16(fbits: int) -> int:
    """Round-to-nearest-even of an fp32 pattern to bf16 (finite inputs)."""
    lsb = (fbits >> 16) & 1
    return ((fbits + 0x7FFF + lsb) >> 16) & 0xFFFF


def dequant_cases():
    rng = np.random.default_rng(20261201)
    cases = []
    fixed = [
        (0x76543210, 1.0, 0.0),            # q = 0..7 in column order
        (0xFEDCBA98, 1.0, 0.0),            # q = 8..15
        (0x00000000, 0.5, -0.25),          # every element is the bias
        (0xFFFFFFFF, 0.0078125, 0.125),    # 15 s + b
        (0x0F0F0F0F, -3.0, 2.0),           # alternating 15 and 0
        (0x12345678, 0.01171875, -0.0625),
    ]
    for _ in range(6):
        s = bf16_value(int(rng.integers(0x3A00, 0x3D80)))      # |s| in about [5e-4, 6e-2]
        b = bf16_value(int(rng.integers(0x3A00, 0x3D00)) | (0x8000 if rng.integers(2) else 0))
        fixed.append((int(rng.integers(0, 2**32)), s, b))
    for word, s, b in fixed:
        sb, bb = bf16_bits_exact(s), bf16_bits_exact(b)
        q = [(word >> (4 * j)) & 0xF for j in range(8)]
        vals = [np.float32(qq * bf16_value(sb) + bf16_value(bb)) for qq in q]  # float64 exact, one rounding
        cases.append({"bits": 4, "word": word, "scale_bf16": sb, "bias_bf16": bb, "q": q,
                      "f32_bits": [f32_bits(float(v)) for v in vals],
                      "bf16_bits": [rne_f32_to_bf16(f32_bits(float(v))) for v in vals]})
    for word, s, b in [(0x03020100, 1.0, 0.0), (0xFF80017F, 0.00390625, -0.5), (0xDEADBEEF, -0.0625, 1.5)]:
        sb, bb = bf16_bits_exact(s), bf16_bits_exact(b)
        q = [(word >> (8 * j)) & 0xFF for j in range(4)]
        vals = [np.float32(qq * bf16_value(sb) + bf16_value(bb)) for qq in q]
        cases.append({"bits": 8, "word": word, "scale_bf16": sb, "bias_bf16": bb, "q": q,
                      "f32_bits": [f32_bits(float(v)) for v in vals],
                      "bf16_bits": [rne_f32_to_bf16(f32_bits(float(v))) for v in vals]})
    return cases


def onehot_matvec_case():
    """A [4 x 128] q4 matrix (2 groups per row); x = e_j for a few j; y = W[:, j]."""
    rng = np.random.default_rng(7)
    out_f, in_f = 4, 128
    words = rng.integers(0, 2**32, size=(out_f, in_f // 8), dtype=np.uint64).astype(np.uint32)
    sc = rng.integers(0x3B00, 0x3D00, size=(out_f, in_f // 64)).astype(np.uint16)
    bi = (rng.integers(0x3A00, 0x3C80, size=(out_f, in_f // 64)) | 0x8000).astype(np.uint16)
    cols = [0, 7, 8, 63, 64, 127]
    expect = {}
    for j in cols:
        col = []
        for o in range(out_f):
            q = (int(words[o, j // 8]) >> (4 * (j % 8))) & 0xF
            v = np.float32(q * bf16_value(int(sc[o, j // 64])) + bf16_value(int(bi[o, j // 64])))
            col.append(f32_bits(float(v)))
        expect[str(j)] = col
    return {"out": out_f, "in": in_f, "group": 64, "words": [int(w) for w in words.ravel()],
            "scales_bf16": [int(v) for v in sc.ravel()], "biases_bf16": [int(v) for v in bi.ravel()],
            "onehot_cols": cols, "y_f32_bits": expect}


def route_cases():
    def top(logits, k, norm):
        n = len(logits)
        if any(math.isnan(v) for v in logits):
            return [-1] * k, [0.0] * k
        finite = list(range(n))
        order = sorted(finite, key=lambda i: (-logits[i], i))  # larger first, lower id on ties
        sel = order[:k]
        m = max(logits[i] for i in finite)
        e = {i: math.exp(logits[i] - m) for i in finite}
        tot = sum(e.values())
        ids = sel + [-1] * (k - len(sel))
        p = [e[i] / tot for i in sel]
        if norm:
            s = sum(p)
            p = [v / s for v in p] if s > 0 else p
        return ids, p + [0.0] * (k - len(sel))

    cases = []
    base = [0.5, -1.0, 2.0, 2.0, 0.25, 3.0, -7.5, 2.0, 1.0, 0.0, -0.5, 1.5, 2.0, -2.0, 0.75, 3.0]
    cases.append(("ties_lower_id_first", base, 8, True))
    cases.append(("ties_no_renorm", base, 4, False))
    cases.append(("all_equal", [1.25] * 16, 8, True))
    cases.append(("nan_poisons_row", [float("nan"), 1.0, float("-inf"), 0.5, float("nan"), 2.0, -1.0, 0.0,
                                      3.0, float("nan"), -2.0, 1.5, 0.25, -0.25, 4.0, -3.0], 8, True))
    cases.append(("neg_inf_chosen_last", [float("-inf")] * 5 + [1.0, float("-inf"), 0.5, float("-inf"), 2.0]
                  + [float("-inf")] * 6, 8, True))
    rng = np.random.default_rng(3)
    wide = [float(np.float32(v)) for v in rng.standard_normal(128) * 3.0]
    wide[17] = wide[90] = float(np.float32(max(wide) + 1.0))  # an exact tie at the top
    cases.append(("n128_tie_at_top", wide, 8, True))
    cases.append(("top1", wide, 1, True))
    out = []
    for name, lg, k, norm in cases:
        ids, w = top(lg, k, norm)
        out.append({"name": name, "logits": [None if math.isnan(v) else v for v in lg], "k": k,
                    "norm_topk": norm, "ids": ids, "weights": w})
    return out


def swiglu_cases():
    gs = [-20.0, -3.5, -1.0, -0.125, 0.0, 0.0625, 0.5, 1.0, 2.75, 8.0, 30.0]
    us = [1.0, -2.0, 0.5, 3.0, 7.0, -1.0, 1.5, -0.25, 2.0, -4.0, 0.75]
    return [{"g": g, "u": u, "h": g / (1.0 + math.exp(-g)) * u} for g, u in zip(gs, us)]


def main():
    kats = {"about": "closed-form known answers; regenerate with tests/golden/make_kats.py",
            "dequant": dequant_cases(), "matvec_onehot": onehot_matvec_case(),
            "route_topk": route_cases(), "swiglu": swiglu_cases()}
    with open(os.path.join(HERE, "kats.json"), "w") as f:
        json.dump(kats, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
