"""ctypes wrapper of liboracle.so — the CPU restatement of the MoE hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke check and by the
CPU-baseline leg of bench.py, never by the product library.

Also holds `dequant_numpy`, an independent NumPy restatement of the reference's
own replica (validate_dequant.py:26-30), used to pin the C dequant.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import Dict, Optional, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

SB_BF16, SB_F16 = 0, 1
SUM_SERIAL, SUM_WAVE = 0, 1
ROUTE_REF, ROUTE_F32 = 0, 1
MODE_F64, MODE_SHADER_F16, MODE_MFMA_BF16 = 0, 1, 2


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


class OrcLayer(C.Structure):
    _fields_ = [("n_exp", C.c_int32), ("hidden", C.c_int32), ("inter", C.c_int32), ("group", C.c_int32)] + [
        (n, C.c_void_p) for n in ("gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s",
                                  "down_b", "router_w", "router_s", "router_b")]


_L = None


def lib() -> C.CDLL:
    global _L
    if _L is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_exp.restype = C.c_float
        L.orc_exp.argtypes = [C.c_float]
        L.orc_silu_mul.restype = C.c_float
        L.orc_silu_mul.argtypes = [C.c_float, C.c_float]
        L.orc_dequant.argtypes = [i32, vp, vp, vp, i32, vp, i64, i64, i32]
        L.orc_qmatvec_shader.argtypes = [i32, vp, vp, vp, i32, vp, vp, i64, i64, i32]
        L.orc_qmatvec_lanes.argtypes = [i32, vp, vp, vp, i32, vp, vp, i64, i64, i32, i32]
        L.orc_qmatvec_f64.argtypes = [i32, vp, vp, vp, i32, vp, vp, vp, i64, i64, i32]
        L.orc_route_topk.argtypes = [vp, i64, i32, i32, i32, i32, i32, vp, vp]
        L.orc_router.argtypes = [C.POINTER(OrcLayer), vp, i64, i32, i32, i32, vp, vp, vp]
        L.orc_moe_decode.argtypes = [C.POINTER(OrcLayer), vp, i64, i32, i32, i32, vp, vp, vp, vp, i32, vp]
        L.orc_group_rows.argtypes = [vp, i64, i32, i32, vp, vp, vp, vp]
        L.orc_moe_prefill.argtypes = [C.POINTER(OrcLayer), vp, i64, i32, vp, vp, i32, vp]
        L.orc_moe_decode_baseline.argtypes = [C.POINTER(OrcLayer), vp, i32, i32, i32, vp, vp, vp]
        L.orc_router_baseline.argtypes = [C.POINTER(OrcLayer), vp, i64, i32, i32, i32, vp, vp]
        L.orc_moe_prefill_baseline.argtypes = [C.POINTER(OrcLayer), vp, i64, i32, vp, vp, i32, vp]
        L.orc_rmsnorm.argtypes = [vp, vp, C.c_float, i64, i64, vp]
        L.orc_rope_neox.argtypes = [vp, i64, i64, i64, C.c_float]
        L.orc_sdpa_decode.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, C.c_double, vp]
        L.orc_argmax.restype = i64
        L.orc_argmax.argtypes = [vp, i64]
        L.orc_f32_to_bf16_n.argtypes = [vp, vp, i64]
        L.orc_omp_max_threads.restype = C.c_int
        L.orc_set_threads.argtypes = [C.c_int]
        _L = L
    return _L


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _rc(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"{what}: oracle rejected the arguments (rc={rc})")


# ---- scalars ---------------------------------------------------------------
def bf16_to_f32(h: int) -> float:
    return lib().orc_bf16_to_f32(h)


def f32_to_bf16(f: float) -> int:
    return lib().orc_f32_to_bf16(f)


def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().orc_f32_to_f16(f)


def exp(x: float) -> float:
    return lib().orc_exp(x)


def silu_mul(g: float, u: float) -> float:
    return lib().orc_silu_mul(g, u)


# ---- tensors ---------------------------------------------------------------
def rmsnorm(x_bf16, w_bf16, eps: float) -> np.ndarray:
    """RMSNorm of the rows of x (bf16 [..., dim]) -> bf16 bits, the documented
    lane order (orc_rmsnorm; rmsnorm.metal:17-35)."""
    x = _c(x_bf16, np.uint16)
    w = _c(w_bf16, np.uint16)
    dim = x.shape[-1]
    rows = x.size // dim
    out = np.empty(x.shape, np.uint16)
    _rc(lib().orc_rmsnorm(_p(x), _p(w), eps, rows, dim, _p(out)), "rmsnorm")
    return out



def dequant(bits: int, w, s, b, rows: int, cols: int, group: int = 64, sb_type: int = SB_BF16) -> np.ndarray:
    w, s, b = _c(w, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    out = np.empty((rows, cols), np.float32)
    _rc(lib().orc_dequant(bits, _p(w), _p(s), _p(b), sb_type, _p(out), rows, cols, group), "dequant")
    return out


def qmatvec(kind: str, bits: int, w, s, b, x_f32, in_f: int, out_f: int, group: int = 64, lanes: int = 64,
            sb_type: int = SB_BF16):
    """kind: 'shader' | 'lanes' -> fp32 y; 'f64' -> (y f64, absbound f64)."""
    w, s, b, x = _c(w, np.uint32), _c(s, np.uint16), _c(b, np.uint16), _c(x_f32, np.float32)
    L = lib()
    if kind == "f64":
        y = np.empty(out_f, np.float64)
        ab = np.empty(out_f, np.float64)
        _rc(L.orc_qmatvec_f64(bits, _p(w), _p(s), _p(b), sb_type, _p(x), _p(y), _p(ab), in_f, out_f, group), kind)
        return y, ab
    y = np.empty(out_f, np.float32)
    if kind == "shader":
        _rc(L.orc_qmatvec_shader(bits, _p(w), _p(s), _p(b), sb_type, _p(x), _p(y), in_f, out_f, group), kind)
    elif kind == "lanes":
        _rc(L.orc_qmatvec_lanes(bits, _p(w), _p(s), _p(b), sb_type, _p(x), _p(y), in_f, out_f, group, lanes), kind)
    else:
        raise ValueError(kind)
    return y


def route_topk(logits, k: int, norm_topk: bool = True, sum_order: int = SUM_WAVE,
               rule: int = ROUTE_REF) -> Tuple[np.ndarray, np.ndarray]:
    """rule ROUTE_REF: the reference's f16 logits and f16 weights; ROUTE_F32: fp32 throughout."""
    lg = _c(logits, np.float32)
    if lg.ndim == 1:
        lg = lg[None, :]
    T, n = lg.shape
    ids = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    _rc(lib().orc_route_topk(_p(lg), T, n, k, int(norm_topk), sum_order, int(rule), _p(ids), _p(w)),
        "route_topk")
    return ids, w


class Layer:
    """Keeps numpy arrays alive and exposes the orc_layer struct."""

    def __init__(self, t: Dict[str, np.ndarray], n_exp: int, hidden: int, inter: int, group: int = 64):
        self.arrs = {k: np.ascontiguousarray(v) for k, v in t.items()}
        self.s = OrcLayer(n_exp, hidden, inter, group, *[self.arrs[k].ctypes.data for k in (
            "gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b",
            "router_w", "router_s", "router_b")])
        self.n_exp, self.hidden, self.inter, self.group = n_exp, hidden, inter, group


def router(layer: Layer, x_bf16, k: int, norm_topk: bool = True, rule: int = ROUTE_REF):
    """(fp32 logits [T, E] before any f16 rounding, ids [T, k], weights [T, k])."""
    x = _c(x_bf16, np.uint16).reshape(-1, layer.hidden)
    T = x.shape[0]
    lg = np.empty((T, layer.n_exp), np.float32)
    ids = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    _rc(lib().orc_router(C.byref(layer.s), _p(x), T, k, int(norm_topk), int(rule), _p(lg), _p(ids), _p(w)),
        "router")
    return lg, ids, w


def moe_decode(layer: Layer, x_bf16, k: int, norm_topk: bool = True, ids=None, w=None, mode: int = MODE_F64,
               rule: int = ROUTE_REF):
    x = _c(x_bf16, np.uint16).reshape(-1, layer.hidden)
    T = x.shape[0]
    y = np.empty((T, layer.hidden), np.float64)
    ids_o = np.empty((T, k), np.int32)
    w_o = np.empty((T, k), np.float32)
    ids_i = None if ids is None else _c(ids, np.int32).reshape(T, k)
    w_i = None if w is None else _c(w, np.float32).reshape(T, k)
    _rc(lib().orc_moe_decode(C.byref(layer.s), _p(x), T, k, int(norm_topk), int(rule), _p(ids_i), _p(w_i),
                             _p(ids_o), _p(w_o), mode, _p(y)), "moe_decode")
    if ids is None:
        return y, ids_o, w_o
    return y, ids_i, w_i


def group_rows(ids, n_exp: int):
    ids = _c(ids, np.int32)
    T, k = ids.shape
    counts = np.empty(n_exp, np.int32)
    offsets = np.empty(n_exp + 1, np.int32)
    row_token = np.empty(T * k, np.int32)
    slot_row = np.empty(T * k, np.int32)
    _rc(lib().orc_group_rows(_p(ids), T, k, n_exp, _p(counts), _p(offsets), _p(row_token), _p(slot_row)),
        "group_rows")
    return counts, offsets, row_token, slot_row


def moe_prefill(layer: Layer, X_bf16, ids, w, mode: int = MODE_F64) -> np.ndarray:
    X = _c(X_bf16, np.uint16).reshape(-1, layer.hidden)
    T = X.shape[0]
    ids, w = _c(ids, np.int32), _c(w, np.float32)
    k = ids.shape[1]
    y = np.empty((T, layer.hidden), np.float64)
    _rc(lib().orc_moe_prefill(C.byref(layer.s), _p(X), T, k, _p(ids), _p(w), mode, _p(y)), "moe_prefill")
    return y


def moe_decode_baseline(layer: Layer, x_bf16, k: int, norm_topk: bool = True, nthreads: int = 0):
    x = _c(x_bf16, np.uint16).reshape(layer.hidden)
    ids = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    y = np.empty(layer.hidden, np.float32)
    _rc(lib().orc_moe_decode_baseline(C.byref(layer.s), _p(x), k, int(norm_topk), nthreads, _p(ids), _p(w), _p(y)),
        "baseline")
    return ids, w, y


def router_baseline(layer: Layer, x_bf16, k: int, norm_topk: bool = True, nthreads: int = 0):
    """The router of T tokens in shader semantics (f16 logits), OpenMP over tokens."""
    x = _c(x_bf16, np.uint16).reshape(-1, layer.hidden)
    T = x.shape[0]
    ids = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    _rc(lib().orc_router_baseline(C.byref(layer.s), _p(x), T, k, int(norm_topk), nthreads, _p(ids), _p(w)),
        "router_baseline")
    return ids, w


def moe_prefill_baseline(layer: Layer, X_bf16, ids, w, nthreads: int = 0) -> np.ndarray:
    """Grouped prefill in the shader semantics of matmul_dequant_4bit.metal -> y fp32 [T, H]."""
    X = _c(X_bf16, np.uint16).reshape(-1, layer.hidden)
    ids, w = _c(ids, np.int32), _c(w, np.float32)
    T, k = ids.shape
    y = np.empty((T, layer.hidden), np.float32)
    _rc(lib().orc_moe_prefill_baseline(C.byref(layer.s), _p(X), T, k, _p(ids), _p(w), nthreads, _p(y)),
        "prefill_baseline")
    return y


def omp_max_threads() -> int:
    return lib().orc_omp_max_threads()


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


# ---- attention half and the whole decoder (forward.rs:398-443, :552-567) ----
def rope_neox(x_bf16, pos: int, theta: float) -> np.ndarray:
    """NeoX RoPE of bf16 [n_heads, head_dim] at `pos` -> new bf16 array (orc_rope_neox)."""
    x = np.array(_c(x_bf16, np.uint16), copy=True)
    _rc(lib().orc_rope_neox(_p(x), x.shape[0], x.shape[1], pos, theta), "rope")
    return x


def sdpa_decode(q_bf16, k_cache, v_cache, seq_len: int, scale: float) -> np.ndarray:
    """GQA single-query attention, fp64 [n_heads, head_dim]; caches bf16 [n_kv, max_len, head_dim]."""
    q, k, v = _c(q_bf16, np.uint16), _c(k_cache, np.uint16), _c(v_cache, np.uint16)
    nh, hd = q.shape
    nkv, ml, _ = k.shape
    out = np.empty((nh, hd), np.float64)
    _rc(lib().orc_sdpa_decode(_p(q), _p(k), _p(v), nh, nkv, hd, ml, seq_len, scale, _p(out)), "sdpa")
    return out


def argmax(x_f32) -> int:
    x = _c(x_f32, np.float32)
    return int(lib().orc_argmax(_p(x), x.size))


def _bf16(a) -> np.ndarray:
    """fp32 (or fp64 rounded to fp32 first) -> bf16 bits, RNE (orc_f32_to_bf16_n)."""
    f = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().orc_f32_to_bf16_n(_p(f), _p(out), f.size)
    return out


def _proj(P: Dict[str, np.ndarray], name: str, x_bf16, in_f: int, out_f: int) -> np.ndarray:
    """4-bit projection in fp64 on the exact weights, rounded to bf16 (the stored activation)."""
    xf = (_c(x_bf16, np.uint16).astype(np.uint32) << 16).view(np.float32)
    y, _ = qmatvec("f64", 4, P[name + "_w"], P[name + "_s"], P[name + "_b"], xf, in_f, out_f)
    return _bf16(y)


def attention_half(P: Dict[str, np.ndarray], x_bf16, k_cache, v_cache, pos: int, cfg: Dict) -> np.ndarray:
    """x1 = bf16(x + o) of one decoder layer for one token at `pos`
    (forward.rs:403-418): projections in fp64 on the exact weights rounded to
    bf16, per-head q/k RMSNorm, NeoX RoPE, k and v into the caches (bf16
    [n_kv, max_len, head_dim], updated in place), attention in fp64 rounded to
    bf16, o projection in fp64 rounded to bf16."""
    H, nh, nkv, hd = cfg["hidden"], cfg["n_heads"], cfg["n_kv"], cfg["head_dim"]
    eps, theta = cfg["eps"], cfg["theta"]
    x = _c(x_bf16, np.uint16)
    xn = rmsnorm(x, P["in_norm"], eps)
    q = _proj(P, "q", xn, H, nh * hd).reshape(nh, hd)
    k = _proj(P, "k", xn, H, nkv * hd).reshape(nkv, hd)
    v = _proj(P, "v", xn, H, nkv * hd).reshape(nkv, hd)
    q = rope_neox(rmsnorm(q, P["q_norm"], eps), pos, theta)
    k = rope_neox(rmsnorm(k, P["k_norm"], eps), pos, theta)
    k_cache[:, pos, :] = k
    v_cache[:, pos, :] = v
    attn = _bf16(sdpa_decode(q, k_cache, v_cache, pos + 1, hd ** -0.5)).reshape(-1)
    o = _proj(P, "o", attn, nh * hd, H)
    return _bf16(_f32(x) + _f32(o))


def moe_half(P: Dict[str, np.ndarray], moe: "Layer", x1_bf16, cfg: Dict, ids=None, w=None):
    """x1 + sum_r w_r expert_r(rmsnorm(x1)) in fp64, rounded to bf16
    (forward.rs:419-441); routing from the oracle router unless given.
    Returns (x_out bf16, ids, w)."""
    x1 = _c(x1_bf16, np.uint16)
    x1n = rmsnorm(x1, P["post_norm"], cfg["eps"])
    if ids is None:
        _, ids, w = router(moe, x1n, cfg["top_k"], cfg["norm_topk"])
    y, _, _ = moe_decode(moe, x1n, cfg["top_k"], cfg["norm_topk"], ids=ids, w=w)
    return _bf16(y[0] + _f32(x1)), ids, w


def decoder_layer(P: Dict[str, np.ndarray], moe: "Layer", x_bf16, k_cache, v_cache, pos: int, cfg: Dict):
    """One decoder layer for one token at `pos` (forward.rs:398-443): the
    attention half, then the MoE half. The caches are updated in place."""
    x1 = attention_half(P, x_bf16, k_cache, v_cache, pos, cfg)
    return moe_half(P, moe, x1, cfg)[0]


def _f32(b) -> np.ndarray:
    return (_c(b, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def token_logits(G: Dict[str, np.ndarray], layers, tok: int, caches, pos: int, cfg: Dict) -> np.ndarray:
    """One greedy decode step (run_one_token, forward.rs:552-567): the q4
    embedding row of `tok` (bf16), every layer at `pos`, the final RMSNorm and
    the 4-bit lm_head in fp64. layers: [(P, moe Layer)]; caches: [(k, v)].
    Returns fp64 logits [vocab]."""
    H, V = cfg["hidden"], cfg["vocab"]
    x = _bf16(dequant(4, G["embed_w"][tok:tok + 1], G["embed_s"][tok:tok + 1], G["embed_b"][tok:tok + 1],
                      1, H).reshape(-1))
    for (P, moe), (kc, vc) in zip(layers, caches):
        x = decoder_layer(P, moe, x, kc, vc, pos, cfg)
    xn = rmsnorm(x, G["final_norm"], cfg["eps"])
    xf = (xn.astype(np.uint32) << 16).view(np.float32)
    y, _ = qmatvec("f64", 4, G["lm_w"], G["lm_s"], G["lm_b"], xf, H, V)
    return y


def prefill(G: Dict[str, np.ndarray], layers, tokens, caches, pos0: int, cfg: Dict):
    """prefill_batched (forward.rs:114-261): the embedding rows of `tokens`,
    then layer-major, for every token i in order at position pos0 + i, the
    decoder layer (the reference runs each token's attention with the per-token
    kernels, forward.rs:141-158, so a token attends to the cache entries the
    earlier tokens of the batch wrote), then the final RMSNorm and lm_head of
    the last token. Returns (last layer's rows bf16 [T, hidden], fp64 logits
    [vocab]); the caches are updated in place."""
    H, V = cfg["hidden"], cfg["vocab"]
    xs = [_bf16(dequant(4, G["embed_w"][t:t + 1], G["embed_s"][t:t + 1], G["embed_b"][t:t + 1], 1, H).reshape(-1))
          for t in tokens]
    for (P, moe), (kc, vc) in zip(layers, caches):
        xs = [decoder_layer(P, moe, x, kc, vc, pos0 + i, cfg) for i, x in enumerate(xs)]
    xn = rmsnorm(xs[-1], G["final_norm"], cfg["eps"])
    xf = (xn.astype(np.uint32) << 16).view(np.float32)
    y, _ = qmatvec("f64", 4, G["lm_w"], G["lm_s"], G["lm_b"], xf, H, V)
    return np.stack(xs), y


# ---- independent NumPy restatement (validate_dequant.py:26-30) --------------
def dequant_numpy(W: np.ndarray, S_f32: np.ndarray, B_f32: np.ndarray, group: int = 64) -> np.ndarray:
    """nibble j of uint32 word = (word >> 4j) & 0xF; element i at word i//8,
    nibble i%8; value = nibble*scale[g] + bias[g] (fp32)."""
    Wn = np.asarray(W).astype(np.uint32)
    out_f = Wn.shape[0]
    in_f = Wn.shape[1] * 8
    nib = np.stack([(Wn >> (4 * j)) & 0xF for j in range(8)], -1).reshape(out_f, in_f).astype(np.float32)
    return nib * np.repeat(S_f32, group, axis=1) + np.repeat(B_f32, group, axis=1)


# ---- NumPy replica of the reference's CPU path (validate_dequant.py:24-30) --------
# The reference checks its dequant with a NumPy shift/mask unpack (nibble j of a
# uint32 word = (word >> 4j) & 0xF, value = nibble * scale + bias in fp32);
# these functions run the MoE hot path on that replica with numpy's BLAS for the
# products. They time the reference's CPU path; results agree with the oracle to
# fp32 rounding (the routing softmax uses numpy's exp).
def _bf16f(a) -> np.ndarray:
    return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32)


def dequant8_numpy(W, S_f32, B_f32, group: int = 64) -> np.ndarray:
    """8-bit MLX affine: byte c % 4 of word c // 4 (little-endian), value = byte * scale + bias."""
    Wb = np.ascontiguousarray(W, np.uint32).view(np.uint8).astype(np.float32)
    return Wb * np.repeat(S_f32, group, axis=1) + np.repeat(B_f32, group, axis=1)


def _route_numpy(lg, k: int, norm_topk: bool):
    """moe_routing_topk.metal on f16 logits: softmax, k largest p (lower id on ties), f16 weights."""
    l16 = np.asarray(lg, np.float32).astype(np.float16).astype(np.float32)
    e = np.exp(l16 - l16.max(axis=-1, keepdims=True))
    p = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    ids = np.argsort(-p, axis=-1, kind="stable")[..., :k]
    sel = np.take_along_axis(p, ids, axis=-1)
    w = sel.astype(np.float16).astype(np.float32)
    if norm_topk:
        ws = sel.sum(axis=-1, keepdims=True, dtype=np.float32)
        w = np.where(ws > 0, (w / ws).astype(np.float16).astype(np.float32), w)
    return ids.astype(np.int32), w


def router_numpy(t: Dict[str, np.ndarray], X_bf16, k: int, norm_topk: bool = True):
    """Router of T tokens: 8-bit dequant + X @ W^T, then the f16 routing rule."""
    Wr = dequant8_numpy(t["router_w"], _bf16f(t["router_s"]), _bf16f(t["router_b"]))
    return _route_numpy(_bf16f(X_bf16).reshape(-1, Wr.shape[1]) @ Wr.T, k, norm_topk)


def _expert_mats(t, e):
    g = dequant_numpy(t["gate_w"][e], _bf16f(t["gate_s"][e]), _bf16f(t["gate_b"][e]))
    u = dequant_numpy(t["up_w"][e], _bf16f(t["up_s"][e]), _bf16f(t["up_b"][e]))
    d = dequant_numpy(t["down_w"][e], _bf16f(t["down_s"][e]), _bf16f(t["down_b"][e]))
    return g, u, d


def decode_layer_numpy(t: Dict[str, np.ndarray], x_bf16, k: int, norm_topk: bool = True) -> np.ndarray:
    """The decode MoE half for one token: router, then per chosen expert the
    dequantized gate/up/down products and SwiGLU, weighted sum in rank order."""
    x = _bf16f(x_bf16).reshape(-1)
    ids, w = router_numpy(t, x_bf16, k, norm_topk)
    y = np.zeros(x.shape[0], np.float32)
    for e, we in zip(ids[0], w[0]):
        g, u, d = _expert_mats(t, e)
        gv, uv = g @ x, u @ x
        y += we * (d @ (gv / (1.0 + np.exp(-gv)) * uv))
    return y


def prefill_numpy(t: Dict[str, np.ndarray], X_bf16, ids, w) -> np.ndarray:
    """Grouped prefill with given routing: per expert, its tokens' rows through
    the dequantized gate/up/down products, then the rank-order combine."""
    X = _bf16f(X_bf16).reshape(ids.shape[0], -1)
    T, k = ids.shape
    Ye = np.zeros((T, k, X.shape[1]), np.float32)
    for e in np.unique(ids):
        rows = np.nonzero(ids == e)
        g, u, d = _expert_mats(t, e)
        Xe = X[rows[0]]
        G, U = Xe @ g.T, Xe @ u.T
        Ye[rows] = (G / (1.0 + np.exp(-G)) * U) @ d.T
    return np.einsum("tk,tkh->th", w, Ye, optimize=False)
