"""The decoder around the MoE block: the host mirror of the reference's Model
(src/forward.rs:30-53, :398-443, :445-462, :552-567) over the C ABI.

A decode step is embed -> for each layer (input RMSNorm, q/k/v projections in
one mat-vec launch, q/k norm + RoPE + cache append, GQA attention, o
projection with the residual add, then the fused MoE block with its
post-attention norm and residual) -> final RMSNorm -> lm_head -> argmax. The
position and token live in a device array, so the whole step is captured once
as a HIP graph and replayed for every token (the reference commits one Metal
command buffer per dispatch instead, forward.rs:289-301).

Every kernel runs through libobsidian_hip; there is no CPU path.
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

from . import (OBS_DECODE_MULTI, OBS_PATH_FUSED_ATTN, OBS_PATH_FUSED_DECODE, DeviceBuffer, MoeConfig, MoeLayer,
               ObsError, ObsidianExecutor, _ptr, lib)


@dataclass
class DecoderConfig:
    """Qwen3MoeConfig (src/model.rs:7-23) plus the cache length."""
    n_layers: int = 48
    hidden: int = 2048
    n_heads: int = 32
    n_kv: int = 4
    head_dim: int = 128
    n_exp: int = 128
    top_k: int = 8
    inter: int = 768
    vocab: int = 151936
    rms_eps: float = 1e-6
    rope_theta: float = 1e7
    norm_topk: bool = True
    group: int = 64
    max_len: int = 4096  # KV cache positions (forward.rs:60-63 defaults to 16384)

    def moe(self) -> MoeConfig:
        return MoeConfig(self.n_exp, self.top_k, self.hidden, self.inter, self.group, self.norm_topk, self.rms_eps)


# Per-layer tensors (names of the checkpoint's model.layers.{l}.* entries):
#   in_norm (input_layernorm.weight), q_w/q_s/q_b, k_*, v_*, o_* (self_attn.*_proj),
#   q_norm, k_norm (self_attn.{q,k}_norm.weight), post_norm (post_attention_layernorm.weight)
#   and the MoE tables (PROJ_KEYS of MoeLayer).
# Global tensors: embed_w/s/b (model.embed_tokens), final_norm (model.norm), lm_w/s/b (lm_head).
ATTN_KEYS = ("in_norm", "q_w", "q_s", "q_b", "k_w", "k_s", "k_b", "v_w", "v_s", "v_b", "o_w", "o_s", "o_b",
             "q_norm", "k_norm", "post_norm")
GLOBAL_KEYS = ("embed_w", "embed_s", "embed_b", "final_norm", "lm_w", "lm_s", "lm_b")


class Model:
    """forward.rs:30-53. `layers` holds per-layer dicts of device pointers (or
    DeviceBuffers) with ATTN_KEYS plus a MoeLayer under "moe"; `glob` holds
    GLOBAL_KEYS. The KV caches, activations and workspaces are allocated here
    once (forward.rs:56-104 allocates the pools once too)."""

    def __init__(self, exe: ObsidianExecutor, cfg: DecoderConfig, layers: List[Dict], glob: Dict,
                 caches: Optional[List] = None):
        """caches: optional per-layer (keys, transposed values) device buffers or
        pointers (bf16 [n_kv, max_len, head_dim] and [n_kv, head_dim, max_len]);
        zeroed ones are allocated otherwise (KvCache::new, kv_cache.rs:15-24)."""
        self.exe, self.cfg, self.layers, self.glob = exe, cfg, layers, glob
        c = cfg
        if c.n_heads * c.head_dim not in (2048, 4096) or c.hidden not in (2048, 4096):
            raise ValueError("the fused mat-vec needs hidden and n_heads * head_dim in {2048, 4096}")
        if caches is not None and len(caches) != c.n_layers:
            raise ValueError("one (keys, values) cache pair per layer")
        self.caches = caches if caches is not None else [
            (exe.zeros((c.n_kv, c.max_len, c.head_dim), np.uint16), exe.zeros((c.n_kv, c.head_dim, c.max_len), np.uint16))
            for _ in range(c.n_layers)]
        self.state = exe.zeros(2, np.int32)              # {pos, tok}
        self.x = exe.alloc(c.hidden, np.uint16)          # residual stream (layer input and output)
        self.x1 = exe.alloc(c.hidden, np.uint16)         # after attention
        self.q = exe.alloc(c.n_heads * c.head_dim, np.uint16)
        self.k = exe.alloc(c.n_kv * c.head_dim, np.uint16)
        self.v = exe.alloc(c.n_kv * c.head_dim, np.uint16)
        self.attn = exe.alloc(c.n_heads * c.head_dim, np.uint16)
        self.logits = exe.alloc(c.vocab, np.float32)
        self.sdpa_ws = exe.alloc(exe.sdpa_workspace(c.n_heads, c.n_kv, c.head_dim, c.max_len), np.uint8)
        self.argmax_ws = exe.alloc(lib().obs_argmax_workspace(), np.uint8)
        self.moe_cfg = c.moe()
        self.graph: Optional[int] = None
        self._pf: Optional[Dict] = None      # prefill buffers, grown to the largest batch
        self.use_fused_attention = True      # one-launch attention half where the shape allows
        self.use_fused_layer = True          # ... and both halves of a layer in one launch
        self.last_seq: List[int] = []        # the tokens whose keys and values the caches hold (run_turn)
        self.last_reused = 0
        self.last_prefilled = 0
        self.last_fallback: Optional[str] = None  # why the last turn's batched prefill fell back, if it did

    # -- the pieces of forward_layer (forward.rs:398-443) ------------------
    def fused_attention(self) -> bool:
        """Whether the attention half runs as one launch (obs_attn_decode: the
        Qwen3-30B-A3B attention shape on a device whose dispatch allows it: 256
        CUs, each group b % 8 of workgroups on one XCD)."""
        c = self.cfg
        return (self.use_fused_attention and (c.hidden, c.n_heads, c.n_kv, c.head_dim) == (2048, 32, 4, 128)
                and bool(self.exe.paths() & OBS_PATH_FUSED_ATTN))

    def fused_moe(self) -> bool:
        """Whether the MoE half can share the attention half's launch
        (obs_layer_decode): the one-launch MoE shape (hidden 2048, inter 768,
        top-8, group 64, at most 256 experts) on a device whose dispatch allows
        the one-launch decode, unless the context is set to the 4-launch path."""
        m = self.moe_cfg
        return ((m.hidden, m.inter, m.top_k, m.group) == (2048, 768, 8, 64) and m.n_exp <= 256
                and bool(self.exe.paths() & OBS_PATH_FUSED_DECODE) and self.exe.decode_path != OBS_DECODE_MULTI)

    def forward_layer(self, il: int, ids_out=None, w_out=None) -> None:
        """self.x <- layer il of self.x at the state's position (ids_out, w_out:
        optional device buffers for the layer's routing)."""
        c, e, L = self.cfg, self.exe, self.layers[il]
        kc, vc = self.caches[il]
        qd, kvd = c.n_heads * c.head_dim, c.n_kv * c.head_dim
        if self.fused_attention() and self.use_fused_layer and self.fused_moe():  # forward.rs:398-443, one launch
            e.layer_decode(L, self.moe_cfg, L["moe"], self.x, kc, vc, c.max_len, c.rms_eps, c.rope_theta, self.state,
                           self.x1, self.x, ids_out=ids_out, w_out=w_out)
            return
        if self.fused_attention():  # forward.rs:403-418 in one launch
            e.attn_decode(L, self.x, kc, vc, c.max_len, c.rms_eps, c.rope_theta, self.state, self.x1)
            e.moe_decode(self.moe_cfg, L["moe"], self.x1, self.x, residual=self.x1, ids_out=ids_out, w_out=w_out)
            return
        # input RMSNorm (forward.rs:403) fused into the q/k/v mat-vec
        e.q4_gemv(self.x, c.hidden, [(L["q_w"], L["q_s"], L["q_b"], qd, None, self.q, None),
                                     (L["k_w"], L["k_s"], L["k_b"], kvd, None, self.k, None),
                                     (L["v_w"], L["v_s"], L["v_b"], kvd, None, self.v, None)],
                  norm_w=L["in_norm"], eps=c.rms_eps)
        e.attn_prep(self.q, self.k, self.v, L["q_norm"], L["k_norm"], kc, vc, c.n_heads, c.n_kv, c.head_dim,
                    c.max_len, c.rms_eps, c.rope_theta, self.state)
        e.sdpa_decode(self.q, kc, vc, self.attn, c.n_heads, c.n_kv, c.head_dim, c.max_len, self.state, self.sdpa_ws)
        e.q4_gemv(self.attn, qd, [(L["o_w"], L["o_s"], L["o_b"], c.hidden, None, self.x1, self.x)])
        e.moe_decode(self.moe_cfg, L["moe"], self.x1, self.x, residual=self.x1, ids_out=ids_out, w_out=w_out)

    def embed(self) -> None:
        """forward.rs:445-462: self.x <- bf16 row state[1] of the 4-bit embedding table."""
        g, c = self.glob, self.cfg
        self.exe.embed_q4(g["embed_w"], g["embed_s"], g["embed_b"], c.hidden, c.vocab, self.state, self.x, c.group)

    def head(self, x=None) -> None:
        """forward.rs:559-566: final norm, lm_head logits (fp32), greedy token into
        the state, position advanced. x: the hidden row (default self.x)."""
        g, c, e = self.glob, self.cfg, self.exe
        e.q4_gemv(self.x if x is None else x, c.hidden,
                  [(g["lm_w"], g["lm_s"], g["lm_b"], c.vocab, self.logits, None, None)],
                  norm_w=g["final_norm"], eps=c.rms_eps)  # final RMSNorm (forward.rs:560) fused
        e.argmax(self.logits, c.vocab, self.state, self.argmax_ws)

    def step(self) -> None:
        """run_one_token (forward.rs:552-567) without the host read: enqueue one
        whole decode step."""
        self.embed()
        for il in range(self.cfg.n_layers):
            self.forward_layer(il)
        self.head()

    # -- state and graph ---------------------------------------------------
    def set_state(self, pos: int, tok: int) -> None:
        if not 0 <= pos < self.cfg.max_len:
            raise ValueError(f"position {pos} outside the cache (max_len {self.cfg.max_len})")
        self.state.upload(np.array([pos, tok], np.int32))

    def read_state(self):
        """(position, token) after the queued steps; raises if a fused kernel
        of those steps recorded a device-side failure (a cross-workgroup wait
        that timed out), whose outputs, and so this token, would be invalid."""
        self.exe.device_status()
        pos, tok = self.state.download()
        return int(pos), int(tok)

    def capture(self) -> int:
        """Record one step as a graph. One eager step runs first (and its state
        is restored) so that every workspace exists before the capture; it
        writes the cache entries at the current position, which the next step
        at that position writes again with the same values."""
        if self.graph is None:
            saved = self.state.download()
            self.step()
            self.state.upload(saved)
            self.exe.capture_begin()
            try:
                self.step()
            finally:
                self.graph = self.exe.capture_end()
        return self.graph

    def replay(self, n: int = 1) -> None:
        g = self.capture()
        for _ in range(n):
            self.exe.graph_launch(g)

    def run_one_token(self, tok: int, pos: int) -> int:
        """forward.rs:552-567: next greedy token after `tok` at `pos`."""
        self.set_state(pos, tok)
        self.step()
        return self.read_state()[1]

    def generate(self, tok: int, pos: int, n: int, graph: bool = True) -> List[int]:
        """n greedy tokens after `tok` at `pos` (one step per token)."""
        if pos + n > self.cfg.max_len:
            raise ValueError("generation runs past the cache")
        self.set_state(pos, tok)
        out = []
        for _ in range(n):
            if graph:
                self.replay(1)
            else:
                self.step()
            out.append(self.read_state()[1])
        return out

    # -- prefill (forward.rs:114-261) ------------------------------------------
    def _prefill_buffers(self, T: int) -> Dict:
        c, e = self.cfg, self.exe
        if self._pf is None or self._pf["T"] < T:
            self._pf = None  # release the smaller set first
            qd, kvd = c.n_heads * c.head_dim, c.n_kv * c.head_dim
            self._pf = {
                "T": T, "tokens": e.alloc(T, np.int32),
                "x": e.alloc((T, c.hidden), np.uint16), "x2": e.alloc((T, c.hidden), np.uint16),
                "xn": e.alloc((T, c.hidden), np.uint16), "q": e.alloc((T, qd), np.uint16),
                "k": e.alloc((T, kvd), np.uint16), "v": e.alloc((T, kvd), np.uint16),
                "attn": e.alloc((T, qd), np.uint16), "o": e.alloc((T, c.hidden), np.uint16),
                "qkv": e.alloc((T, qd + 2 * kvd), np.uint16),
                "ws": e.alloc(e.moe_prefill_workspace(self.moe_cfg, T), np.uint8),
            }
        return self._pf

    def fused_qkv(self, il: int):
        """(w, s, b) of layer il's q, k and v projections as one [q + k + v rows,
        hidden] matrix when they are stored back to back (upload_weights and
        the checkpoint layout here place them so), else None."""
        c, L = self.cfg, self.layers[il]
        qd, kvd, H = c.n_heads * c.head_dim, c.n_kv * c.head_dim, c.hidden
        out = []
        for kind, row_bytes in (("w", H // 2), ("s", H // c.group * 2), ("b", H // c.group * 2)):
            q, k, v = (_ptr(L[f"{p}_{kind}"]) for p in "qkv")
            if k != q + qd * row_bytes or v != k + kvd * row_bytes:
                return None
            out.append(q)
        return tuple(out)

    def prefill_layers(self, tokens, pos0: int, trace: Optional[list] = None):
        """The layer loop of prefill_batched (forward.rs:134-238): embed the T
        tokens, then per layer, for all of them at once, the input RMSNorm,
        q/k/v as 4-bit GEMMs, q/k norm + RoPE + cache appends at pos0 + t,
        causal attention, o as a GEMM plus the residual, and the MoE prefill
        (post-attention norm, GPU routing and grouping, grouped GEMMs,
        rank-order combine with the residual). With OBSIDIAN_NO_GEMM set
        (forward.rs:124-126, read per call like the reference's switch) the MoE
        half runs token by token through the decode path instead of the
        grouped GEMMs (forward.rs:233-247), the anchor the grouped path is
        checked against at full size. Returns the buffer holding the last
        layer's output rows [T, hidden]. trace: a list that receives, per
        layer, host copies (input rows, rows after attention, output rows)."""
        c, e, g = self.cfg, self.exe, self.glob
        toks = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        T = int(toks.size)
        if T == 0:
            raise ValueError("empty prompt")
        if pos0 < 0 or pos0 + T > c.max_len:
            raise ValueError(f"context overflow: positions {pos0}..{pos0 + T} past max_len {c.max_len}")
        no_gemm = "OBSIDIAN_NO_GEMM" in os.environ
        B = self._prefill_buffers(T)
        e._check(lib().obs_upload(e.ctx, B["tokens"].ptr, toks.ctypes.data, toks.nbytes))
        qd, kvd, H = c.n_heads * c.head_dim, c.n_kv * c.head_dim, c.hidden
        e.embed_q4_rows(g["embed_w"], g["embed_s"], g["embed_b"], H, c.vocab, B["tokens"], T, B["x"], c.group)
        x, x2 = B["x"], B["x2"]
        for il in range(c.n_layers):
            L = self.layers[il]
            kc, vc = self.caches[il]
            if trace is not None:
                stages = [x.download()[:T].copy()]
            e.rmsnorm_raw(x, L["in_norm"], B["xn"], T, H, c.rms_eps)                           # :145
            fused = self.fused_qkv(il)
            if fused is not None:  # q, k, v as one GEMM; their column ranges of each output row
                ld = qd + 2 * kvd
                e.q4_matmul(*fused, B["xn"], B["qkv"], T, H, ld, c.group)                     # :146-148
                q, k, v = B["qkv"].ptr, B["qkv"].ptr + 2 * qd, B["qkv"].ptr + 2 * (qd + kvd)
                ldq = ldkv = ld
            else:
                e.q4_matmul(L["q_w"], L["q_s"], L["q_b"], B["xn"], B["q"], T, H, qd, c.group)
                e.q4_matmul(L["k_w"], L["k_s"], L["k_b"], B["xn"], B["k"], T, H, kvd, c.group)
                e.q4_matmul(L["v_w"], L["v_s"], L["v_b"], B["xn"], B["v"], T, H, kvd, c.group)
                q, k, v, ldq, ldkv = B["q"], B["k"], B["v"], 0, 0
            e.attn_prep_rows(q, k, v, L["q_norm"], L["k_norm"], kc, vc, c.n_heads, c.n_kv, c.head_dim,
                             c.max_len, c.rms_eps, c.rope_theta, pos0, T, ldq, ldkv)            # :149-153
            e.sdpa_prefill(q, kc, vc, B["attn"], c.n_heads, c.n_kv, c.head_dim, c.max_len, pos0, T, ldq)  # :155
            e.q4_matmul(L["o_w"], L["o_s"], L["o_b"], B["attn"], B["o"], T, qd, H, c.group)    # :156
            e.scaled_add_raw(x, B["o"], 1.0, T * H)                                             # x1 = x + o
            if trace is not None:
                stages.append(x.download()[:T].copy())
            if no_gemm:  # per-token expert mat-vecs (forward.rs:233-247): one decode MoE call per row
                for t in range(T):
                    off = t * H * 2
                    e.moe_decode(self.moe_cfg, L["moe"], x.ptr + off, x2.ptr + off, residual=x.ptr + off)
            else:
                e.moe_prefill(self.moe_cfg, L["moe"], x, x2, T, residual=x, ws=B["ws"])         # :162-238
            x, x2 = x2, x
            if trace is not None:
                trace.append(tuple(stages) + (x.download()[:T].copy(),))
        return x

    def prefill(self, tokens, pos0: int) -> int:
        """prefill_batched (forward.rs:114-261): the tokens at positions
        pos0.. through every layer, layer-major, then the final norm, lm_head
        and greedy pick of the last one. Returns the next token; the state
        becomes (pos0 + T, next token)."""
        T = len(tokens)
        if T == 0:
            raise ValueError("empty prompt")
        self.set_state(pos0 + T - 1, 0)  # the head's argmax advances it; the layers take pos0 directly
        x = self.prefill_layers(tokens, pos0)
        self.head(x.ptr + (T - 1) * self.cfg.hidden * 2)                                         # :240-261
        return self.read_state()[1]

    def fill_kv(self, tok: int, pos: int) -> None:
        """forward.rs:543-550: one token through every layer (its keys and values
        into the caches) without the lm_head."""
        self.set_state(pos, tok)
        self.embed()
        for il in range(self.cfg.n_layers):
            self.forward_layer(il)

    def run_turn(self, prompt, max_new: int, eos: int, batch_min: int = 24) -> List[int]:
        """forward.rs:471-535: one turn with prefix reuse. The caches keep the
        previous turn's tokens (last_seq); the longest common prefix with this
        prompt is reused and only the rest is prefilled (batched from
        batch_min tokens, token by token below), keeping at least the last
        prompt token; then greedy decode until max_new tokens or eos."""
        prompt = [int(t) for t in prompt]
        if not prompt:
            return []
        cap = self.cfg.max_len
        if len(prompt) + max_new > cap:  # keep the prompt's tail (forward.rs:477-482)
            keep = min(max(cap - (max_new + 1), 0), len(prompt))
            if keep == 0:
                raise ValueError(f"max_new {max_new} leaves no room for the prompt in the cache ({cap})")
            prompt = prompt[len(prompt) - keep:]
        lcp = 0
        while lcp < min(len(self.last_seq), len(prompt)) and self.last_seq[lcp] == prompt[lcp]:
            lcp += 1
        lcp = min(lcp, len(prompt) - 1)
        suffix = prompt[lcp:]
        # batched from batch_min tokens unless OBSIDIAN_NO_BATCH is set; a failed
        # batched prefill falls back to per-token steps (forward.rs:494-507),
        # which write the same cache positions again
        self.last_fallback = None
        nxt = None
        if len(suffix) >= batch_min and "OBSIDIAN_NO_BATCH" not in os.environ:
            try:
                nxt = self.prefill(suffix, lcp)
            except ObsError as e:
                self.last_fallback = str(e)
        if nxt is None:
            for i, tk in enumerate(suffix[:-1]):
                self.fill_kv(tk, lcp + i)
            nxt = self.run_one_token(suffix[-1], len(prompt) - 1)
        gen = [nxt]
        pos = len(prompt)
        while len(gen) < max_new and nxt != eos and pos < cap:
            self.set_state(pos, nxt)  # run_one_token as a replay of the captured step
            self.replay(1)
            nxt = self.read_state()[1]
            gen.append(nxt)
            pos += 1
        # the tokens whose keys and values the caches hold: the last generated
        # token was never fed (the reference records it too, forward.rs:521-523,
        # so a next prompt that repeats it would reuse a cache slot never written)
        self.last_seq = prompt + gen[:-1]
        self.last_reused = lcp
        self.last_prefilled = len(prompt) - lcp
        return gen

    def close(self) -> None:
        if self.graph is not None:
            ObsidianExecutor.graph_destroy(self.graph)
            self.graph = None


def upload_weights(exe: ObsidianExecutor, layers: List[Dict[str, np.ndarray]], glob: Dict[str, np.ndarray]):
    """Host arrays -> device buffers in the layout Model expects (layers[i]
    holds ATTN_KEYS and the MoE PROJ_KEYS)."""
    dl = []
    for t in layers:
        qkv_keys = {f"{p}_{kind}" for p in "qkv" for kind in "wsb"}
        d = {k: exe.upload(t[k]) for k in ATTN_KEYS if k not in qkv_keys}
        for kind in "wsb":  # q, k, v back to back (one matrix for the prefill GEMM)
            buf = exe.upload(np.concatenate([t[f"{p}_{kind}"] for p in "qkv"]))
            d[f"_qkv_{kind}"] = buf
            rows = [t[f"{p}_{kind}"].shape[0] for p in "qkv"]
            row_bytes = t[f"q_{kind}"].nbytes // rows[0]
            d[f"q_{kind}"] = buf.ptr
            d[f"k_{kind}"] = buf.ptr + rows[0] * row_bytes
            d[f"v_{kind}"] = buf.ptr + (rows[0] + rows[1]) * row_bytes
        moe = {k: t[k] for k in t if k not in ATTN_KEYS}
        moe["norm_w"] = t["post_norm"]
        d["moe"] = MoeLayer.upload(exe, moe)
        dl.append(d)
    dg = {k: exe.upload(glob[k]) for k in GLOBAL_KEYS}
    return dl, dg
