"""The benched decoder step at its full Qwen3-30B-A3B shape: one layer of
hidden 2048, 32 query / 4 kv heads of 128, a 128-expert top-8
MoE block of inter 768 with its post-attention norm, a KV cache of 4,096
positions already holding 4,000, and the 151,936-row 4-bit lm_head. The step
runs the same one-launch attention and MoE kernels as the benched 48-layer
graph (forward.rs:398-443, :552-567).

Bars: the attention half within 1e-2 of the fp64 oracle, the appended key and
value within 1e-2, routing ids and weights bit-exact with the oracle router on
the GPU's post-attention row, the MoE half within 1e-2 of fp64, every logit
finite and within 1e-2 of the fp64 lm_head on the GPU's last row, and the
greedy token equal to the argmax of the GPU's own logits."""
import numpy as np
import pytest

import oracle as O
from obsidian_hip import decoder as D
from obsidian_hip import synth

pytestmark = pytest.mark.gpu


def _f(b):
    return synth.bf16_bits_to_f32(b).astype(np.float64)


def _close(got, want, tol=1e-2, floor_mult=1.0):
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    assert rel <= tol, rel
    floor = floor_mult * tol * np.sqrt(np.mean(want ** 2))
    assert np.all(np.abs(got - want) <= tol * np.abs(want) + floor)
    return rel


def test_full_shape_layer_and_head(exe):
    cfg = D.DecoderConfig(n_layers=1, max_len=4096)
    ocfg = {"hidden": cfg.hidden, "n_heads": cfg.n_heads, "n_kv": cfg.n_kv, "head_dim": cfg.head_dim,
            "eps": cfg.rms_eps, "theta": cfg.rope_theta, "top_k": cfg.top_k, "norm_topk": cfg.norm_topk,
            "vocab": cfg.vocab}
    layers, glob = synth.decoder_weights(21, 1, cfg.hidden, cfg.n_heads, cfg.n_kv, cfg.head_dim, cfg.n_exp,
                                         cfg.inter, cfg.vocab)
    pos, tok = 4000, 123457
    rng = np.random.default_rng(22)
    kc = np.zeros((cfg.n_kv, cfg.max_len, cfg.head_dim), np.uint16)
    vc = np.zeros_like(kc)
    kc[:, :pos] = synth.bf16_normal(rng, (cfg.n_kv, pos, cfg.head_dim))
    vc[:, :pos] = synth.bf16_normal(rng, (cfg.n_kv, pos, cfg.head_dim))
    dl, dg = D.upload_weights(exe, layers, glob)
    dk, dv = exe.upload(kc), exe.upload(np.ascontiguousarray(vc.transpose(0, 2, 1)))
    m = D.Model(exe, cfg, dl, dg, caches=[(dk, dv)])
    assert m.fused_attention()
    ids = exe.alloc(cfg.top_k, np.int32)
    w = exe.alloc(cfg.top_k, np.float32)
    try:
        m.set_state(pos, tok)
        m.embed()
        x_in = m.x.download()
        m.forward_layer(0, ids, w)
        x1, x_out = m.x1.download(), m.x.download()
        m.head()
        logits = m.logits.download()
        pos2, tok2 = m.read_state()  # checks the device status too
        gk, gv = dk.download()[:, pos], dv.download()[:, :, pos]
    finally:
        m.close()
    want_x = synth.f32_to_bf16_bits(O.dequant(4, glob["embed_w"][tok:tok + 1], glob["embed_s"][tok:tok + 1],
                                              glob["embed_b"][tok:tok + 1], 1, cfg.hidden)[0])
    assert np.array_equal(x_in, want_x)
    kc_o, vc_o = kc.copy(), vc.copy()
    x1_ref = O.attention_half(layers[0], x_in, kc_o, vc_o, pos, ocfg)
    r_attn = _close(_f(x1), _f(x1_ref))
    _close(_f(gk), _f(kc_o[:, pos]), 1e-2, 2.0)
    _close(_f(gv), _f(vc_o[:, pos]), 1e-2, 2.0)
    moe = O.Layer(layers[0], cfg.n_exp, cfg.hidden, cfg.inter)
    out_ref, ri, rw = O.moe_half(layers[0], moe, x1, ocfg)
    assert np.array_equal(ids.download(), ri[0]) and np.array_equal(w.download().view(np.uint32), rw[0].view(np.uint32))
    r_moe = _close(_f(x_out), _f(out_ref))
    assert np.all(np.isfinite(logits))
    xn = O.rmsnorm(x_out, glob["final_norm"], cfg.rms_eps)
    ref, _ = O.qmatvec("f64", 4, glob["lm_w"], glob["lm_s"], glob["lm_b"], synth.bf16_bits_to_f32(xn),
                       cfg.hidden, cfg.vocab)
    r_head = _close(logits.astype(np.float64), ref, 1e-2, 2.0)
    assert (pos2, tok2) == (pos + 1, O.argmax(logits))
    print(f"full shape: attention {r_attn:.2e}, moe {r_moe:.2e}, lm_head {r_head:.2e}, token {tok2}")
