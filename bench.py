#!/usr/bin/env python3
"""bench.py — MoE expert hot path on one MI355X.

Workload (one "step"): the decode MoE half of a 48-layer Qwen3-30B-A3B-shaped
model for one token (T=1): per layer 8-bit router over 128 experts -> top-8 ->
8 x (4-bit gate/up [768, 2048] + SwiGLU + down [2048, 768]) -> weighted
combine. The 48-layer expert table (16.3 GB, random bits, bf16 scales/biases)
is resident in HBM; layers run back to back on one stream, each with its own
seeded input, replayed from a HIP graph. Several input sets rotate so expert
weights stream from HBM rather than the 256 MB Infinity Cache.

value = algorithmic bytes per layer (8 experts x 2,654,208 B + router
278,528 B + 8,192 B activations) / measured time per layer, in GB/s.
Also reported: prefill grouped GEMM TFLOP/s (T=2048, Zipf routing), the
dominant kernel's roofline and the reference CPU path timed on this host.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "project-obsidian_amd"))

METRIC = "MoE-layer decode µs + HBM GB/s (% peak); prefill grouped-GEMM TFLOP/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

E, K, H, I, G = 128, 8, 2048, 768, 64
PROJ_BYTES = I * H // 2 + 2 * 2 * (I * H // G)          # 884,736
EXPERT_BYTES = 3 * PROJ_BYTES                              # 2,654,208
ROUTER_BYTES = E * H + 2 * 2 * (E * H // G)                # 278,528
LAYER_BYTES = K * EXPERT_BYTES + ROUTER_BYTES + 2 * 2 * H  # 21,520,384
GATEUP_BYTES = K * 2 * PROJ_BYTES + 2 * H                  # per decode_gateup launch
PREFILL_T = 2048
PREFILL_FLOP = 2 * PREFILL_T * K * 3 * H * I               # 154,618,822,656


def gpu_table(torch, n_layers, seed):
    """Stacked switch_mlp tensors + 8-bit router per layer, generated on the GPU."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    dev = "cuda"

    def words(*shape):
        return torch.randint(-2**31, 2**31, shape, dtype=torch.int32, device=dev, generator=gen)

    def scales(*shape):
        return (torch.randn(shape, device=dev, generator=gen) * 0.02).abs().to(torch.bfloat16)

    def biases(*shape):
        return (torch.randn(shape, device=dev, generator=gen) * 0.01).to(torch.bfloat16)

    layers = []
    for _ in range(n_layers):
        t = {}
        for p, (r, c) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            t[p + "_w"] = words(E, r, c // 8)
            t[p + "_s"] = scales(E, r, c // G)
            t[p + "_b"] = biases(E, r, c // G)
        t["router_w"] = words(E, H // 4)
        t["router_s"] = scales(E, H // G)
        t["router_b"] = biases(E, H // G)
        layers.append(t)
    return layers


def bench_decode(torch, oh, exe, args):
    n_layers = args.layers
    table = gpu_table(torch, n_layers, 1234)
    layers = [oh.MoeLayer({k: v.data_ptr() for k, v in t.items()}) for t in table]
    cfg = oh.MoeConfig(E, K, H, I, G, True)
    n_sets = args.input_sets
    gen = torch.Generator(device="cuda")
    gen.manual_seed(99)
    xs = [torch.randn((n_layers, H), device="cuda", generator=gen).to(torch.bfloat16) for _ in range(n_sets)]
    ys = [torch.empty((n_layers, H), dtype=torch.bfloat16, device="cuda") for _ in range(n_sets)]
    torch.cuda.synchronize()

    def sweep(s):
        for l in range(n_layers):
            exe.moe_decode(cfg, layers[l], xs[s][l].data_ptr(), ys[s][l].data_ptr())

    sweep(0)  # allocates the context workspace before capture
    exe.sync()
    graphs = []
    for s in range(n_sets):
        exe.capture_begin()
        sweep(s)
        graphs.append(exe.capture_end())
    for i in range(args.warmup):
        exe.graph_launch(graphs[i % n_sets])
    exe.sync()
    torch.cuda.synchronize()
    exe.timer_start()
    for i in range(args.steps):
        exe.graph_launch(graphs[i % n_sets])
    ms = exe.timer_stop()
    exe.device_status()  # a timed-out wait in a fused launch would make the timing meaningless
    torch.cuda.synchronize()
    ms_step = ms / args.steps
    us_layer = ms_step * 1000.0 / n_layers
    gbs = LAYER_BYTES * n_layers / (ms_step * 1e-3) / 1e9

    # dominant kernel: every launch of a sweep bracketed by HIP events on the
    # context's stream; a hold kernel first lets the host queue the whole sweep
    # so no host gap falls inside an event pair.
    exe.profile_clear()
    for r in range(args.prof_reps):
        exe.stream_hold(30000)
        exe.profile_enable(True)
        sweep(r % n_sets)
        exe.profile_enable(False)
        exe.profile_accumulate()
    exe.device_status()
    stats = exe.profile_stats()
    exe.profile_clear()
    for g in graphs:
        exe.graph_destroy(g)
    kernels = {n: {"avg_us": 1000.0 * t / c, "launches": c} for n, (t, c) in stats.items()}
    # The fused path is one launch per layer, so its average launch duration
    # is the timed region (HIP events on the context's stream around the graph
    # replays) divided by the launches in it; the per-launch event pairs above
    # add the event records' own overhead and are reported beside it. The
    # 4-launch path's largest kernel is gate/up, timed by its event pairs.
    roof = None
    if "decode_fused" in kernels:
        name, nbytes, us = "decode_fused", LAYER_BYTES, us_layer
    elif "decode_gateup" in kernels:
        name, nbytes, us = "decode_gateup", GATEUP_BYTES, kernels["decode_gateup"]["avg_us"]
    else:
        name = None
    if name is not None:
        ach = nbytes / (us * 1e-6) / 1e9
        traffic, prov = measured_traffic(name)
        roof = {"kernel": name, "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": prov,
                "bytes_per_launch": nbytes, "avg_launch_us": round(us, 3),
                "event_pair_us": round(kernels[name]["avg_us"], 3)}
    del table, xs, ys
    torch.cuda.empty_cache()
    return {"ms_step": ms_step, "us_layer": us_layer, "gbs": gbs, "kernels": kernels, "roofline": roof}


def bench_router(torch, oh, exe, reps=200):
    """The router on the GPU: 8-bit gate logits + softmax/top-8 for T = 1
    and T = 512 tokens (gate_gpu + MoeRouter.route_dispatch, forward.rs:386-397,
    router.rs:62-83), as one launch (obs_route: T{T}_us) and as the two calls
    (obs_q8_gate_logits + obs_route_topk: T{T}_us_two_launches). Each form is
    captured `reps` times in one graph; the time per call is the replay time
    over reps."""
    t = gpu_table(torch, 1, 555)[0]
    w8, s8, b8 = (t[k].data_ptr() for k in ("router_w", "router_s", "router_b"))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    out = {}
    for T in (1, 512):
        x = torch.randn((T, H), device="cuda", generator=gen).to(torch.bfloat16)
        lg = torch.empty((T, E), dtype=torch.float32, device="cuda")
        ids = torch.empty((T, K), dtype=torch.int32, device="cuda")
        w = torch.empty((T, K), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()

        def two_calls():
            exe.q8_gate_logits(w8, s8, b8, x.data_ptr(), lg.data_ptr(), T, H, E)
            exe.route_topk(lg.data_ptr(), ids.data_ptr(), w.data_ptr(), T, E, K, True)

        def one_launch():
            exe.route(w8, s8, b8, x.data_ptr(), lg.data_ptr(), ids.data_ptr(), w.data_ptr(), T, H, E, K, True)

        for name, call in ((f"T{T}_us_two_launches", two_calls), (f"T{T}_us", one_launch)):
            call()
            exe.sync()
            exe.capture_begin()
            for _ in range(reps):
                call()
            g = exe.capture_end()
            exe.graph_launch(g)
            exe.sync()
            exe.timer_start()
            exe.graph_launch(g)
            ms = exe.timer_stop()
            exe.graph_destroy(g)
            out[name] = round(1000.0 * ms / reps, 2)
        exe.device_status()
    del t
    return out


def gpu_decoder(torch, oh, D, exe, n_layers, max_len, seed):
    """A Qwen3-30B-A3B-shaped decoder (48 layers, vocab 151,936) with seeded random
    weights generated on the GPU: centred 4-bit attention and expert matrices
    (uncentred experts all push the residual stream one way until the SwiGLU
    intermediates leave the f16 range within a few tokens), norm weights
    around 1, an 8-bit router, a 4-bit embedding and lm_head; KV caches filled
    with random bf16 (the positions before the timed ones stand for an earlier
    context)."""
    c = D.DecoderConfig(n_layers=n_layers, max_len=max_len)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)

    def quant(rows, cols, std=0.02):
        w = torch.randint(-2**31, 2**31, (rows, cols // 8), dtype=torch.int32, device="cuda", generator=gen)
        sf = (torch.randn((rows, cols // G), device="cuda", generator=gen) * std).abs()
        s = sf.to(torch.bfloat16)
        sf = s.float()
        b = (-7.5 * sf + torch.randn(sf.shape, device="cuda", generator=gen) * sf / 8).to(torch.bfloat16)
        return w, s, b

    def norm(n):
        return (1.0 + 0.1 * torch.randn(n, device="cuda", generator=gen)).to(torch.bfloat16)

    def moe_table():
        t = {}
        for p, (r, cols), std in (("gate", (I, H), 0.02), ("up", (I, H), 0.02), ("down", (H, I), 0.01)):
            w, sc, b = quant(E * r, cols, std)
            t[p + "_w"], t[p + "_s"], t[p + "_b"] = (w.view(E, r, cols // 8), sc.view(E, r, cols // G),
                                                     b.view(E, r, cols // G))
        t["router_w"] = torch.randint(-2**31, 2**31, (E, H // 4), dtype=torch.int32, device="cuda", generator=gen)
        t["router_s"] = (torch.randn((E, H // G), device="cuda", generator=gen) * 0.02).abs().to(torch.bfloat16)
        t["router_b"] = (torch.randn((E, H // G), device="cuda", generator=gen) * 0.01).to(torch.bfloat16)
        return t

    moe = [moe_table() for _ in range(n_layers)]
    keep, layers, caches = [], [], []
    qd, kvd = c.n_heads * c.head_dim, c.n_kv * c.head_dim
    for il in range(n_layers):
        t = {}
        # q, k, v back to back: one matrix for the prefill GEMM, three parts for the decode mat-vec
        qkv = quant(qd + 2 * kvd, c.hidden)
        for name, r0, r1 in (("q", 0, qd), ("k", qd, qd + kvd), ("v", qd + kvd, qd + 2 * kvd)):
            t[name + "_w"], t[name + "_s"], t[name + "_b"] = (a[r0:r1] for a in qkv)
        t["o_w"], t["o_s"], t["o_b"] = quant(c.hidden, qd)
        t["in_norm"], t["post_norm"] = norm(c.hidden), norm(c.hidden)
        t["q_norm"], t["k_norm"] = norm(c.head_dim), norm(c.head_dim)
        ptrs = {k: v.data_ptr() for k, v in t.items()}
        mp = {k: v.data_ptr() for k, v in moe[il].items()}
        mp["norm_w"] = ptrs["post_norm"]
        ptrs["moe"] = oh.MoeLayer(mp)
        layers.append(ptrs)
        kc = torch.randn((c.n_kv, max_len, c.head_dim), device="cuda", generator=gen).to(torch.bfloat16)
        vc = torch.randn((c.n_kv, c.head_dim, max_len), device="cuda", generator=gen).to(torch.bfloat16)
        caches.append((kc.data_ptr(), vc.data_ptr()))
        keep += [t, kc, vc]
    g = {}
    g["embed_w"], g["embed_s"], g["embed_b"] = quant(c.vocab, c.hidden, 0.05)
    g["lm_w"], g["lm_s"], g["lm_b"] = quant(c.vocab, c.hidden)
    g["final_norm"] = norm(c.hidden)
    keep += [g, moe]
    torch.cuda.synchronize()
    model = D.Model(exe, c, layers, {k: v.data_ptr() for k, v in g.items()}, caches=caches)
    return model, keep


def decoder_token_bytes(c, seq):
    """HBM bytes one decode step reads at attended length seq: attention
    weights and MoE bytes per layer, the lm_head, the KV cache and the
    embedding row (the per-token analogue of the MoE layer figure)."""
    qd, kvd = c.n_heads * c.head_dim, c.n_kv * c.head_dim
    def q4(rows, cols):
        return rows * cols // 2 + 2 * 2 * rows * (cols // G)
    attn = q4(qd + 2 * kvd, c.hidden) + q4(c.hidden, qd)
    kv = 2 * kvd * 2 * seq
    return c.n_layers * (attn + LAYER_BYTES + kv) + q4(c.vocab, c.hidden) + q4(1, c.hidden)


def bench_decoder(torch, oh, exe, args):
    """Greedy decode steps of the 48-layer decoder around
    context 4096, one captured graph per step, replayed back to back."""
    from obsidian_hip import decoder as D
    ctx = 4096
    n_pos = args.dec_warmup + args.dec_steps
    max_len = (ctx + n_pos + 31) // 32 * 32
    model, keep = gpu_decoder(torch, oh, D, exe, args.layers, max_len, 4321)
    start = ctx - n_pos // 2
    model.set_state(start, 1)
    model.capture()  # one eager step, then the capture
    model.set_state(start, 1)
    model.replay(args.dec_warmup)
    exe.sync()
    pos0, _ = model.read_state()
    exe.timer_start()
    model.replay(args.dec_steps)
    ms = exe.timer_stop()
    pos1, tok = model.read_state()  # checks the device status of the timed steps
    if pos1 - pos0 != args.dec_steps:
        raise RuntimeError(f"decoder: {pos1 - pos0} positions advanced in {args.dec_steps} steps")
    import numpy as np
    lg = model.logits.download()
    if not bool(np.all(np.isfinite(lg))) or not 0 <= tok < model.cfg.vocab:
        raise RuntimeError("decoder: the last timed step produced non-finite logits or an invalid token")
    ms_tok = ms / args.dec_steps
    seq_mid = (pos0 + pos1) / 2.0 + 1.0  # mean attended length of the timed steps
    nbytes = decoder_token_bytes(model.cfg, seq_mid)
    # kernel breakdown of one eager step (event pairs; the hold kernel lets the host queue it)
    exe.profile_clear()
    model.set_state(start, 1)
    exe.stream_hold(30000)
    exe.profile_enable(True)
    model.step()
    exe.profile_enable(False)
    exe.profile_accumulate()
    exe.device_status()
    stats = exe.profile_stats()
    exe.profile_clear()
    kern = {n: round(1000.0 * t, 1) for n, (t, c) in sorted(stats.items(), key=lambda kv: -kv[1][0])}
    out = {"tokens_per_s": 1000.0 / ms_tok, "ms_per_token": ms_tok, "positions": [pos0, pos1 - 1],
           "bytes_per_token": int(nbytes), "gbs": nbytes / (ms_tok * 1e-3) / 1e9, "last_token": tok,
           "step_kernels_us": kern}
    if args.pf_tokens:
        out["prefill"] = bench_decoder_prefill(exe, model, args)
    model.close()
    del keep
    torch.cuda.empty_cache()
    return out


def prefill_flops(c, T, pos0=0):
    """Matrix flops of a T-token prefill of the whole decoder at positions
    pos0..: the q/k/v/o projections, the router, the 8 experts' gate/up/down
    per token, causal attention (QK and PV over each token's positions) and
    the last token's lm_head."""
    qd, kvd = c.n_heads * c.head_dim, c.n_kv * c.head_dim
    proj = 2 * T * c.hidden * (qd + 2 * kvd) + 2 * T * qd * c.hidden
    moe = 2 * T * c.n_exp * c.hidden + 2 * T * c.top_k * 3 * c.hidden * c.inter
    attn = 2 * 2 * c.n_heads * c.head_dim * sum(pos0 + t + 1 for t in range(T))
    return c.n_layers * (proj + moe + attn) + 2 * c.vocab * c.hidden


def bench_decoder_prefill(exe, model, args):
    """Model.prefill of a T-token prompt at position 0 through every layer
    (prefill_batched, forward.rs:114-261): one untimed, then timed repetitions
    between HIP events; then a per-kernel breakdown of one more from event
    pairs."""
    import numpy as np
    T, reps = args.pf_tokens, args.pf_reps
    rng = np.random.default_rng(77)
    toks = rng.integers(0, model.cfg.vocab, T).astype(np.int32)
    model.prefill(toks, 0)
    exe.sync()
    exe.timer_start()
    for _ in range(reps):
        model.prefill(toks, 0)  # each reads its next token back (read_state checks the device status)
    ms = exe.timer_stop() / reps
    exe.profile_clear()
    exe.profile_enable(True)
    model.prefill(toks, 0)
    exe.profile_enable(False)
    exe.profile_accumulate()
    stats = exe.profile_stats()
    exe.profile_clear()
    flops = prefill_flops(model.cfg, T)
    kern = {n: round(1000.0 * t, 1) for n, (t, c) in sorted(stats.items(), key=lambda kv: -kv[1][0])}
    return {"T": T, "ms": ms, "tokens_per_s": T / (ms * 1e-3), "tflops": flops / (ms * 1e-3) / 1e12,
            "flops": flops, "kernels_us": kern}


def measured_traffic(kernel):
    """(HBM bytes per launch of `kernel`, provenance) from the committed counter
    summary (rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes, each scaled by
    the same counter over a plain device copy of known size). The figure counts
    only while the digest of the kernel's sources it was measured at matches
    the sources now (obsidian_hip.profiles.source_digest); otherwise None."""
    from obsidian_hip import profiles
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(kernel)
    except (OSError, ValueError):
        return None, "not measured"
    if rec is None:
        return None, "not measured"
    now = profiles.source_digest(kernel)
    if rec.get("source_sha") != now:
        return None, f"stale: measured at sources {rec.get('source_sha')}, sources now {now}"
    return rec.get("traffic_bytes_per_launch"), f"profiles/hbm_traffic.json (sources {now})"


def calibrate_copy(torch, mib):
    """A plain device-to-device copy of `mib` MiB, three times: the known-size
    kernel that scales the FETCH_SIZE / WRITE_SIZE counters to bytes."""
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").random_(0, 256)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    ok = bool(torch.equal(dst[:4096], src[:4096]))
    print(json.dumps({"calibration": "device copy", "bytes_read": n, "bytes_written": n, "copies": 3, "ok": ok}))


def bench_prefill(torch, oh, exe, args):
    import numpy as np
    from obsidian_hip import synth

    t = gpu_table(torch, 1, 4321)[0]
    layer = oh.MoeLayer({k: v.data_ptr() for k, v in t.items()})
    cfg = oh.MoeConfig(E, K, H, I, G, True)
    ids, w = synth.zipf_routing(PREFILL_T, E, K, 1.1, seed=0)
    d_ids = torch.from_numpy(ids).cuda()
    d_w = torch.from_numpy(w).cuda()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    X = torch.randn((PREFILL_T, H), device="cuda", generator=gen).to(torch.bfloat16)
    Y = torch.empty_like(X)
    ws_bytes = exe.moe_prefill_workspace(cfg, PREFILL_T)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()

    def run():
        exe.moe_prefill(cfg, layer, X.data_ptr(), Y.data_ptr(), PREFILL_T, ids=d_ids.data_ptr(),
                        weights=d_w.data_ptr(), ws=ws.data_ptr(), ws_bytes=ws_bytes)

    try:
        run()
    except oh.ObsError as e:
        if e.code == oh.OBS_E_UNSUPPORTED:
            return None
        raise
    exe.sync()
    for _ in range(args.warmup):
        run()
    exe.sync()
    reps = max(args.steps, 5)
    exe.timer_start()
    for _ in range(reps):
        run()
    ms = exe.timer_stop() / reps
    exe.device_status()
    exe.profile_clear()
    for _ in range(3):
        exe.stream_hold(20000)
        exe.profile_enable(True)
        run()
        exe.profile_enable(False)
        exe.profile_accumulate()
    stats = exe.profile_stats()
    exe.profile_clear()
    kernels = {n: {"avg_us": 1000.0 * tt / c, "launches": c} for n, (tt, c) in stats.items()}
    # both GEMMs: one moe_ffn launch, or grouped_gemm_gateup + grouped_gemm_down
    gemm_us = sum(v["avg_us"] for n, v in kernels.items() if n.startswith("grouped_gemm") or n == "moe_ffn")
    ys = Y.float().cpu()
    if not bool(torch.isfinite(ys).all()):
        raise RuntimeError("prefill produced non-finite outputs")
    out = {"T": PREFILL_T, "ms": ms, "tflops": PREFILL_FLOP / (ms * 1e-3) / 1e12,
           "gemm_us": gemm_us, "gemm_tflops": PREFILL_FLOP / (gemm_us * 1e-6) / 1e12 if gemm_us else None,
           "kernels": kernels}
    del t, X, Y, ws
    torch.cuda.empty_cache()
    return out


def bench_peaks(torch, exe, read_bytes=2 << 30, mfma_iters=50000, reps=5):
    """The achievable peaks on this device (obs_measure_read / obs_measure_mfma):
    a cold read of read_bytes (8x the 256 MB Infinity Cache) with the fused
    decode's 16-byte non-temporal loads, and bf16 MFMAs with nothing else to do,
    with the core clock they ran at. Best of `reps` launches each."""
    buf = torch.empty(read_bytes, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    clocks = torch.zeros(2, dtype=torch.int64, device="cuda")
    torch.cuda.synchronize()
    exe.measure_read(buf.data_ptr(), read_bytes, sink.data_ptr())
    best = None
    for _ in range(reps):
        exe.timer_start()
        exe.measure_read(buf.data_ptr(), read_bytes, sink.data_ptr())
        ms = exe.timer_stop()
        best = ms if best is None else min(best, ms)
    read_gbs = read_bytes / (best * 1e-3) / 1e9
    flops = exe.measure_mfma(mfma_iters // 10, sink.data_ptr(), clocks.data_ptr())
    best, clk = None, None
    for _ in range(reps):
        exe.timer_start()
        flops = exe.measure_mfma(mfma_iters, sink.data_ptr(), clocks.data_ptr())
        ms = exe.timer_stop()
        cyc, ticks = (int(v) for v in clocks.cpu())
        if best is None or ms < best:
            best, clk = ms, cyc / (ticks / 1e8) / 1e9
    del buf
    torch.cuda.empty_cache()
    tf = flops / (best * 1e-3) / 1e12
    return {"hbm_read_gbs": round(read_gbs, 1), "hbm_read_bytes": read_bytes,
            "hbm_read_frac_of_peak": round(read_gbs / HBM_PEAK_GBS, 4),
            "mfma_bf16_tflops": round(tf, 1), "mfma_clock_ghz": round(clk, 3),
            "mfma_frac_of_peak": round(tf / BF16_PEAK_TFLOPS, 4),
            "method": ("obs_measure_read: 2 GiB read once with 16-byte non-temporal loads, 8 workgroups per CU; "
                       "obs_measure_mfma: v_mfma_f32_32x32x16_bf16 only, 4 chains per wave, 8 waves per CU; "
                       "best of 5 launches each, HIP events on the context's stream")}


def _median_us(fn, reps):
    """Median wall time of `reps` calls of fn, in microseconds (one untimed call first)."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return 1e6 * ts[len(ts) // 2]


def cpu_baseline(n_threads, pf_sample=256):
    """The reference's CPU path on this host, per benched workload: the
    oracle's C rendering of the Metal shaders' semantics (serial fp32 dot per
    output row, OpenMP over rows; kind "port") and the NumPy replica of
    validate_dequant.py:24-30 with numpy's BLAS for the products. Medians of 20
    repetitions (3 for the prefill, on a sample of its tokens)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import oracle as O
    from obsidian_hip import synth

    O.set_threads(n_threads)
    t = synth.moe_layer(77, E, H, I, G)
    L = O.Layer(t, E, H, I, G)
    rng = np.random.default_rng(5)
    xs = synth.bf16_normal(rng, (64, H))
    W, S, B = t["down_w"][0], t["down_s"][0], t["down_b"][0]
    xd = synth.bf16_bits_to_f32(synth.bf16_normal(rng, I))
    Sf, Bf = synth.bf16_bits_to_f32(S), synth.bf16_bits_to_f32(B)
    X512 = synth.bf16_normal(rng, (512, H))
    ids, w = synth.zipf_routing(PREFILL_T, E, K, 1.1, seed=0)
    Xp = synth.bf16_normal(rng, (PREFILL_T, H))
    n = min(pf_sample, PREFILL_T)
    it = iter(range(10 ** 9))
    # the C rendering first, then the NumPy replica (so neither's idle threads spin during the other)
    c = {"0": _median_us(lambda: O.qmatvec("shader", 4, W, S, B, xd, I, H), 20),
         "1a": _median_us(lambda: O.router_baseline(L, xs[:1], K, True, n_threads), 20),
         "1b": _median_us(lambda: O.router_baseline(L, X512, K, True, n_threads), 20),
         "2": _median_us(lambda: O.moe_decode_baseline(L, xs[next(it) % 64], K, True, n_threads), 20),
         "3": _median_us(lambda: O.moe_prefill_baseline(L, Xp[:n], ids[:n], w[:n], n_threads), 3)}
    npy = {"0": _median_us(lambda: O.dequant_numpy(W, Sf, Bf) @ xd, 20),
           "1a": _median_us(lambda: O.router_numpy(t, xs[:1], K, True), 20),
           "1b": _median_us(lambda: O.router_numpy(t, X512, K, True), 20),
           "2": _median_us(lambda: O.decode_layer_numpy(t, xs[next(it) % 64], K), 20),
           "3": _median_us(lambda: O.prefill_numpy(t, Xp[:n], ids[:n], w[:n]), 3)}
    out = {"0_down_proj_matvec": {"c_us": round(c["0"], 1), "numpy_us": round(npy["0"], 1)},
           "1_router": {"T1": {"c_us": round(c["1a"], 1), "numpy_us": round(npy["1a"], 1)},
                        "T512": {"c_us": round(c["1b"], 1), "numpy_us": round(npy["1b"], 1)}},
           "2_decode_layer": {"c_us": round(c["2"], 1), "numpy_us": round(npy["2"], 1)},
           "3_prefill": {"sample_tokens": n, "c_ms_sample": round(c["3"] / 1000, 1),
                         "numpy_ms_sample": round(npy["3"] / 1000, 1),
                         "c_ms_T2048_est": round(c["3"] / 1000 * PREFILL_T / n, 1)}}
    c2 = c["2"]
    try:
        from threadpoolctl import threadpool_info
        blas = sorted({d.get("num_threads") for d in threadpool_info() if d.get("user_api") == "blas"})
    except Exception:  # threadpoolctl missing: report unknown
        blas = []
    return {"value": round(LAYER_BYTES / (c2 * 1e-6) / 1e9, 3), "unit": "GB/s", "us_per_layer": round(c2, 1),
            "cores": n_threads, "kind": "port",
            "sample": ("median of 20 decode MoE layers (T=1, top-8 of 128, one resident layer, rotating inputs), "
                       "C rendering of the shader semantics, OpenMP over rows"),
            "host_cpus": len(os.sched_getaffinity(0)), "numpy_blas_threads": blas, "configs": out}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--input-sets", type=int, default=4)
    ap.add_argument("--prof-reps", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-decoder", action="store_true")
    ap.add_argument("--dec-steps", type=int, default=32)
    ap.add_argument("--dec-warmup", type=int, default=4)
    ap.add_argument("--pf-tokens", type=int, default=2048, help="decoder prefill prompt length (0: skip)")
    ap.add_argument("--pf-reps", type=int, default=3)
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain MIB-MiB device copy (counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding is a design note, not a measured path.", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.calibrate_copy:
        calibrate_copy(torch, args.calibrate_copy)
        return
    import obsidian_hip as oh

    exe = oh.ObsidianExecutor(0)
    dec = bench_decode(torch, oh, exe, args)
    rtr = bench_router(torch, oh, exe)
    pre = None if args.no_prefill else bench_prefill(torch, oh, exe, args)
    dcd = None if args.no_decoder else bench_decoder(torch, oh, exe, args)
    peaks = bench_peaks(torch, exe)
    if dec["roofline"] is not None:
        dec["roofline"]["achievable_peak"] = peaks["hbm_read_gbs"]
        dec["roofline"]["frac_of_achievable"] = round(dec["roofline"]["achieved"] / peaks["hbm_read_gbs"], 4)
    cpu = None
    if not args.no_cpu:
        # every core this process may run on, capped by OMP_NUM_THREADS where it is set (the
        # host's CPU share per GPU)
        threads = len(os.sched_getaffinity(0))
        if os.environ.get("OMP_NUM_THREADS", "").isdigit() and int(os.environ["OMP_NUM_THREADS"]) > 0:
            threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
        cpu = cpu_baseline(threads)
    exe.close()

    line = {
        "metric": METRIC,
        "value": round(dec["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "dtype_detail": ("decode: 4-bit MLX-affine weights against f16 activation operands (v_dot2_f32_f16), "
                         "fp32 accumulation; prefill: bf16 MFMA operands, fp32 accumulation"),
        "data": "synthetic (seeded random 4-bit weights, bf16 scales/biases, bf16 activations)",
        "device_status": "ok",  # obs_device_status after every timed region (a failure raises before this line)
        "config": {"workload": "decode MoE layer T=1, top-8 of 128 experts, 48-layer HBM-resident table",
                   "experts": E, "top_k": K, "hidden": H, "moe_inter": I, "group": G,
                   "layers_per_step": args.layers, "parallelism": "none (1 GPU)"},
        "decode_us_per_layer": round(dec["us_layer"], 3),
        "decode_frac_of_hbm_peak": round(dec["gbs"] / HBM_PEAK_GBS, 4),
        "decode_kernels": {n: round(v["avg_us"], 3) for n, v in dec["kernels"].items()},
        "roofline": dec["roofline"],
        "router": dict(rtr, workload="8-bit gate [128 x 2048] + softmax/top-8 (f16 logits): one launch per call "
                                      "(T*_us) and the two-launch form (T*_us_two_launches), graph of 200 calls"),
        "prefill": None if pre is None else {
            "T": pre["T"], "ms": round(pre["ms"], 4), "tflops": round(pre["tflops"], 1),
            "gemm_us": round(pre["gemm_us"], 2),
            "gemm_tflops": None if pre["gemm_tflops"] is None else round(pre["gemm_tflops"], 1),
            "frac_of_bf16_peak": None if pre["gemm_tflops"] is None else round(pre["gemm_tflops"] / BF16_PEAK_TFLOPS, 4),
            "frac_of_achievable_mfma": None if pre["gemm_tflops"] is None else
            round(pre["gemm_tflops"] / peaks["mfma_bf16_tflops"], 4),
            "kernels": {n: round(v["avg_us"], 2) for n, v in pre["kernels"].items()}},
        "achievable": peaks,
        "decoder": None if dcd is None else {
            "workload": f"greedy decode, {args.layers}-layer Qwen3-30B-A3B shape, bf16 KV cache, "
                        f"positions {dcd['positions'][0]}-{dcd['positions'][1]} (context ~4096)",
            "tokens_per_s": round(dcd["tokens_per_s"], 1), "ms_per_token": round(dcd["ms_per_token"], 4),
            "bytes_per_token": dcd["bytes_per_token"], "gbs": round(dcd["gbs"], 1),
            "frac_of_hbm_peak": round(dcd["gbs"] / HBM_PEAK_GBS, 4),
            "step_kernels_us": dcd["step_kernels_us"],
            "prefill": None if dcd.get("prefill") is None else {
                "workload": f"prefill of a {dcd['prefill']['T']}-token prompt at position 0 through "
                            f"{args.layers} layers, last-token lm_head + greedy pick",
                "tokens_per_s": round(dcd["prefill"]["tokens_per_s"], 1), "ms": round(dcd["prefill"]["ms"], 3),
                "tflops": round(dcd["prefill"]["tflops"], 1),
                "frac_of_bf16_peak": round(dcd["prefill"]["tflops"] / BF16_PEAK_TFLOPS, 4),
                "kernels_us": dcd["prefill"]["kernels_us"]}},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
