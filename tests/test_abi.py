"""The C ABI boundary without a GPU: the built library loads, exports every
function include/obsidian_hip.h declares (and the Python host binds exactly
that set), rejects a null context before touching the device, and sizes the
prefill workspace on the host alone.

The reference's boundary is ObsidianExecutor plus the per-kernel dispatch
helpers (src/executor.rs:39-70, src/forward.rs:289-321, src/router.rs:25-94);
the header cites the item each export replaces.
"""
import ctypes as C
import os
import re
import subprocess

import pytest

import obsidian_hip as oh

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "obsidian_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b(obs_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("obs_create", "obs_destroy", "obs_last_error", "obs_q4_matvec", "obs_q4_matmul",
                 "obs_q8_gate_logits", "obs_route_topk", "obs_moe_decode", "obs_moe_prefill",
                 "obs_moe_prefill_workspace"):
        assert must in names
    assert len(names) >= 30


def test_library_exports_every_declared_symbol():
    L = C.CDLL(oh.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing


def test_dynamic_symbol_table_matches_header():
    out = subprocess.run(["nm", "-D", "--defined-only", oh.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.split() and ln.split()[-1].startswith("obs_")}
    assert exported == set(declared_functions())


def test_python_binding_covers_exactly_the_header():
    assert set(oh.EXPORTS) == set(declared_functions())
    oh.lib()  # every signature binds


def test_rust_binding_in_integration_covers_exactly_the_header():
    """INTEGRATION.md's `extern "C"` block declares every export once, and
    nothing the header does not."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = text.split("```rust", 1)[1].split("```", 1)[0]
    fns = re.findall(r"\bpub fn (obs_\w+)\s*\(", block)
    assert len(fns) == len(set(fns)), sorted(n for n in set(fns) if fns.count(n) > 1)
    assert set(fns) == set(declared_functions())


def test_null_context_is_rejected_before_any_device_work():
    L = oh.lib()
    host_only = {"obs_create", "obs_create_error", "obs_destroy", "obs_last_error", "obs_get_stream",
                 "obs_graph_destroy", "obs_moe_prefill_workspace", "obs_profile_count",
                 "obs_ckpt_close", "obs_ckpt_error", "obs_moe_layer_bytes", "obs_sdpa_workspace",
                 "obs_argmax_workspace", "obs_dispatch_gate"}
    for name in declared_functions():
        if name in host_only:
            continue
        fn = getattr(L, name)
        args = [None if a in (C.c_void_p, C.c_char_p) or (isinstance(a, type) and issubclass(a, C._Pointer)) else 0
                for a in fn.argtypes]
        assert fn(*args) == oh.OBS_E_INVALID, name
    assert L.obs_last_error(None) == b"null context"
    assert L.obs_get_stream(None) is None
    assert L.obs_profile_count(None) == 0
    L.obs_destroy(None)
    L.obs_graph_destroy(None)
    assert L.obs_create(0, None) == oh.OBS_E_INVALID
    # checkpoint handles: the null checks above ran obs_ckpt_open(NULL, ...), whose
    # message is kept per thread; closing NULL is a no-op
    assert L.obs_ckpt_error(None) == b"obs_ckpt_open: null argument"
    L.obs_ckpt_close(None)
    assert L.obs_moe_layer_bytes(None) == 0
    assert L.obs_argmax_workspace() == 256 * 8
    assert L.obs_sdpa_workspace(32, 4, 128, 4096) == 4 * 64 * 16 * 130 * 4  # fp32 (m, l, O) per split and head slot
    assert L.obs_sdpa_workspace(32, 4, 64, 4096) == 0 and L.obs_sdpa_workspace(32, 3, 128, 4096) == 0


def test_prefill_workspace_is_host_arithmetic():
    L = oh.lib()
    cfg = oh.MoeConfig(128, 8, 2048, 768, 64, True).to_c()
    assert L.obs_moe_prefill_workspace(None, 16) == 0
    assert L.obs_moe_prefill_workspace(C.byref(cfg), 0) == 0
    sizes = [L.obs_moe_prefill_workspace(C.byref(cfg), T) for T in (1, 2, 64, 2048)]
    assert sizes == sorted(sizes) and len(set(sizes)) == 4
    for T, ws in zip((1, 2, 64, 2048), sizes):
        rows = T * 8
        # at least the two bf16 intermediates: H [T*k, I] and the expert outputs [T*k, H]
        assert ws >= rows * 768 * 2 + rows * 2048 * 2
        assert ws % 256 == 0


def test_create_without_a_gpu_reports_unsupported():
    import torch
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is present; covered by the GPU tests")
    L = oh.lib()
    ctx = C.c_void_p()
    assert L.obs_create(0, C.byref(ctx)) == oh.OBS_E_UNSUPPORTED
    assert ctx.value is None
    assert b"no HIP device" in L.obs_create_error()
    with pytest.raises(oh.ObsError) as ei:
        oh.ObsidianExecutor(0)
    assert ei.value.code == oh.OBS_E_UNSUPPORTED


def test_dispatch_gate_rule():
    """The one-launch paths a device may take, from its CU count and the two
    dispatch facts obs_create probes (pure host rule, no device)."""
    L = oh.lib()
    D, A, F = oh.OBS_PATH_FUSED_DECODE, oh.OBS_PATH_FUSED_ATTN, oh.OBS_PATH_FFN_ONE_LAUNCH
    assert L.obs_dispatch_gate(256, 1, 1) == D | A | F
    assert L.obs_dispatch_gate(304, 1, 1) == D | A | F
    # the fused decode / attention need 256 CUs (one workgroup each) and the XCD map
    assert L.obs_dispatch_gate(255, 1, 1) == F
    assert L.obs_dispatch_gate(32, 1, 1) == F
    assert L.obs_dispatch_gate(256, 0, 1) == 0
    assert L.obs_dispatch_gate(256, 1, 0) == D | A
    assert L.obs_dispatch_gate(0, 0, 0) == 0
    assert L.obs_dispatch_gate(100, 1, 0) == 0
