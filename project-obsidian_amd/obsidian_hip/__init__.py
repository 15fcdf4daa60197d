"""obsidian_hip — Python host over the libobsidian_hip C ABI (include/obsidian_hip.h).

The names mirror the reference host so code reads like the Rust engine:

* ``ObsidianExecutor``  — src/executor.rs:39-70 (device + queue; here a HIP
  context and stream).
* ``MoeRouter``         — src/router.rs:16-94 (``route``, ``route_dispatch``,
  ``read_route``).
* ``Model``-style ops   — src/forward.rs: ``dequant`` (:303), ``matmul_raw``
  (:313), ``swiglu`` (:370), ``scaled_add`` (:376), ``gate_gpu`` (:386), and the
  MoE halves of ``forward_layer`` (:421-441) / ``prefill_batched`` (:164-247).

Every call goes through the native library; there is no CPU fallback. If the
library is missing or no gfx950 device is present, the call raises.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libobsidian_hip.so")

OBS_OK = 0
OBS_E_INVALID = -1
OBS_E_SHAPE = -2
OBS_E_ALIGN = -3
OBS_E_HIP = -4
OBS_E_NOMEM = -5
OBS_E_UNSUPPORTED = -6

OBS_DECODE_AUTO, OBS_DECODE_MULTI, OBS_DECODE_FUSED = 0, 1, 2
OBS_PATH_FUSED_DECODE, OBS_PATH_FUSED_ATTN, OBS_PATH_FFN_ONE_LAUNCH = 1, 2, 4  # obs_dispatch_gate bits
# routing rules (obs_route_topk, MoeConfig.route_rule)
ROUTE_REF, ROUTE_F32 = 0, 1

_ERRNAMES = {
    OBS_E_INVALID: "OBS_E_INVALID",
    OBS_E_SHAPE: "OBS_E_SHAPE",
    OBS_E_ALIGN: "OBS_E_ALIGN",
    OBS_E_HIP: "OBS_E_HIP",
    OBS_E_NOMEM: "OBS_E_NOMEM",
    OBS_E_UNSUPPORTED: "OBS_E_UNSUPPORTED",
}

# Every symbol the C ABI exports (include/obsidian_hip.h).
EXPORTS = (
    "obs_create", "obs_destroy", "obs_last_error", "obs_create_error", "obs_set_stream",
    "obs_get_stream", "obs_alloc", "obs_free", "obs_upload", "obs_download", "obs_memset",
    "obs_sync", "obs_timer_start", "obs_timer_stop", "obs_dequant", "obs_q4_matvec",
    "obs_q4_matmul", "obs_q8_gate_logits", "obs_route_topk", "obs_route", "obs_swiglu", "obs_scaled_add", "obs_rmsnorm",
    "obs_moe_decode", "obs_moe_decode_static", "obs_moe_prefill_workspace", "obs_moe_prefill", "obs_capture_begin",
    "obs_capture_end", "obs_graph_launch", "obs_graph_destroy", "obs_set_decode_path",
    "obs_device_status", "obs_stream_hold", "obs_profile_enable",
    "obs_profile_accumulate", "obs_profile_count", "obs_profile_stat", "obs_profile_clear",
    "obs_ckpt_open", "obs_ckpt_close", "obs_ckpt_error", "obs_ckpt_config", "obs_ckpt_tensor_info",
    "obs_ckpt_read", "obs_moe_layer_bytes", "obs_ckpt_load_moe_layer", "obs_ckpt_load_tensor",
    "obs_q4_gemv", "obs_attn_prep", "obs_sdpa_workspace", "obs_sdpa_decode", "obs_embed_q4",
    "obs_argmax_workspace", "obs_argmax", "obs_embed_q4_rows", "obs_attn_prep_rows", "obs_sdpa_prefill",
    "obs_attn_decode", "obs_layer_decode", "obs_dispatch_gate", "obs_dispatch_info", "obs_set_dispatch_facts", "obs_debug_ffn_wait",
    "obs_measure_read", "obs_measure_mfma",
)


class ObsError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{_ERRNAMES.get(code, code)}: {msg}")
        self.code = code


class ObsMoeConfig(C.Structure):
    _fields_ = [("n_exp", C.c_uint32), ("top_k", C.c_uint32), ("hidden", C.c_uint32),
                ("inter", C.c_uint32), ("group", C.c_uint32), ("norm_topk", C.c_int32),
                ("rms_eps", C.c_float), ("route_rule", C.c_int32)]


class ObsMoeLayer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b",
        "router_w", "router_s", "router_b", "norm_w")]


class ObsGemvPart(C.Structure):
    _fields_ = [("w", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p), ("y_f32", C.c_void_p),
                ("y_bf16", C.c_void_p), ("residual", C.c_void_p), ("rows", C.c_uint32)]


class ObsAttnLayer(C.Structure):
    KEYS = ("q_w", "q_s", "q_b", "k_w", "k_s", "k_b", "v_w", "v_s", "v_b", "o_w", "o_s", "o_b",
            "in_norm", "q_norm", "k_norm")
    _fields_ = [(k, C.c_void_p) for k in KEYS]


class ObsTensorInfo(C.Structure):
    _fields_ = [("dtype", C.c_int32), ("ndim", C.c_uint32), ("shape", C.c_uint64 * 8), ("nbytes", C.c_uint64),
                ("n_pieces", C.c_uint32)]


# OBS_DT_* codes -> (safetensors name, numpy dtype of the raw bytes; bf16 and fp8 as bit patterns)
DTYPES = {
    0: ("BOOL", np.bool_), 1: ("U8", np.uint8), 2: ("I8", np.int8), 3: ("F8_E5M2", np.uint8),
    4: ("F8_E4M3", np.uint8), 5: ("I16", np.int16), 6: ("U16", np.uint16), 7: ("F16", np.float16),
    8: ("BF16", np.uint16), 9: ("I32", np.int32), 10: ("U32", np.uint32), 11: ("F32", np.float32),
    12: ("F64", np.float64), 13: ("I64", np.int64), 14: ("U64", np.uint64),
}

_DT_CODE = {v[0]: k for k, v in DTYPES.items()}

_lib_handle = None


def lib() -> C.CDLL:
    """Load libobsidian_hip.so (built in-tree); raise if it is absent."""
    global _lib_handle
    if _lib_handle is not None:
        return _lib_handle
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() (or make in project-obsidian_amd/)")
    L = C.CDLL(LIB_PATH)
    vp, u32, i32, f32, sz = C.c_void_p, C.c_uint32, C.c_int32, C.c_float, C.c_size_t
    sig = {
        "obs_create": (i32, [C.c_int, C.POINTER(vp)]),
        "obs_destroy": (None, [vp]),
        "obs_last_error": (C.c_char_p, [vp]),
        "obs_create_error": (C.c_char_p, []),
        "obs_set_stream": (i32, [vp, vp]),
        "obs_get_stream": (vp, [vp]),
        "obs_alloc": (i32, [vp, sz, C.POINTER(vp)]),
        "obs_free": (i32, [vp, vp]),
        "obs_upload": (i32, [vp, vp, vp, sz]),
        "obs_download": (i32, [vp, vp, vp, sz]),
        "obs_memset": (i32, [vp, vp, C.c_int, sz]),
        "obs_sync": (i32, [vp]),
        "obs_timer_start": (i32, [vp]),
        "obs_timer_stop": (i32, [vp, C.POINTER(f32)]),
        "obs_dequant": (i32, [vp, C.c_int, vp, vp, vp, vp, vp, u32, u32, u32]),
        "obs_q4_matvec": (i32, [vp, vp, vp, vp, vp, vp, vp, u32, u32, u32]),
        "obs_q4_matmul": (i32, [vp, vp, vp, vp, vp, vp, u32, u32, u32, u32]),
        "obs_q8_gate_logits": (i32, [vp, vp, vp, vp, vp, vp, u32, u32, u32, u32]),
        "obs_route_topk": (i32, [vp, vp, vp, vp, u32, u32, u32, C.c_int, C.c_int]),
        "obs_route": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, C.c_int, C.c_int]),
        "obs_swiglu": (i32, [vp, vp, vp, vp, u32]),
        "obs_scaled_add": (i32, [vp, vp, vp, f32, u32]),
        "obs_rmsnorm": (i32, [vp, vp, vp, vp, u32, u32, f32]),
        "obs_moe_decode": (i32, [vp, C.POINTER(ObsMoeConfig), C.POINTER(ObsMoeLayer), vp, vp, vp, vp, vp]),
        "obs_moe_decode_static": (i32, [vp, C.POINTER(ObsMoeConfig), C.POINTER(ObsMoeLayer), vp, vp, vp, vp, vp]),
        "obs_moe_prefill_workspace": (sz, [C.POINTER(ObsMoeConfig), u32]),
        "obs_moe_prefill": (i32, [vp, C.POINTER(ObsMoeConfig), C.POINTER(ObsMoeLayer), vp, vp, vp, u32,
                                  vp, vp, vp, sz]),
        "obs_capture_begin": (i32, [vp]),
        "obs_capture_end": (i32, [vp, C.POINTER(vp)]),
        "obs_graph_launch": (i32, [vp, vp]),
        "obs_graph_destroy": (None, [vp]),
        "obs_set_decode_path": (i32, [vp, C.c_int]),
        "obs_device_status": (i32, [vp]),
        "obs_dispatch_gate": (u32, [C.c_int, C.c_int, C.c_int]),
        "obs_dispatch_info": (i32, [vp, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int)]),
        "obs_set_dispatch_facts": (i32, [vp, C.c_int, C.c_int]),
        "obs_debug_ffn_wait": (i32, [vp, u32, u32]),
        "obs_measure_read": (i32, [vp, vp, sz, vp]),
        "obs_measure_mfma": (i32, [vp, u32, vp, vp, C.POINTER(C.c_double)]),
        "obs_stream_hold": (i32, [vp, u32]),
        "obs_profile_enable": (i32, [vp, C.c_int]),
        "obs_profile_accumulate": (i32, [vp]),
        "obs_profile_count": (C.c_int, [vp]),
        "obs_profile_stat": (i32, [vp, C.c_int, C.POINTER(C.c_char_p), C.POINTER(C.c_double),
                                   C.POINTER(C.c_int64)]),
        "obs_profile_clear": (i32, [vp]),
        "obs_ckpt_open": (i32, [C.c_char_p, C.c_char_p, C.POINTER(vp)]),
        "obs_ckpt_close": (None, [vp]),
        "obs_ckpt_error": (C.c_char_p, [vp]),
        "obs_ckpt_config": (i32, [vp, C.POINTER(ObsMoeConfig), C.POINTER(u32)]),
        "obs_ckpt_tensor_info": (i32, [vp, C.c_char_p, C.POINTER(ObsTensorInfo)]),
        "obs_ckpt_read": (i32, [vp, C.c_char_p, vp, sz]),
        "obs_moe_layer_bytes": (sz, [C.POINTER(ObsMoeConfig)]),
        "obs_ckpt_load_moe_layer": (i32, [vp, vp, u32, C.POINTER(ObsMoeConfig), vp, sz, C.POINTER(ObsMoeLayer)]),
        "obs_ckpt_load_tensor": (i32, [vp, vp, C.c_char_p, vp, sz]),
        "obs_q4_gemv": (i32, [vp, vp, u32, u32, C.POINTER(ObsGemvPart), u32, vp, f32]),
        "obs_attn_prep": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, f32, f32, vp]),
        "obs_sdpa_workspace": (sz, [u32, u32, u32, u32]),
        "obs_sdpa_decode": (i32, [vp, vp, vp, vp, vp, u32, u32, u32, u32, vp, vp, sz]),
        "obs_embed_q4": (i32, [vp, vp, vp, vp, u32, u32, u32, vp, vp]),
        "obs_argmax_workspace": (sz, []),
        "obs_argmax": (i32, [vp, vp, u32, vp, vp, sz]),
        "obs_embed_q4_rows": (i32, [vp, vp, vp, vp, u32, u32, u32, vp, u32, vp]),
        "obs_attn_prep_rows": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, f32, f32, u32, u32, u32,
                                     u32]),
        "obs_sdpa_prefill": (i32, [vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32]),
        "obs_attn_decode": (i32, [vp, C.POINTER(ObsAttnLayer), vp, vp, vp, u32, f32, f32, vp, vp]),
        "obs_layer_decode": (i32, [vp, C.POINTER(ObsAttnLayer), C.POINTER(ObsMoeConfig), C.POINTER(ObsMoeLayer), vp,
                                   vp, vp, u32, f32, f32, vp, vp, vp, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib_handle = L
    return L


def _ptr(x) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    if isinstance(x, int):
        return x
    raise TypeError(f"expected DeviceBuffer / int device pointer, got {type(x)}")


@dataclass
class DeviceBuffer:
    """A device allocation (the reference's Metal `Buffer`, forward.rs:264)."""
    exec: "ObsidianExecutor"
    ptr: int
    nbytes: int
    dtype: np.dtype
    shape: Tuple[int, ...]
    owned: bool = True

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        self.exec._check(lib().obs_download(self.exec.ctx, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def upload(self, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr, dtype=self.dtype)
        if a.nbytes != self.nbytes:
            raise ValueError(f"size mismatch: {a.nbytes} != {self.nbytes}")
        self.exec._check(lib().obs_upload(self.exec.ctx, self.ptr, a.ctypes.data, a.nbytes))

    def free(self) -> None:
        if self.owned and self.ptr:
            lib().obs_free(self.exec.ctx, self.ptr)
            self.ptr = 0


class ObsidianExecutor:
    """HIP context + stream. executor.rs:39-58 `ObsidianExecutor::new`."""

    def __init__(self, device: int = 0):
        L = lib()
        ctx = C.c_void_p()
        rc = L.obs_create(device, C.byref(ctx))
        if rc != OBS_OK:
            raise ObsError(rc, L.obs_create_error().decode())
        self.ctx = ctx.value
        self.decode_path = OBS_DECODE_AUTO  # as obs_set_decode_path last set it
        self._bufs: List[DeviceBuffer] = []

    # -- errors ----------------------------------------------------------
    def _check(self, rc: int) -> None:
        if rc != OBS_OK:
            raise ObsError(rc, lib().obs_last_error(self.ctx).decode())

    def last_error(self) -> str:
        return lib().obs_last_error(self.ctx).decode()

    # -- buffers (device.new_buffer / contents / drain) ------------------
    def alloc(self, shape, dtype) -> DeviceBuffer:
        shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        dtype = np.dtype(dtype)
        nbytes = max(int(np.prod(shape)) * dtype.itemsize, 1)
        p = C.c_void_p()
        self._check(lib().obs_alloc(self.ctx, nbytes, C.byref(p)))
        buf = DeviceBuffer(self, p.value, nbytes, dtype, shape)
        self._bufs.append(buf)
        return buf

    def upload(self, arr: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(arr)
        buf = self.alloc(a.shape, a.dtype)
        if a.nbytes:
            self._check(lib().obs_upload(self.ctx, buf.ptr, a.ctypes.data, a.nbytes))
        return buf

    def zeros(self, shape, dtype) -> DeviceBuffer:
        buf = self.alloc(shape, dtype)
        self._check(lib().obs_memset(self.ctx, buf.ptr, 0, buf.nbytes))
        return buf

    def sync(self) -> None:
        """Model::drain (forward.rs:282-286)."""
        self._check(lib().obs_sync(self.ctx))

    drain = sync

    def timer_start(self) -> None:
        self._check(lib().obs_timer_start(self.ctx))

    def timer_stop(self) -> float:
        ms = C.c_float()
        self._check(lib().obs_timer_stop(self.ctx, C.byref(ms)))
        return ms.value

    def set_stream(self, stream: Optional[int]) -> None:
        self._check(lib().obs_set_stream(self.ctx, stream))

    def set_decode_path(self, path: int) -> None:
        self._check(lib().obs_set_decode_path(self.ctx, int(path)))
        self.decode_path = int(path)

    def device_status(self) -> None:
        """Raise if a one-launch kernel of this context recorded a device-side
        failure (a bounded wait that timed out); the flag is cleared."""
        self._check(lib().obs_device_status(self.ctx))

    def dispatch_info(self) -> Tuple[int, bool, bool]:
        """(CUs, each group b % 8 of workgroups on one XCD, in-order dispatch per XCD) as the
        probe at context creation found them."""
        n, xm, io = C.c_int(), C.c_int(), C.c_int()
        self._check(lib().obs_dispatch_info(self.ctx, C.byref(n), C.byref(xm), C.byref(io)))
        return n.value, bool(xm.value), bool(io.value)

    def set_dispatch_facts(self, xcd_map_ok: bool, inorder_ok: bool) -> None:
        self._check(lib().obs_set_dispatch_facts(self.ctx, int(xcd_map_ok), int(inorder_ok)))

    def paths(self) -> int:
        """The OBS_PATH_* one-launch paths this context's device may take."""
        n, xm, io = self.dispatch_info()
        return int(lib().obs_dispatch_gate(n, int(xm), int(io)))

    def measure_read(self, src, nbytes: int, sink) -> None:
        """Launch the streaming-read peak kernel over nbytes at src (time it with timer_start/stop)."""
        self._check(lib().obs_measure_read(self.ctx, _ptr(src), int(nbytes), _ptr(sink)))

    def measure_mfma(self, iters: int, sink, clocks) -> float:
        """Launch the MFMA-only peak kernel; returns its flop count."""
        f = C.c_double()
        self._check(lib().obs_measure_mfma(self.ctx, int(iters), _ptr(sink), _ptr(clocks), C.byref(f)))
        return f.value

    def debug_ffn_wait(self, extra_count: int, wait_us: int) -> None:
        self._check(lib().obs_debug_ffn_wait(self.ctx, int(extra_count), int(wait_us)))

    # -- graph capture / replay ------------------------------------------
    def capture_begin(self) -> None:
        self._check(lib().obs_capture_begin(self.ctx))

    def capture_end(self) -> int:
        g = C.c_void_p()
        self._check(lib().obs_capture_end(self.ctx, C.byref(g)))
        return g.value

    def graph_launch(self, graph: int) -> None:
        self._check(lib().obs_graph_launch(self.ctx, graph))

    @staticmethod
    def graph_destroy(graph: int) -> None:
        lib().obs_graph_destroy(graph)

    # -- in-stream kernel timing -------------------------------------------
    def stream_hold(self, us: int) -> None:
        self._check(lib().obs_stream_hold(self.ctx, int(us)))

    def profile_enable(self, on: bool) -> None:
        self._check(lib().obs_profile_enable(self.ctx, int(bool(on))))

    def profile_accumulate(self) -> None:
        self._check(lib().obs_profile_accumulate(self.ctx))

    def profile_stats(self) -> Dict[str, Tuple[float, int]]:
        """{kernel name: (total ms, launches)}"""
        L = lib()
        out = {}
        for i in range(L.obs_profile_count(self.ctx)):
            name, ms, n = C.c_char_p(), C.c_double(), C.c_int64()
            self._check(L.obs_profile_stat(self.ctx, i, C.byref(name), C.byref(ms), C.byref(n)))
            out[name.value.decode()] = (ms.value, n.value)
        return out

    def profile_clear(self) -> None:
        self._check(lib().obs_profile_clear(self.ctx))

    def close(self) -> None:
        if getattr(self, "ctx", None):
            for b in self._bufs:
                b.free()
            self._bufs.clear()
            lib().obs_destroy(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # -- kernels ---------------------------------------------------------
    def dequant_tensor(self, bits: int, w, s, b, rows: int, cols: int, group: int = 64,
                       out_f32=None, out_bf16=None) -> None:
        """mx.dequantize (validate_dequant.py:21): fp32 and/or bf16 output."""
        self._check(lib().obs_dequant(self.ctx, bits, _ptr(w), _ptr(s), _ptr(b), _ptr(out_f32),
                                      _ptr(out_bf16), rows, cols, group))

    def q4_matvec(self, w, s, b, x, in_f: int, out_f: int, group: int = 64, y_f32=None, y_bf16=None) -> None:
        self._check(lib().obs_q4_matvec(self.ctx, _ptr(w), _ptr(s), _ptr(b), _ptr(x), _ptr(y_f32),
                                        _ptr(y_bf16), in_f, out_f, group))

    def q4_matmul(self, w, s, b, X, Y, T: int, in_f: int, out_f: int, group: int = 64) -> None:
        self._check(lib().obs_q4_matmul(self.ctx, _ptr(w), _ptr(s), _ptr(b), _ptr(X), _ptr(Y), T, in_f,
                                        out_f, group))

    def q8_gate_logits(self, w, s, b, x, logits, T: int, in_f: int, n_exp: int, group: int = 64) -> None:
        self._check(lib().obs_q8_gate_logits(self.ctx, _ptr(w), _ptr(s), _ptr(b), _ptr(x), _ptr(logits), T,
                                             in_f, n_exp, group))

    def route_topk(self, logits, ids, weights, T: int, n_exp: int, k: int, norm_topk: bool,
                   rule: int = None) -> None:
        """rule: ROUTE_REF (default; the reference's f16 logits and weights) or ROUTE_F32."""
        rule = ROUTE_REF if rule is None else rule
        self._check(lib().obs_route_topk(self.ctx, _ptr(logits), _ptr(ids), _ptr(weights), T, n_exp, k,
                                         int(bool(norm_topk)), int(rule)))

    def route(self, w8, scales, biases, x, logits, ids, weights, T: int, in_dim: int, n_exp: int, k: int,
              norm_topk: bool, group: int = 64, rule: int = None) -> None:
        """q8_gate_logits + route_topk in one launch (obs_route); logits is written as well."""
        rule = ROUTE_REF if rule is None else rule
        self._check(lib().obs_route(self.ctx, _ptr(w8), _ptr(scales), _ptr(biases), _ptr(x), _ptr(logits), _ptr(ids),
                                    _ptr(weights), T, in_dim, n_exp, group, k, int(bool(norm_topk)), int(rule)))

    def swiglu_raw(self, g, u, h, n: int) -> None:
        self._check(lib().obs_swiglu(self.ctx, _ptr(g), _ptr(u), _ptr(h), n))

    def scaled_add_raw(self, acc, y, scale: float, n: int) -> None:
        self._check(lib().obs_scaled_add(self.ctx, _ptr(acc), _ptr(y), float(scale), n))

    def rmsnorm_raw(self, x, w, out, rows: int, dim: int, eps: float) -> None:
        self._check(lib().obs_rmsnorm(self.ctx, _ptr(x), _ptr(w), _ptr(out), rows, dim, float(eps)))

    def moe_decode(self, cfg: "MoeConfig", layer: "MoeLayer", x, y, residual=None, ids_out=None,
                   w_out=None) -> None:
        c, l = cfg.to_c(), layer.to_c()
        self._check(lib().obs_moe_decode(self.ctx, C.byref(c), C.byref(l), _ptr(x), _ptr(residual), _ptr(y),
                                         _ptr(ids_out), _ptr(w_out)))

    def moe_decode_static(self, cfg: "MoeConfig", layer: "MoeLayer", x, y, residual=None, ids_out=None,
                          w_out=None) -> None:
        """moe_decode with no allocation (the device's static scratch); calls
        that overlap in time on one GPU race."""
        c, l = cfg.to_c(), layer.to_c()
        self._check(lib().obs_moe_decode_static(self.ctx, C.byref(c), C.byref(l), _ptr(x), _ptr(residual),
                                                _ptr(y), _ptr(ids_out), _ptr(w_out)))

    # -- the rest of a decode step (forward.rs:398-419, :445-462, :552-567) --
    def q4_gemv(self, x, in_f: int, parts: Sequence[Tuple], group: int = 64, norm_w=None, eps: float = 1e-6) -> None:
        """parts: (w, s, b, rows, y_f32, y_bf16, residual) tuples, 1 to 3; norm_w:
        RMSNorm x first (fused)."""
        arr = (ObsGemvPart * len(parts))()
        for i, (w, s_, b, rows, yf, yb, res) in enumerate(parts):
            arr[i] = ObsGemvPart(_ptr(w), _ptr(s_), _ptr(b), _ptr(yf), _ptr(yb), _ptr(res), rows)
        self._check(lib().obs_q4_gemv(self.ctx, _ptr(x), in_f, group, arr, len(parts), _ptr(norm_w), float(eps)))

    def attn_prep(self, q, k, v, q_norm, k_norm, k_cache, v_cache_t, n_heads: int, n_kv: int, head_dim: int,
                  max_len: int, eps: float, theta: float, state) -> None:
        self._check(lib().obs_attn_prep(self.ctx, _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm),
                                        _ptr(k_cache), _ptr(v_cache_t), n_heads, n_kv, head_dim, max_len, eps,
                                        theta, _ptr(state)))

    @staticmethod
    def sdpa_workspace(n_heads: int, n_kv: int, head_dim: int, max_len: int) -> int:
        return lib().obs_sdpa_workspace(n_heads, n_kv, head_dim, max_len)

    def sdpa_decode(self, q, k_cache, v_cache_t, out, n_heads: int, n_kv: int, head_dim: int, max_len: int, state,
                    ws, ws_bytes: Optional[int] = None) -> None:
        ws_bytes = ws.nbytes if ws_bytes is None else ws_bytes
        self._check(lib().obs_sdpa_decode(self.ctx, _ptr(q), _ptr(k_cache), _ptr(v_cache_t), _ptr(out), n_heads,
                                          n_kv, head_dim, max_len, _ptr(state), _ptr(ws), ws_bytes))

    def embed_q4(self, w, s, b, hidden: int, vocab: int, state, out, group: int = 64) -> None:
        self._check(lib().obs_embed_q4(self.ctx, _ptr(w), _ptr(s), _ptr(b), hidden, group, vocab, _ptr(state),
                                       _ptr(out)))

    def argmax(self, x, n: int, state, ws, ws_bytes: Optional[int] = None) -> None:
        ws_bytes = ws.nbytes if ws_bytes is None else ws_bytes
        self._check(lib().obs_argmax(self.ctx, _ptr(x), n, _ptr(state), _ptr(ws), ws_bytes))

    def attn_decode(self, layer: Dict, x, k_cache, v_cache_t, max_len: int, eps: float, theta: float, state,
                    x1) -> None:
        """The attention half of a decode layer in one launch (Qwen3-30B-A3B
        shape): layer holds ATTN_KEYS-style device pointers (q_w .. o_b,
        in_norm, q_norm, k_norm)."""
        L = ObsAttnLayer(*(_ptr(layer[k]) for k in ObsAttnLayer.KEYS))
        self._check(lib().obs_attn_decode(self.ctx, C.byref(L), _ptr(x), _ptr(k_cache), _ptr(v_cache_t), max_len,
                                          float(eps), float(theta), _ptr(state), _ptr(x1)))

    def layer_decode(self, layer: Dict, cfg: "MoeConfig", moe: "MoeLayer", x, k_cache, v_cache_t, max_len: int,
                     eps: float, theta: float, state, x1, y, ids_out=None, w_out=None) -> None:
        """forward_layer (forward.rs:398-443) in one launch: attn_decode
        (x -> x1) then moe_decode with the post-attention norm (x1 -> y, x1 the
        residual), bit for bit."""
        L = ObsAttnLayer(*(_ptr(layer[k]) for k in ObsAttnLayer.KEYS))
        c, m = cfg.to_c(), moe.to_c()
        self._check(lib().obs_layer_decode(self.ctx, C.byref(L), C.byref(c), C.byref(m), _ptr(x), _ptr(k_cache),
                                           _ptr(v_cache_t), max_len, float(eps), float(theta), _ptr(state), _ptr(x1),
                                           _ptr(y), _ptr(ids_out), _ptr(w_out)))

    # -- prefill of the layers around the MoE block (forward.rs:114-160) --
    def embed_q4_rows(self, w, s, b, hidden: int, vocab: int, tokens, n_tokens: int, out, group: int = 64) -> None:
        self._check(lib().obs_embed_q4_rows(self.ctx, _ptr(w), _ptr(s), _ptr(b), hidden, group, vocab, _ptr(tokens),
                                            n_tokens, _ptr(out)))

    def attn_prep_rows(self, q, k, v, q_norm, k_norm, k_cache, v_cache_t, n_heads: int, n_kv: int, head_dim: int,
                       max_len: int, eps: float, theta: float, pos0: int, n_tokens: int, q_ld: int = 0,
                       kv_ld: int = 0) -> None:
        """q_ld, kv_ld: row strides in elements (0: dense rows)."""
        self._check(lib().obs_attn_prep_rows(self.ctx, _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm),
                                             _ptr(k_cache), _ptr(v_cache_t), n_heads, n_kv, head_dim, max_len, eps,
                                             theta, pos0, n_tokens, q_ld, kv_ld))

    def sdpa_prefill(self, q, k_cache, v_cache_t, out, n_heads: int, n_kv: int, head_dim: int, max_len: int,
                     pos0: int, n_tokens: int, q_ld: int = 0) -> None:
        self._check(lib().obs_sdpa_prefill(self.ctx, _ptr(q), _ptr(k_cache), _ptr(v_cache_t), _ptr(out), n_heads,
                                           n_kv, head_dim, max_len, pos0, n_tokens, q_ld))

    def download_raw(self, ptr: int, shape, dtype) -> np.ndarray:
        """Copies device bytes at `ptr` into a new host array (Buffer::contents after a drain)."""
        out = np.empty(shape, dtype=dtype)
        if out.nbytes:
            self._check(lib().obs_download(self.ctx, out.ctypes.data, ptr, out.nbytes))
        return out

    def prefill_routing(self, cfg: "MoeConfig", T: int, ws) -> Tuple[np.ndarray, np.ndarray]:
        """(ids int32 [T, top_k], weights fp32 [T, top_k]) that a moe_prefill
        with computed routing left at the start of its workspace: the values
        prefill_batched reads back per token with read_route (forward.rs:175-182)."""
        R = T * cfg.top_k
        base = _ptr(ws)
        ids = self.download_raw(base, (T, cfg.top_k), np.int32)
        w = self.download_raw(base + (4 * R + 255) // 256 * 256, (T, cfg.top_k), np.float32)
        return ids, w

    def moe_prefill_workspace(self, cfg: "MoeConfig", T: int) -> int:
        c = cfg.to_c()
        return int(lib().obs_moe_prefill_workspace(C.byref(c), T))

    def moe_prefill(self, cfg: "MoeConfig", layer: "MoeLayer", X, Y, T: int, ids=None, weights=None,
                    residual=None, ws=None, ws_bytes: Optional[int] = None) -> None:
        c, l = cfg.to_c(), layer.to_c()
        if ws_bytes is None:
            ws_bytes = ws.nbytes if isinstance(ws, DeviceBuffer) else 0
        self._check(lib().obs_moe_prefill(self.ctx, C.byref(c), C.byref(l), _ptr(X), _ptr(residual), _ptr(Y), T,
                                          _ptr(ids), _ptr(weights), _ptr(ws), ws_bytes))


@dataclass
class MoeConfig:
    """Shape constants from Qwen3MoeConfig (src/model.rs:7-23)."""
    n_exp: int = 128
    top_k: int = 8
    hidden: int = 2048
    inter: int = 768
    group: int = 64
    norm_topk: bool = True
    rms_eps: float = 1e-6  # rms_norm_eps (model.rs:18); used when the layer has norm_w
    # ROUTE_REF: f16 logits and weights, as moe_routing_topk.metal sees them; ROUTE_F32: fp32
    route_rule: int = 0

    def to_c(self) -> ObsMoeConfig:
        return ObsMoeConfig(self.n_exp, self.top_k, self.hidden, self.inter, self.group, int(bool(self.norm_topk)),
                            float(self.rms_eps), int(self.route_rule))


PROJ_KEYS = ("gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b",
             "router_w", "router_s", "router_b")


@dataclass
class MoeLayer:
    """One layer of the HBM-resident expert table: device pointers of the
    stacked switch_mlp tensors plus the 8-bit router gate (replaces the SSD
    ExpertIndex + expert_pool, disk_io.rs:36-102, forward.rs:79-89)."""
    ptrs: Dict[str, int] = field(default_factory=dict)
    block: Optional[DeviceBuffer] = None  # the device block a checkpoint load filled

    @classmethod
    def upload(cls, exe: ObsidianExecutor, tensors: Dict[str, np.ndarray]) -> "MoeLayer":
        """tensors: the PROJ_KEYS arrays, plus optionally "norm_w" (the layer's
        post_attention_layernorm.weight, bf16 [hidden], forward.rs:419)."""
        ptrs = {k: exe.upload(tensors[k]).ptr for k in PROJ_KEYS}
        if tensors.get("norm_w") is not None:
            ptrs["norm_w"] = exe.upload(tensors["norm_w"]).ptr
        return cls(ptrs)

    def to_c(self) -> ObsMoeLayer:
        return ObsMoeLayer(*[self.ptrs[k] for k in PROJ_KEYS], self.ptrs.get("norm_w"))


class MoeRouter:
    """router.rs:16-94. `route` = dispatch + drain + read; `route_dispatch`
    returns device buffers; `read_route` reads them after a drain."""

    def __init__(self, n_experts: int, top_k: int, norm_topk: bool, rule: int = 0):
        self.n_experts, self.top_k, self.norm_topk, self.rule = n_experts, top_k, norm_topk, rule

    def route_dispatch(self, exe: ObsidianExecutor, gate_logits: DeviceBuffer, T: int = 1):
        idx = exe.alloc((T, self.top_k), np.int32)
        w = exe.alloc((T, self.top_k), np.float32)
        exe.route_topk(gate_logits, idx, w, T, self.n_experts, self.top_k, self.norm_topk, self.rule)
        return idx, w

    def read_route(self, idx_buf: DeviceBuffer, w_buf: DeviceBuffer):
        ids = idx_buf.download()
        w = w_buf.download()
        if ids.shape[0] == 1:
            return [int(i) for i in ids[0]], [float(v) for v in w[0]]
        return ids, w

    def route(self, exe: ObsidianExecutor, gate_logits: DeviceBuffer):
        idx, w = self.route_dispatch(exe, gate_logits, 1)
        exe.drain()
        out = self.read_route(idx, w)
        idx.free()
        w.free()
        return out


def gate_gpu(exe: ObsidianExecutor, layer: MoeLayer, cfg: MoeConfig, x: DeviceBuffer, T: int = 1) -> DeviceBuffer:
    """forward.rs:386-397: router logits for T tokens (fp32 here)."""
    out = exe.alloc((T, cfg.n_exp), np.float32)
    exe.q8_gate_logits(layer.ptrs["router_w"], layer.ptrs["router_s"], layer.ptrs["router_b"], x, out, T,
                       cfg.hidden, cfg.n_exp, cfg.group)
    return out


def dequant(exe: ObsidianExecutor, w, s, b, x: DeviceBuffer, in_f: int, out_f: int) -> DeviceBuffer:
    """forward.rs:303-310: y = dequant(W) . x (one token), bf16 out."""
    y = exe.alloc((out_f,), np.uint16)
    exe.q4_matvec(w, s, b, x, in_f, out_f, 64, y_bf16=y)
    return y


def matmul_raw(exe: ObsidianExecutor, w, s, b, xc: DeviceBuffer, t: int, in_f: int, out_f: int) -> DeviceBuffer:
    """forward.rs:313-321: Y[t, out] = Xc[t, in] . dequant(W)^T (bf16)."""
    y = exe.alloc((t, out_f), np.uint16)
    exe.q4_matmul(w, s, b, xc, y, t, in_f, out_f, 64)
    return y


def swiglu(exe: ObsidianExecutor, g: DeviceBuffer, u: DeviceBuffer, n: int) -> DeviceBuffer:
    """forward.rs:370-375."""
    h = exe.alloc((n,), np.uint16)
    exe.swiglu_raw(g, u, h, n)
    return h


def scaled_add(exe: ObsidianExecutor, acc: DeviceBuffer, y: DeviceBuffer, scale: float, n: int) -> None:
    """forward.rs:376-380: acc += scale * y (in place)."""
    exe.scaled_add_raw(acc, y, scale, n)


def rmsnorm(exe: ObsidianExecutor, x: DeviceBuffer, w: DeviceBuffer, dim: int, rows: int = 1,
            eps: float = 1e-6) -> DeviceBuffer:
    """forward.rs:345-357 (Model::rmsnorm, rmsnorm.metal): a new bf16 [rows, dim]
    buffer holding rmsnorm(x) * w."""
    out = exe.alloc((rows, dim), np.uint16)
    exe.rmsnorm_raw(x, w, out, rows, dim, eps)
    return out


@dataclass
class TensorInfo:
    dtype: str
    shape: Tuple[int, ...]
    nbytes: int
    n_pieces: int


class Checkpoint:
    """A model directory on disk: config.json (Qwen3MoeConfig::from_file,
    model.rs:26-30), the safetensors shards of model.safetensors.index.json
    (Weights::load_non_expert, weight_loader.rs:19-71) and the split expert
    files of tools/split_experts.py (ExpertIndex::open, disk_io.rs:36-63).

    ``load_moe_layer`` makes one layer's stacked expert table resident in HBM
    (replacing the per-token paging of read_experts_parallel, disk_io.rs:79-102).
    Parsing and host reads need no GPU; loads go through the native library."""

    def __init__(self, model_dir: str, expert_dir: Optional[str] = None):
        L = lib()
        h = C.c_void_p()
        rc = L.obs_ckpt_open(os.fsencode(model_dir), os.fsencode(expert_dir) if expert_dir else None, C.byref(h))
        if rc != OBS_OK:
            raise ObsError(rc, L.obs_ckpt_error(None).decode())
        self.h = h.value

    def _check(self, rc: int) -> None:
        if rc != OBS_OK:
            raise ObsError(rc, lib().obs_ckpt_error(self.h).decode())

    def config(self) -> Tuple[MoeConfig, int]:
        """(MoeConfig, num_hidden_layers) from config.json."""
        c, n = ObsMoeConfig(), C.c_uint32()
        self._check(lib().obs_ckpt_config(self.h, C.byref(c), C.byref(n)))
        return MoeConfig(c.n_exp, c.top_k, c.hidden, c.inter, c.group, bool(c.norm_topk), c.rms_eps,
                         c.route_rule), n.value

    def tensor_info(self, name: str) -> TensorInfo:
        i = ObsTensorInfo()
        self._check(lib().obs_ckpt_tensor_info(self.h, name.encode(), C.byref(i)))
        return TensorInfo(DTYPES[i.dtype][0], tuple(int(i.shape[k]) for k in range(i.ndim)), int(i.nbytes),
                          int(i.n_pieces))

    def read(self, name: str) -> np.ndarray:
        """The tensor's on-disk bytes as a host array (bf16 as uint16 bit patterns)."""
        info = self.tensor_info(name)
        out = np.empty(info.shape, dtype=DTYPES[_DT_CODE[info.dtype]][1])
        self._check(lib().obs_ckpt_read(self.h, name.encode(), out.ctypes.data, out.nbytes))
        return out

    def load_tensor(self, exe: ObsidianExecutor, name: str) -> DeviceBuffer:
        info = self.tensor_info(name)
        buf = exe.alloc(info.shape, DTYPES[_DT_CODE[info.dtype]][1])
        exe._check(lib().obs_ckpt_load_tensor(exe.ctx, self.h, name.encode(), buf.ptr, buf.nbytes))
        return buf

    def load_moe_layer(self, exe: ObsidianExecutor, layer: int, cfg: Optional[MoeConfig] = None) -> MoeLayer:
        """Layer `layer`'s expert table, router gate and post-attention norm in
        one device block (bf16 scales; f16 ones converted on the device)."""
        cfg = cfg or self.config()[0]
        c = cfg.to_c()
        nbytes = lib().obs_moe_layer_bytes(C.byref(c))
        if nbytes == 0:
            raise ObsError(OBS_E_SHAPE, f"unsupported layer config {cfg}")
        block = exe.alloc((nbytes,), np.uint8)
        out = ObsMoeLayer()
        exe._check(lib().obs_ckpt_load_moe_layer(exe.ctx, self.h, layer, C.byref(c), block.ptr, nbytes,
                                                   C.byref(out)))
        ptrs = {k: getattr(out, k) for k in PROJ_KEYS}
        if out.norm_w:
            ptrs["norm_w"] = out.norm_w
        return MoeLayer(ptrs, block)

    def close(self) -> None:
        if self.h:
            lib().obs_ckpt_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
