"""MI355X (gfx950) decode backend for Emprise's qwen35 engine.

The product is native: ``libemprise_hip.so`` (HIP kernels behind the C ABI in
``include/emprise_hip.h``) and ``libemprise_host.so`` (the C++ host: GGUF loader,
qwen35 graph, greedy loop, report; ``include/emprise_host.h``). This module only
loads them with ctypes. There is no fallback: if a library is missing, loading
raises, so nothing can silently run on another path.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
HIP_LIB = PKG_DIR / "libemprise_hip.so"
HOST_LIB = PKG_DIR / "libemprise_host.so"

F32, F16, Q4_K, Q6_K, BF16 = 0, 1, 12, 14, 30

OK, EINVAL, EDEVICE, ENOMEM, ESTATE = 0, 1, 2, 3, 4


# emprise_trace_fn (include/emprise_host.h): (user, position, name, data, n)
TRACE_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float),
                            ctypes.c_uint64)


class EmpriseError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[status {status}] {message}")
        self.status = status


class InvalidArgument(EmpriseError, ValueError):
    """Shape/argument errors (the reference's std::invalid_argument)."""


def encoded_bytes(wtype: int, n: int) -> int:
    """GGUF encoded size (reference gguf.cpp:72-85)."""
    if wtype == F32:
        return n * 4
    if wtype in (F16, BF16):
        return n * 2
    if wtype == Q6_K:
        if n % 256:
            raise ValueError("Q6_K requires blocks of 256 elements")
        return n // 256 * 210
    if wtype == Q4_K:
        if n % 256:
            raise ValueError("Q4_K requires blocks of 256 elements")
        return n // 256 * 144
    raise ValueError(f"Unsupported GGUF tensor encoding: {wtype}")


_hip = None


def hip_lib() -> ctypes.CDLL:
    """Loads libemprise_hip.so (raises when it has not been built)."""
    global _hip
    if _hip is not None:
        return _hip
    if not HIP_LIB.exists():
        raise RuntimeError(f"{HIP_LIB} is missing: run __graft_entry__.build() (make -C emprise_amd)")
    lib = ctypes.CDLL(str(HIP_LIB))
    u64, i32, f32, vp, st = ctypes.c_uint64, ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_int
    P = ctypes.POINTER
    sig = {
        "emprise_hip_last_error": (ctypes.c_char_p, []),
        "emprise_hip_create": (st, [i32, u64, i32, P(vp)]),
        "emprise_hip_destroy": (None, [vp]),
        "emprise_hip_name": (ctypes.c_char_p, [vp]),
        "emprise_hip_capacity": (u64, [vp]),
        "emprise_hip_weight_bytes": (u64, [vp]),
        "emprise_hip_alloc": (st, [vp, ctypes.c_size_t, P(u64)]),
        "emprise_hip_free": (st, [vp, u64]),
        "emprise_hip_upload": (st, [vp, u64, vp, ctypes.c_size_t]),
        "emprise_hip_download": (st, [vp, vp, u64, ctypes.c_size_t]),
        "emprise_hip_fill": (st, [vp, u64, f32, ctypes.c_size_t]),
        "emprise_hip_stream_read": (st, [vp, u64, u64, u64]),
        "emprise_hip_upload_weight": (st, [vp, ctypes.c_uint32, u64, u64, vp, ctypes.c_size_t, P(u64)]),
        "emprise_hip_weight_free": (st, [vp, u64]),
        "emprise_hip_weight_data": (u64, [vp, u64]),
        "emprise_hip_dequantize_rows": (st, [vp, u64, u64, u64, u64]),
        "emprise_hip_weight_download_gguf": (st, [vp, u64, vp, ctypes.c_size_t]),
        "emprise_hip_linear": (st, [vp, u64, u64, u64]),
        "emprise_hip_linear_many": (st, [vp, i32, P(u64), u64, P(u64)]),
        "emprise_hip_linear_batch": (st, [vp, u64, u64, u64, i32]),
        "emprise_hip_linear_batch_strided": (st, [vp, u64, u64, u64, u64, u64, i32]),
        "emprise_hip_linear_batch_many": (st, [vp, i32, vp, u64, u64, u64, u64, i32]),
        "emprise_hip_ffn_gate_up_batch": (st, [vp, u64, u64, u64, u64, u64, u64, i32]),
        "emprise_hip_linear_norm": (st, [vp, vp, i32, P(u64), P(u64)]),
        "emprise_hip_feed_forward": (st, [vp, vp, u64, u64, u64, u64, u64]),
        "emprise_hip_ffn_gate_up": (st, [vp, vp, u64, u64, u64, u64]),
        "emprise_hip_rmsnorm": (st, [vp, u64, u64, u64, i32, f32]),
        "emprise_hip_rmsnorm_rows": (st, [vp, u64, u64, u64, i32, i32, f32]),
        "emprise_hip_add_rmsnorm_rows": (st, [vp, u64, u64, u64, u64, i32, i32, f32]),
        "emprise_hip_add": (st, [vp, u64, u64, i32]),
        "emprise_hip_swiglu": (st, [vp, u64, u64, i32]),
        "emprise_hip_embed": (st, [vp, u64, u64, u64]),
        "emprise_hip_embed_rows": (st, [vp, u64, u64, i32, u64]),
        "emprise_hip_argmax": (st, [vp, u64, i32, u64]),
        "emprise_hip_quantize_q8": (st, [vp, u64, i32, u64, u64]),
        "emprise_hip_delta_net": (st, [vp, vp]),
        "emprise_hip_delta_net_noalloc": (st, [vp, vp]),
        "emprise_hip_delta_net_batch": (st, [vp, vp, i32, u64, u64]),
        "emprise_hip_recurrent": (st, [vp, vp, vp, u64, u64]),
        "emprise_hip_attention": (st, [vp, vp, u64, u64]),
        "emprise_hip_attention_batch": (st, [vp, vp, u64, i32, u64, i32, u64, u64]),
        "emprise_hip_reset_state": (st, [vp]),
        "emprise_hip_sync": (st, [vp]),
        "emprise_hip_advance": (st, [vp, u64, u64, u64, u64]),
        "emprise_hip_lm_head": (st, [vp, vp, u64, u64, u64]),
        "emprise_hip_graph_begin": (st, [vp]),
        "emprise_hip_graph_end": (st, [vp, P(u64)]),
        "emprise_hip_graph_launch": (st, [vp, u64]),
        "emprise_hip_graph_destroy": (st, [vp, u64]),
        "emprise_hip_event_record": (st, [vp, i32]),
        "emprise_hip_event_elapsed": (st, [vp, i32, i32, P(f32)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _hip = lib
    return lib


class Input(ctypes.Structure):
    """emprise_hip_input: v = x + delta; x_out = v; input = rms(v) * norm."""
    _fields_ = [("x", ctypes.c_uint64), ("delta", ctypes.c_uint64), ("x_out", ctypes.c_uint64),
                ("norm", ctypes.c_uint64), ("eps", ctypes.c_float)]


class DeltaNetParams(ctypes.Structure):
    _fields_ = [("key_heads", ctypes.c_int), ("value_heads", ctypes.c_int), ("state_dim", ctypes.c_int),
                ("conv_width", ctypes.c_int), ("eps", ctypes.c_float),
                ("qkv", ctypes.c_uint64), ("gate", ctypes.c_uint64), ("alpha", ctypes.c_uint64),
                ("beta", ctypes.c_uint64), ("conv", ctypes.c_uint64), ("ssm_a", ctypes.c_uint64),
                ("dt", ctypes.c_uint64), ("norm", ctypes.c_uint64), ("conv_state", ctypes.c_uint64),
                ("rec_state", ctypes.c_uint64), ("out", ctypes.c_uint64)]


class RecurrentParams(ctypes.Structure):
    _fields_ = [("qkv_w", ctypes.c_uint64), ("gate_w", ctypes.c_uint64), ("alpha_w", ctypes.c_uint64),
                ("beta_w", ctypes.c_uint64), ("out_w", ctypes.c_uint64), ("conv", ctypes.c_uint64),
                ("ssm_a", ctypes.c_uint64), ("dt", ctypes.c_uint64), ("norm", ctypes.c_uint64),
                ("key_heads", ctypes.c_int), ("value_heads", ctypes.c_int), ("state_dim", ctypes.c_int),
                ("conv_width", ctypes.c_int), ("eps", ctypes.c_float),
                ("conv_state", ctypes.c_uint64), ("rec_state", ctypes.c_uint64)]


class AttentionParams(ctypes.Structure):
    _fields_ = [("heads", ctypes.c_int), ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("rotary", ctypes.c_int), ("context", ctypes.c_int), ("eps", ctypes.c_float),
                ("rope_base", ctypes.c_float), ("q_norm", ctypes.c_uint64), ("k_norm", ctypes.c_uint64),
                ("keys", ctypes.c_uint64), ("values", ctypes.c_uint64), ("position", ctypes.c_uint64),
                ("rope_position", ctypes.c_uint64)]


class HipBackend:
    """Python handle over the C ABI (mirrors emprise::Backend's device API)."""

    def __init__(self, device: int = 0, weight_budget: int = 0, quantize_activations: bool = False):
        self.lib = hip_lib()
        h = ctypes.c_void_p()
        self._check(self.lib.emprise_hip_create(device, weight_budget, int(quantize_activations), ctypes.byref(h)))
        self.h = h
        self._buffers = []

    def _check(self, status: int):
        if status != OK:
            msg = self.lib.emprise_hip_last_error().decode()
            if status == EINVAL:
                raise InvalidArgument(status, msg)
            raise EmpriseError(status, msg)

    def close(self):
        if getattr(self, "h", None):
            self.lib.emprise_hip_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def name(self) -> str:
        return self.lib.emprise_hip_name(self.h).decode()

    @property
    def capacity(self) -> int:
        return self.lib.emprise_hip_capacity(self.h)

    # buffers
    def alloc(self, nbytes: int) -> int:
        out = ctypes.c_uint64()
        self._check(self.lib.emprise_hip_alloc(self.h, nbytes, ctypes.byref(out)))
        return out.value

    def free(self, buf: int):
        self._check(self.lib.emprise_hip_free(self.h, buf))

    def upload(self, dst: int, array: np.ndarray):
        a = np.ascontiguousarray(array)
        self._check(self.lib.emprise_hip_upload(self.h, dst, a.ctypes.data, a.nbytes))

    def download(self, src: int, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        self._check(self.lib.emprise_hip_download(self.h, out.ctypes.data, src, out.nbytes))
        return out

    def to_device(self, array: np.ndarray) -> int:
        a = np.ascontiguousarray(array)
        buf = self.alloc(max(a.nbytes, 4))
        self.upload(buf, a)
        return buf

    def fill(self, dst: int, value: float, n: int):
        self._check(self.lib.emprise_hip_fill(self.h, dst, value, n))

    def stream_read(self, src: int, nbytes: int, sink: int):
        """Reads nbytes (a multiple of 4 KiB) as a plain non-temporal stream; sink takes
        one word per workgroup (4096 uint32): the achievable-read-bandwidth probe."""
        self._check(self.lib.emprise_hip_stream_read(self.h, src, nbytes, sink))

    # weights
    def upload_weight(self, wtype: int, cols: int, rows: int, data) -> int:
        raw = np.ascontiguousarray(np.frombuffer(memoryview(data).cast("B"), dtype=np.uint8))
        out = ctypes.c_uint64()
        self._check(self.lib.emprise_hip_upload_weight(self.h, wtype, cols, rows, raw.ctypes.data, raw.nbytes,
                                                       ctypes.byref(out)))
        return out.value

    def vector(self, values: np.ndarray) -> int:
        v = np.ascontiguousarray(values, dtype=np.float32)
        return self.upload_weight(F32, v.size, 1, v.tobytes())

    def weight_free(self, w: int):
        self._check(self.lib.emprise_hip_weight_free(self.h, w))

    def weight_data(self, w: int) -> int:
        return self.lib.emprise_hip_weight_data(self.h, w)

    def dequantize_rows(self, w: int, row0: int, n: int, out: int):
        self._check(self.lib.emprise_hip_dequantize_rows(self.h, w, row0, n, out))

    def weight_download_gguf(self, w: int, nbytes: int) -> bytes:
        out = np.empty(nbytes, dtype=np.uint8)
        self._check(self.lib.emprise_hip_weight_download_gguf(self.h, w, out.ctypes.data, nbytes))
        return out.tobytes()

    # ops
    def linear(self, w: int, x: int, y: int):
        self._check(self.lib.emprise_hip_linear(self.h, w, x, y))

    def linear_many(self, ws, x: int, ys):
        n = len(ws)
        self._check(self.lib.emprise_hip_linear_many(self.h, n, (ctypes.c_uint64 * n)(*ws), x,
                                                     (ctypes.c_uint64 * n)(*ys)))

    def linear_norm(self, inp: Input, ws, ys):
        n = len(ws)
        self._check(self.lib.emprise_hip_linear_norm(self.h, ctypes.byref(inp), n, (ctypes.c_uint64 * n)(*ws),
                                                     (ctypes.c_uint64 * n)(*ys)))

    def linear_batch(self, w: int, X: int, Y: int, K: int):
        self._check(self.lib.emprise_hip_linear_batch(self.h, w, X, Y, K))

    def linear_batch_strided(self, w: int, X: int, ldx: int, Y: int, ldy: int, K: int):
        self._check(self.lib.emprise_hip_linear_batch_strided(self.h, w, X, ldx, Y, ldy, K))

    def linear_batch_many(self, ws, X: int, ldx: int, Y: int, ldy: int, K: int):
        n = len(ws)
        self._check(self.lib.emprise_hip_linear_batch_many(self.h, n, (ctypes.c_uint64 * n)(*ws), X, ldx, Y, ldy, K))

    def ffn_gate_up_batch(self, gate: int, up: int, X: int, ldx: int, Y: int, ldy: int, K: int):
        self._check(self.lib.emprise_hip_ffn_gate_up_batch(self.h, gate, up, X, ldx, Y, ldy, K))

    def feed_forward(self, gate: int, up: int, down: int, x: int, y: int, inp: Input | None = None):
        self._check(self.lib.emprise_hip_feed_forward(self.h, ctypes.byref(inp) if inp else None, x, gate, up, down, y))

    def ffn_gate_up(self, gate: int, up: int, x: int, hidden: int, inp: Input | None = None):
        self._check(self.lib.emprise_hip_ffn_gate_up(self.h, ctypes.byref(inp) if inp else None, x, gate, up, hidden))

    def rmsnorm(self, x: int, w: int, out: int, n: int, eps: float):
        self._check(self.lib.emprise_hip_rmsnorm(self.h, x, w, out, n, eps))

    def rmsnorm_rows(self, x: int, w: int, out: int, n: int, rows: int, eps: float):
        self._check(self.lib.emprise_hip_rmsnorm_rows(self.h, x, w, out, n, rows, eps))

    def add_rmsnorm_rows(self, x: int, delta: int, w: int, out: int, n: int, rows: int, eps: float):
        self._check(self.lib.emprise_hip_add_rmsnorm_rows(self.h, x, delta, w, out, n, rows, eps))

    def add(self, x: int, y: int, n: int):
        self._check(self.lib.emprise_hip_add(self.h, x, y, n))

    def swiglu(self, gate: int, up: int, n: int):
        self._check(self.lib.emprise_hip_swiglu(self.h, gate, up, n))

    def embed(self, w: int, token: int, out: int):
        self._check(self.lib.emprise_hip_embed(self.h, w, token, out))

    def embed_rows(self, w: int, tokens: int, count: int, out: int):
        self._check(self.lib.emprise_hip_embed_rows(self.h, w, tokens, count, out))

    def argmax(self, logits: int, n: int, index: int):
        self._check(self.lib.emprise_hip_argmax(self.h, logits, n, index))

    def quantize_q8(self, x: int, cols: int, q: int, scales: int):
        self._check(self.lib.emprise_hip_quantize_q8(self.h, x, cols, q, scales))

    def delta_net(self, p: DeltaNetParams):
        self._check(self.lib.emprise_hip_delta_net(self.h, ctypes.byref(p)))

    def delta_net_noalloc(self, p: DeltaNetParams):
        """emprise_hip_delta_net_noalloc: delta_net with no device allocation (fixed scratch)."""
        self._check(self.lib.emprise_hip_delta_net_noalloc(self.h, ctypes.byref(p)))

    def delta_net_batch(self, p: DeltaNetParams, count: int, stride: int, out_stride: int):
        """delta_net over `count` positions: row t of qkv/gate/alpha/beta at t*stride floats,
        row t of out at t*out_stride floats."""
        self._check(self.lib.emprise_hip_delta_net_batch(self.h, ctypes.byref(p), count, stride, out_stride))

    def recurrent(self, p: RecurrentParams, x: int, y: int, inp: Input | None = None):
        self._check(self.lib.emprise_hip_recurrent(self.h, ctypes.byref(p), ctypes.byref(inp) if inp else None, x, y))

    def attention(self, p: AttentionParams, qkv: int, out: int):
        self._check(self.lib.emprise_hip_attention(self.h, ctypes.byref(p), qkv, out))

    def attention_batch(self, p: AttentionParams, qkv: int, count: int, stride: int, first: int, out: int,
                        out_stride: int):
        """attention over positions first .. first+count-1: qkv row t at t*stride floats,
        out row t at t*out_stride floats."""
        self._check(self.lib.emprise_hip_attention_batch(self.h, ctypes.byref(p), qkv, count, stride, first, out,
                                                         out_stride))

    def advance(self, state: int, prompt: int = 0, history: int = 0, nxt: int = 0):
        self._check(self.lib.emprise_hip_advance(self.h, state, prompt, history, nxt))

    def lm_head(self, inp: Input, w: int, logits: int, index: int):
        self._check(self.lib.emprise_hip_lm_head(self.h, ctypes.byref(inp), w, logits, index))

    def sync(self):
        self._check(self.lib.emprise_hip_sync(self.h))

    def graph_begin(self):
        self._check(self.lib.emprise_hip_graph_begin(self.h))

    def graph_end(self) -> int:
        out = ctypes.c_uint64()
        self._check(self.lib.emprise_hip_graph_end(self.h, ctypes.byref(out)))
        return out.value

    def graph_launch(self, g: int):
        self._check(self.lib.emprise_hip_graph_launch(self.h, g))

    def graph_destroy(self, g: int):
        self._check(self.lib.emprise_hip_graph_destroy(self.h, g))

    def event_record(self, slot: int):
        self._check(self.lib.emprise_hip_event_record(self.h, slot))

    def event_elapsed(self, a: int, b: int) -> float:
        ms = ctypes.c_float()
        self._check(self.lib.emprise_hip_event_elapsed(self.h, a, b, ctypes.byref(ms)))
        return ms.value


def gpu_available() -> bool:
    """True when a HIP device is visible (counts devices without initialising one)."""
    try:
        import torch  # noqa: F401  (device counting only)
        return torch.cuda.device_count() > 0
    except Exception:
        return os.path.exists("/dev/kfd")


# ---- host library (include/emprise_host.h) -------------------------------------------

class ModelOptions(ctypes.Structure):
    _fields_ = [("path", ctypes.c_char_p), ("context", ctypes.c_size_t), ("device", ctypes.c_int),
                ("weight_vram_budget", ctypes.c_uint64), ("quantize_activations", ctypes.c_int),
                ("fused", ctypes.c_int), ("graph", ctypes.c_int), ("batch_prefill", ctypes.c_int)]


class ModelProfile(ctypes.Structure):
    _fields_ = [("matrix_seconds", ctypes.c_double), ("non_matrix_seconds", ctypes.c_double),
                ("norm_seconds", ctypes.c_double), ("attention_seconds", ctypes.c_double),
                ("recurrent_seconds", ctypes.c_double), ("matrix_calls", ctypes.c_uint64),
                ("evaluated_tokens", ctypes.c_uint64), ("decode_steps", ctypes.c_uint64),
                ("traced_steps", ctypes.c_uint64)]


class ModelInfo(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("layers", ctypes.c_int), ("heads", ctypes.c_int),
                ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("rotary", ctypes.c_int),
                ("key_heads", ctypes.c_int), ("value_heads", ctypes.c_int), ("state_dim", ctypes.c_int),
                ("conv_width", ctypes.c_int), ("ffn", ctypes.c_int), ("vocab", ctypes.c_int), ("eos", ctypes.c_int),
                ("eps", ctypes.c_float), ("rope_base", ctypes.c_float), ("context", ctypes.c_size_t),
                ("weight_bytes", ctypes.c_uint64), ("token_weight_bytes", ctypes.c_uint64),
                ("load_seconds", ctypes.c_double)]


class TraceRecord(ctypes.Structure):
    """emprise_hip_trace_record: one kernel launch of a traced step."""
    _fields_ = [("kernel", ctypes.c_char_p), ("bytes", ctypes.c_uint64), ("ms", ctypes.c_float)]


class SynthConfig(ctypes.Structure):
    _fields_ = [("seed", ctypes.c_uint64), ("hidden", ctypes.c_int), ("layers", ctypes.c_int), ("ffn", ctypes.c_int),
                ("vocab", ctypes.c_int), ("heads", ctypes.c_int), ("kv_heads", ctypes.c_int),
                ("head_dim", ctypes.c_int), ("rotary", ctypes.c_int), ("key_heads", ctypes.c_int),
                ("value_heads", ctypes.c_int), ("state_dim", ctypes.c_int), ("conv_width", ctypes.c_int),
                ("full_attention_interval", ctypes.c_int), ("context_length", ctypes.c_int),
                ("rope_base", ctypes.c_float), ("eps", ctypes.c_float), ("eos", ctypes.c_int),
                ("matrix_type", ctypes.c_uint32), ("q4_k_m_mix", ctypes.c_int), ("mtp", ctypes.c_int),
                ("tokenizer", ctypes.c_int)]


# The benchmark's model shapes. TINY is config 0 (hidden 512, 4 layers GDN,GDN,GDN,attention,
# FFN 1536, vocab 4096; GDN 4 QK / 8 V heads of 64, conv 4; attention 8 Q / 2 KV heads of 64,
# rope theta 1e7). NINE_B is config 3 (hidden 4096, 32 layers as [GDN,GDN,GDN,attention] x 8,
# GDN 16 QK / 32 V heads of 128, attention 16 Q / 4 KV heads of 256 with 64 rotary dims,
# FFN 12288, vocab 151936). EOS is set to an id that is never produced.
TINY = dict(hidden=512, layers=4, ffn=1536, vocab=4096, heads=8, kv_heads=2, head_dim=64, rotary=16,
            key_heads=4, value_heads=8, state_dim=64, conv_width=4, full_attention_interval=4,
            context_length=4096, rope_base=1e7, eps=1e-6, eos=4096)
NINE_B = dict(hidden=4096, layers=32, ffn=12288, vocab=151936, heads=16, kv_heads=4, head_dim=256, rotary=64,
              key_heads=16, value_heads=32, state_dim=128, conv_width=4, full_attention_interval=4,
              context_length=32768, rope_base=1e7, eps=1e-6, eos=151936)

_host = None


def host_lib() -> ctypes.CDLL:
    """Loads libemprise_host.so (raises when it has not been built)."""
    global _host
    if _host is not None:
        return _host
    hip_lib()
    if not HOST_LIB.exists():
        raise RuntimeError(f"{HOST_LIB} is missing: run __graft_entry__.build() (make -C emprise_amd)")
    lib = ctypes.CDLL(str(HOST_LIB))
    vp, P = ctypes.c_void_p, ctypes.POINTER
    lib.emprise_host_last_error.restype = ctypes.c_char_p
    lib.emprise_model_open.restype = ctypes.c_int
    lib.emprise_model_open.argtypes = [P(ModelOptions), P(vp)]
    lib.emprise_model_close.argtypes = [vp]
    lib.emprise_model_backend_name.restype = ctypes.c_char_p
    lib.emprise_model_backend_name.argtypes = [vp]
    lib.emprise_model_get_info.restype = ctypes.c_int
    lib.emprise_model_get_info.argtypes = [vp, P(ModelInfo)]
    lib.emprise_model_get_profile.restype = ctypes.c_int
    lib.emprise_model_get_profile.argtypes = [vp, P(ModelProfile)]
    lib.emprise_model_reset.restype = ctypes.c_int
    lib.emprise_model_reset.argtypes = [vp]
    lib.emprise_model_evaluate.restype = ctypes.c_int
    lib.emprise_model_evaluate.argtypes = [vp, ctypes.c_int, P(ctypes.c_float)]
    lib.emprise_model_set_trace.restype = ctypes.c_int
    lib.emprise_model_set_trace.argtypes = [vp, TRACE_FN, vp]
    lib.emprise_model_last_hidden.restype = ctypes.c_int
    lib.emprise_model_last_hidden.argtypes = [vp, P(ctypes.c_float)]
    lib.emprise_tokenizer_open.restype = ctypes.c_int
    lib.emprise_tokenizer_open.argtypes = [ctypes.c_char_p, P(vp)]
    lib.emprise_tokenizer_close.argtypes = [vp]
    lib.emprise_model_tokenizer.restype = vp
    lib.emprise_model_tokenizer.argtypes = [vp]
    lib.emprise_tokenizer_encode.restype = ctypes.c_int
    lib.emprise_tokenizer_encode.argtypes = [vp, ctypes.c_char_p, ctypes.c_size_t, ctypes.c_int, P(ctypes.c_int),
                                             ctypes.c_size_t, P(ctypes.c_size_t)]
    lib.emprise_tokenizer_decode.restype = ctypes.c_int
    lib.emprise_tokenizer_decode.argtypes = [vp, ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t, P(ctypes.c_size_t)]
    lib.emprise_tokenizer_chat_prompt.restype = ctypes.c_int
    lib.emprise_tokenizer_chat_prompt.argtypes = [vp, ctypes.c_char_p, ctypes.c_size_t, ctypes.c_char_p,
                                                  ctypes.c_size_t, P(ctypes.c_size_t)]
    lib.emprise_model_last_hidden_normed.restype = ctypes.c_int
    lib.emprise_model_last_hidden_normed.argtypes = [vp, P(ctypes.c_float)]
    lib.emprise_model_evaluate_block.restype = ctypes.c_int
    lib.emprise_model_evaluate_block.argtypes = [vp, P(ctypes.c_int), ctypes.c_size_t, P(ctypes.c_float)]
    lib.emprise_model_has_mtp.restype = ctypes.c_int
    lib.emprise_model_has_mtp.argtypes = [vp]
    lib.emprise_model_mtp_draft.restype = ctypes.c_int
    lib.emprise_model_mtp_draft.argtypes = [vp, P(ctypes.c_float), ctypes.c_int, ctypes.c_size_t, P(ctypes.c_float)]
    lib.emprise_model_mtp_hidden.restype = ctypes.c_int
    lib.emprise_model_mtp_hidden.argtypes = [vp, P(ctypes.c_float)]
    lib.emprise_model_reset_mtp.restype = ctypes.c_int
    lib.emprise_model_reset_mtp.argtypes = [vp]
    lib.emprise_gguf_inspect.restype = ctypes.c_int
    lib.emprise_gguf_inspect.argtypes = [ctypes.c_char_p, P(ctypes.c_uint64), P(ctypes.c_uint64)]
    lib.emprise_model_prefill.restype = ctypes.c_int
    lib.emprise_model_prefill.argtypes = [vp, P(ctypes.c_int), ctypes.c_size_t, P(ctypes.c_float)]
    lib.emprise_model_generate.restype = ctypes.c_int
    lib.emprise_model_generate.argtypes = [vp, P(ctypes.c_int), ctypes.c_size_t, ctypes.c_size_t, P(ctypes.c_int),
                                           P(ctypes.c_size_t), P(ctypes.c_double)]
    lib.emprise_model_trace_step.restype = ctypes.c_int
    lib.emprise_model_trace_step.argtypes = [vp, ctypes.c_int, P(TraceRecord), ctypes.c_size_t, P(ctypes.c_size_t)]
    lib.emprise_synth_write.restype = ctypes.c_int
    lib.emprise_synth_write.argtypes = [P(SynthConfig), ctypes.c_char_p]
    lib.emprise_synth_prompt.restype = ctypes.c_int
    lib.emprise_synth_prompt.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_size_t, P(ctypes.c_int)]
    _host = lib
    return lib


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _host_check(status: int):
    if status != OK:
        msg = host_lib().emprise_host_last_error().decode()
        if status == EINVAL:
            raise InvalidArgument(status, msg)
        raise EmpriseError(status, msg)


def synth_write(path, seed: int = 0, matrix_type: int = Q6_K, q4_k_m_mix: bool = False, mtp: bool = False,
                tokenizer: bool = False, **shape):
    """Writes a deterministic synthetic qwen35 GGUF (see emprise_synth_write); mtp adds the
    next-n block blk.<layers>, tokenizer a qwen35 GPT-2 BPE tokenizer."""
    c = SynthConfig(seed=seed, matrix_type=matrix_type, q4_k_m_mix=int(q4_k_m_mix), mtp=int(mtp),
                    tokenizer=int(tokenizer), **shape)
    _host_check(host_lib().emprise_synth_write(ctypes.byref(c), str(path).encode()))


class Tokenizer:
    """The qwen35 GPT-2 BPE tokenizer of a GGUF file (emprise_tokenizer_*; reference
    include/emprise/tokenizer.hpp). Tokenizer(path) reads the file's metadata without a
    device; Model.tokenizer is the model's own."""

    def __init__(self, path=None, _handle=None, _owner=None):
        if _handle is not None:
            self.t, self._owned, self._owner = _handle, False, _owner
        else:
            h = ctypes.c_void_p()
            _host_check(host_lib().emprise_tokenizer_open(str(path).encode(), ctypes.byref(h)))
            self.t, self._owned, self._owner = h, True, None

    def encode(self, text: str, parse_special: bool = True) -> list:
        b = text.encode() if isinstance(text, str) else bytes(text)
        n = ctypes.c_size_t()
        _host_check(host_lib().emprise_tokenizer_encode(self.t, b, len(b), int(parse_special), None, 0,
                                                        ctypes.byref(n)))
        ids = (ctypes.c_int * max(n.value, 1))()
        _host_check(host_lib().emprise_tokenizer_encode(self.t, b, len(b), int(parse_special), ids, n.value,
                                                        ctypes.byref(n)))
        return list(ids[:n.value])

    def decode(self, token: int) -> bytes:
        n = ctypes.c_size_t()
        _host_check(host_lib().emprise_tokenizer_decode(self.t, token, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(max(n.value, 1))
        _host_check(host_lib().emprise_tokenizer_decode(self.t, token, buf, n.value, ctypes.byref(n)))
        return buf.raw[:n.value]

    def chat_prompt(self, user: str) -> str:
        b = user.encode()
        n = ctypes.c_size_t()
        _host_check(host_lib().emprise_tokenizer_chat_prompt(self.t, b, len(b), None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(max(n.value, 1))
        _host_check(host_lib().emprise_tokenizer_chat_prompt(self.t, b, len(b), buf, n.value, ctypes.byref(n)))
        return buf.raw[:n.value].decode()

    def close(self):
        if self._owned and self.t:
            host_lib().emprise_tokenizer_close(self.t)
        self.t = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def gguf_inspect(path):
    """Validates a GGUF file without a device: (tensor count, metadata key count)."""
    t, m = ctypes.c_uint64(), ctypes.c_uint64()
    _host_check(host_lib().emprise_gguf_inspect(str(path).encode(), ctypes.byref(t), ctypes.byref(m)))
    return t.value, m.value


def synth_prompt(seed: int, vocab: int, n: int) -> list:
    ids = (ctypes.c_int * max(n, 1))()
    _host_check(host_lib().emprise_synth_prompt(seed, vocab, n, ids))
    return list(ids[:n])


class Model:
    """The C++ host's qwen35 model on the MI355X (Model::Model / evaluate / generate)."""

    def __init__(self, path, context: int = 4096, device: int = 0, vram_budget: int = 0, fast_q8: bool = False,
                 fused: bool = True, graph: bool = True, batch_prefill: int = 0):
        """batch_prefill: prompts with at least this many tokens before the last prefill
        in batches (GEMM projections); 0 = the library default (64), -1 = never."""
        lib = host_lib()
        self._path = str(path).encode()
        o = ModelOptions(self._path, context, device, vram_budget, int(fast_q8), int(fused), int(graph),
                         int(batch_prefill))
        m = ctypes.c_void_p()
        _host_check(lib.emprise_model_open(ctypes.byref(o), ctypes.byref(m)))
        self.m = m
        self.info = ModelInfo()
        _host_check(lib.emprise_model_get_info(self.m, ctypes.byref(self.info)))

    @property
    def backend_name(self) -> str:
        return host_lib().emprise_model_backend_name(self.m).decode()

    def close(self):
        if getattr(self, "m", None):
            host_lib().emprise_model_close(self.m)
            self.m = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def reset(self):
        _host_check(host_lib().emprise_model_reset(self.m))

    def evaluate(self, token: int, logits: bool = True):
        out = np.empty(self.info.vocab, dtype=np.float32) if logits else None
        ptr = out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if logits else None
        _host_check(host_lib().emprise_model_evaluate(self.m, token, ptr))
        return out

    def set_trace(self, hook):
        """ModelOptions::trace (model.hpp:18-19): hook(position, name, array) is called
        synchronously by evaluate() at the reference's trace points (attn_norm-L,
        attn_residual-L, l_out-L, result_norm, logits), with a copy of the tensor; None
        removes it."""
        if hook is None:
            _host_check(host_lib().emprise_model_set_trace(self.m, TRACE_FN(), None))
            self._trace = None  # released only once the library no longer holds it
            return

        def tramp(_user, position, name, data, n):
            hook(int(position), name.decode(), np.ctypeslib.as_array(data, shape=(n,)).copy())
        self._trace = TRACE_FN(tramp)
        _host_check(host_lib().emprise_model_set_trace(self.m, self._trace, None))

    def prefill(self, tokens, logits: bool = True):
        """Model::prefill: tokens from the current position on (batched), the last
        position's logits."""
        p = (ctypes.c_int * len(tokens))(*tokens)
        out = np.empty(self.info.vocab, dtype=np.float32) if logits else None
        ptr = out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if logits else None
        _host_check(host_lib().emprise_model_prefill(self.m, p, len(tokens), ptr))
        return out

    def last_hidden(self, normed: bool = False) -> np.ndarray:
        """The residual after the last position with logits (Model::last_hidden_raw), or
        with normed=True that residual through the output norm (Model::last_hidden)."""
        out = np.empty(self.info.hidden, dtype=np.float32)
        fn = host_lib().emprise_model_last_hidden_normed if normed else host_lib().emprise_model_last_hidden
        _host_check(fn(self.m, _fptr(out)))
        return out

    def evaluate_block(self, tokens) -> np.ndarray:
        """Model::evaluate_block: the tokens from the current position on, every
        position's logits (len(tokens) x vocab)."""
        p = (ctypes.c_int * len(tokens))(*tokens)
        out = np.empty((len(tokens), self.info.vocab), dtype=np.float32)
        _host_check(host_lib().emprise_model_evaluate_block(self.m, p, len(tokens), _fptr(out)))
        return out

    @property
    def has_mtp(self) -> bool:
        return bool(host_lib().emprise_model_has_mtp(self.m))

    @property
    def tokenizer(self):
        """The model's tokenizer (Model::tokenizer), or None when the file has none."""
        h = host_lib().emprise_model_tokenizer(self.m)
        return Tokenizer(_handle=ctypes.c_void_p(h), _owner=self) if h else None

    def mtp_draft(self, hidden, token: int, position: int) -> np.ndarray:
        """Model::mtp_draft: the MTP head's logits for the token after `token`."""
        h = np.ascontiguousarray(hidden, dtype=np.float32)
        if h.shape != (self.info.hidden,):
            raise ValueError(f"hidden must have {self.info.hidden} floats")
        out = np.empty(self.info.vocab, dtype=np.float32)
        _host_check(host_lib().emprise_model_mtp_draft(self.m, _fptr(h), token, position, _fptr(out)))
        return out

    def mtp_hidden(self) -> np.ndarray:
        out = np.empty(self.info.hidden, dtype=np.float32)
        _host_check(host_lib().emprise_model_mtp_hidden(self.m, _fptr(out)))
        return out

    def reset_mtp(self):
        _host_check(host_lib().emprise_model_reset_mtp(self.m))

    def profile(self) -> dict:
        """Model::profile (emprise_model_get_profile)."""
        p = ModelProfile()
        _host_check(host_lib().emprise_model_get_profile(self.m, ctypes.byref(p)))
        return {k: getattr(p, k) for k, _ in ModelProfile._fields_}

    def trace_step(self, token: int):
        """One eager step with per-launch HIP event timing: [(kernel, bytes, ms), ...]."""
        cap = 4096
        rec = (TraceRecord * cap)()
        n = ctypes.c_size_t()
        _host_check(host_lib().emprise_model_trace_step(self.m, token, rec, cap, ctypes.byref(n)))
        return [(rec[i].kernel.decode(), rec[i].bytes, rec[i].ms) for i in range(n.value)]

    def generate(self, prompt, count: int):
        """Returns (tokens, arrivals): greedy ids and per-token completion times (s)."""
        p = (ctypes.c_int * len(prompt))(*prompt)
        toks = (ctypes.c_int * max(count, 1))()
        arr = (ctypes.c_double * max(count, 1))()
        n = ctypes.c_size_t()
        _host_check(host_lib().emprise_model_generate(self.m, p, len(prompt), count, toks, ctypes.byref(n), arr))
        return list(toks[:n.value]), list(arr[:n.value])
