"""ctypes bindings of the CPU oracle (TEST INFRASTRUCTURE ONLY).

liboracle.so is the plain-C restatement of the reference's CPU path (eo.c);
_ref/libemprise_ref.so is the reference's own quant/gguf/backend sources compiled
unchanged (present only where it was built from /root/reference). Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and
only to check or time the CPU path -- never as the measured or shipped path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libemprise_ref.so"

F32, F16, Q4_K, Q6_K, BF16 = 0, 1, 12, 14, 30

_lib = None
_ref = None
_fp = ctypes.POINTER(ctypes.c_float)


def _f(a: np.ndarray):
    return a.ctypes.data_as(_fp)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not ORACLE_LIB.exists():
            raise RuntimeError(f"{ORACLE_LIB} missing: run make -C oracle")
        L = ctypes.CDLL(str(ORACLE_LIB))
        vp, sz, u64, u32, i32, f32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_float
        L.eo_half_to_float.restype = f32
        L.eo_half_to_float.argtypes = [ctypes.c_uint16]
        L.eo_encoded_bytes.restype = u64
        L.eo_encoded_bytes.argtypes = [u32, u64]
        L.eo_dequantize.restype = i32
        L.eo_dequantize.argtypes = [u32, vp, sz, _fp, sz]
        L.eo_matvec.restype = i32
        L.eo_matvec.argtypes = [u32, vp, sz, _fp, sz, _fp, sz]
        for fn in (L.eo_sigmoid, L.eo_silu, L.eo_softplus):
            fn.restype = f32
            fn.argtypes = [f32]
        L.eo_rms.argtypes = [_fp, sz, _fp, f32]
        L.eo_rope.argtypes = [_fp, i32, i32, f32]
        L.eo_attention.argtypes = [i32, i32, i32, i32, f32, f32, _fp, _fp, _fp, _fp, _fp, _fp, _fp, sz, i32, _fp]
        L.eo_delta_net.argtypes = [i32, i32, i32, i32, f32] + [_fp] * 11
        L.eo_feed_forward.restype = i32
        L.eo_feed_forward.argtypes = [u32, vp, u32, vp, u32, vp, sz, sz, _fp, _fp]
        L.eo_model_load.restype = vp
        L.eo_model_load.argtypes = [ctypes.c_char_p, sz, i32, ctypes.c_char_p, sz]
        L.eo_model_free.argtypes = [vp]
        L.eo_model_vocab.restype = i32
        L.eo_model_vocab.argtypes = [vp]
        L.eo_model_hidden.restype = i32
        L.eo_model_hidden.argtypes = [vp]
        L.eo_model_reset.argtypes = [vp]
        L.eo_model_evaluate.restype = i32
        L.eo_model_evaluate.argtypes = [vp, i32, _fp]
        L.eo_model_evaluate_many.restype = i32
        L.eo_model_evaluate_many.argtypes = [vp, ctypes.POINTER(ctypes.c_int), sz, _fp]
        L.eo_model_generate.restype = i32
        L.eo_model_generate.argtypes = [vp, ctypes.POINTER(ctypes.c_int), sz, sz, ctypes.POINTER(ctypes.c_int), _fp]
        L.eo_model_last_hidden.restype = i32
        L.eo_model_last_hidden.argtypes = [vp, _fp]
        L.eo_model_last_hidden_normed.restype = i32
        L.eo_model_last_hidden_normed.argtypes = [vp, _fp]
        L.eo_model_has_mtp.restype = i32
        L.eo_model_has_mtp.argtypes = [vp]
        L.eo_model_reset_mtp.argtypes = [vp]
        L.eo_model_mtp_draft.restype = i32
        L.eo_model_mtp_draft.argtypes = [vp, _fp, i32, sz, _fp]
        L.eo_model_mtp_hidden.restype = i32
        L.eo_model_mtp_hidden.argtypes = [vp, _fp]
        L.eo_quantize_q8.argtypes = [_fp, sz, _fp]
        L.eo_model_seek.restype = i32
        L.eo_model_seek.argtypes = [vp, sz]
        L.eo_model_set_quantize_activations.argtypes = [vp, i32]
        L.eo_model_set_trace.argtypes = [vp, TRACE_FN, vp]
        L.eo_last_error.restype = ctypes.c_char_p
        _lib = L
    return _lib


def ref_available() -> bool:
    return REF_LIB.exists()


REF_MODEL_LIB = HERE / "_ref" / "libemprise_refmodel.so"
_refm = None


def ref_model_available() -> bool:
    return REF_MODEL_LIB.exists()


def refm() -> ctypes.CDLL:
    """The reference's own Model and Tokenizer (model.cpp, tokenizer.cpp, ...) over a C
    ABI (ref_model_shim.cpp), on its CPU backend."""
    global _refm
    if _refm is None:
        if not REF_MODEL_LIB.exists():
            raise RuntimeError(f"{REF_MODEL_LIB} missing (built only where the reference tree is mounted)")
        R = ctypes.CDLL(str(REF_MODEL_LIB))
        vp, u64, i32, i64 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_int64
        R.refm_last_error.restype = ctypes.c_char_p
        R.refm_open.restype = vp
        R.refm_open.argtypes = [ctypes.c_char_p, u64, ctypes.c_uint]
        R.refm_close.argtypes = [vp]
        R.refm_set_trace.argtypes = [vp, TRACE_FN, vp]
        R.refm_reset.restype = i32
        R.refm_reset.argtypes = [vp]
        R.refm_evaluate.restype = i32
        R.refm_evaluate.argtypes = [vp, i32, _fp, u64]
        R.refm_evaluate_block.restype = i32
        R.refm_evaluate_block.argtypes = [vp, ctypes.POINTER(ctypes.c_int), u64, _fp, u64]
        R.refm_prefill.restype = i32
        R.refm_prefill.argtypes = [vp, ctypes.POINTER(ctypes.c_int), u64, _fp, u64]
        R.refm_last_hidden.restype = i32
        R.refm_last_hidden.argtypes = [vp, i32, _fp, u64]
        R.refm_mtp_draft.restype = i32
        R.refm_mtp_draft.argtypes = [vp, _fp, u64, i32, u64, _fp, u64]
        R.refm_mtp_hidden.restype = i32
        R.refm_mtp_hidden.argtypes = [vp, _fp, u64]
        R.refm_reset_mtp.restype = i32
        R.refm_reset_mtp.argtypes = [vp]
        R.refm_encode.restype = i64
        R.refm_encode.argtypes = [vp, ctypes.c_char_p, u64, i32, ctypes.POINTER(ctypes.c_int), u64]
        R.refm_decode.restype = i64
        R.refm_decode.argtypes = [vp, i32, ctypes.c_char_p, u64]
        R.refm_chat_prompt.restype = i64
        R.refm_chat_prompt.argtypes = [vp, ctypes.c_char_p, u64, ctypes.c_char_p, u64]
        _refm = R
    return _refm


def ref() -> ctypes.CDLL:
    global _ref
    if _ref is None:
        if not REF_LIB.exists():
            raise RuntimeError(f"{REF_LIB} missing (built only where the reference tree is mounted)")
        R = ctypes.CDLL(str(REF_LIB))
        vp, sz, u64, u32, i32, f32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_float
        R.ref_last_error.restype = ctypes.c_char_p
        R.ref_half_to_float.restype = f32
        R.ref_half_to_float.argtypes = [ctypes.c_uint16]
        R.ref_encoded_bytes.restype = i32
        R.ref_encoded_bytes.argtypes = [u32, u64, ctypes.POINTER(u64)]
        R.ref_dequantize.restype = i32
        R.ref_dequantize.argtypes = [u32, vp, sz, _fp, sz]
        R.ref_matvec.restype = i32
        R.ref_matvec.argtypes = [u32, vp, sz, _fp, sz, _fp, sz]
        R.ref_open.restype = vp
        R.ref_open.argtypes = [ctypes.c_char_p, u64]
        R.ref_close.argtypes = [vp]
        R.ref_tensor_info.restype = i32
        R.ref_tensor_info.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(u32), ctypes.POINTER(u64), ctypes.POINTER(u32), ctypes.POINTER(u64)]
        R.ref_tensor_read.restype = i32
        R.ref_tensor_read.argtypes = [vp, ctypes.c_char_p, vp, u64]
        R.ref_metadata_json.restype = i32
        R.ref_metadata_json.argtypes = [vp, ctypes.c_char_p, sz]
        R.ref_linear.restype = i32
        R.ref_linear.argtypes = [vp, ctypes.c_char_p, _fp, sz, _fp, sz]
        R.ref_feed_forward.restype = i32
        R.ref_feed_forward.argtypes = [vp, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _fp, sz, _fp]
        R.ref_delta_net.restype = i32
        R.ref_delta_net.argtypes = [vp, i32, i32, i32, i32, f32] + [_fp] * 11
        R.ref_recurrent_block.restype = i32
        R.ref_recurrent_block.argtypes = [vp, ctypes.c_char_p, i32, i32, i32, i32, f32, _fp, _fp, _fp, _fp, _fp, sz, _fp, _fp, _fp]
        _ref = R
    return _ref


# ---- numpy-facing helpers -------------------------------------------------------

def half_to_float(h: int) -> float:
    return lib().eo_half_to_float(h)


def dequantize(wtype: int, raw: bytes, n: int) -> np.ndarray:
    buf = np.frombuffer(raw, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    if lib().eo_dequantize(wtype, buf.ctypes.data, buf.nbytes, _f(out), n):
        raise ValueError(lib().eo_last_error().decode())
    return out


def matvec(wtype: int, raw, x: np.ndarray, rows: int) -> np.ndarray:
    buf = np.frombuffer(memoryview(raw).cast("B"), dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    if lib().eo_matvec(wtype, buf.ctypes.data, buf.nbytes, _f(x), x.size, _f(y), rows):
        raise ValueError(lib().eo_last_error().decode())
    return y


def quantize_q8(x: np.ndarray) -> np.ndarray:
    """The --fast-q8 input rule as the CPU check states it (core.cpp:119-125)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().eo_quantize_q8(_f(x), x.size, _f(out))
    return out


def rms(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True)
    w = np.ascontiguousarray(w, dtype=np.float32)
    lib().eo_rms(_f(y), y.size, _f(w), eps)
    return y


def rope(x: np.ndarray, rotary: int, pos: int, base: float) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True)
    lib().eo_rope(_f(y), rotary, pos, base)
    return y


def delta_net(key_heads, value_heads, state_dim, conv_width, eps, qkv, gate, alpha, beta, conv, ssm_a, dt, norm,
              conv_state, rec_state):
    """Backend::delta_net restated; conv_state/rec_state are updated in place."""
    vd = value_heads * state_dim
    out = np.empty(vd, dtype=np.float32)
    args = [np.ascontiguousarray(a, dtype=np.float32) for a in (qkv, gate, alpha, beta, conv, ssm_a, dt, norm)]
    lib().eo_delta_net(key_heads, value_heads, state_dim, conv_width, eps, *[_f(a) for a in args],
                       _f(conv_state), _f(rec_state), _f(out))
    return out


def attention(heads, kv_heads, head_dim, rotary, rope_base, eps, q_norm, k_norm, qg, k, v, keys, values, length, pos):
    """attention_preout restated; keys/values (context x kv*hd) get row length-1."""
    out = np.empty(heads * head_dim, dtype=np.float32)
    qg = np.array(qg, dtype=np.float32, copy=True)
    k = np.array(k, dtype=np.float32, copy=True)
    v = np.ascontiguousarray(v, dtype=np.float32)
    qn = np.ascontiguousarray(q_norm, dtype=np.float32)
    kn = np.ascontiguousarray(k_norm, dtype=np.float32)
    lib().eo_attention(heads, kv_heads, head_dim, rotary, rope_base, eps, _f(qn), _f(kn), _f(qg), _f(k), _f(v),
                       _f(keys), _f(values), length, pos, _f(out))
    return out


# eo_trace_fn / emprise_trace_fn: (user, position, name, data, n)
TRACE_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float),
                            ctypes.c_uint64)


def trace_recorder(store: dict):
    """A trace hook that keeps a copy of every tensor as store[f"{position}.{name}"]
    (the naming of the reference's tests/fused_check.cpp:21-23)."""
    def hook(_user, position, name, data, n):
        store[f"{position}.{name.decode()}"] = np.ctypeslib.as_array(data, shape=(n,)).copy()
    return TRACE_FN(hook)


class Model:
    """The whole CPU decode path over a GGUF file (Model::Impl::evaluate restated)."""

    def __init__(self, path: str, context: int = 4096, threads: int = 0, fast_q8: bool = False):
        err = ctypes.create_string_buffer(512)
        self.m = lib().eo_model_load(str(path).encode(), context, threads, err, 512)
        if not self.m:
            raise RuntimeError(err.value.decode())
        # --fast-q8: every Q6_K projection sees quantize_q8 of its input
        lib().eo_model_set_quantize_activations(self.m, 1 if fast_q8 else 0)
        self.vocab = lib().eo_model_vocab(self.m)
        self.hidden = lib().eo_model_hidden(self.m)

    def close(self):
        if self.m:
            lib().eo_model_free(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        lib().eo_model_reset(self.m)

    def set_trace(self, store):
        """ModelOptions::trace: every tensor evaluate() passes the hook is kept in `store`
        (see trace_recorder); None removes the hook."""
        hook = trace_recorder(store) if store is not None else None
        lib().eo_model_set_trace(self.m, hook if hook else TRACE_FN(), None)
        self._trace = hook  # the previous hook is released only once the library holds the new one

    def evaluate(self, token: int, logits: bool = True):
        out = np.empty(self.vocab, dtype=np.float32) if logits else None
        if lib().eo_model_evaluate(self.m, token, _f(out) if logits else None):
            raise RuntimeError(lib().eo_last_error().decode())
        return out

    def evaluate_many(self, tokens, logits: bool = True):
        """len(tokens) positions at once, with the bits of that many evaluate() calls;
        the logits are the last position's."""
        out = np.empty(self.vocab, dtype=np.float32) if logits else None
        t = (ctypes.c_int * len(tokens))(*tokens)
        if lib().eo_model_evaluate_many(self.m, t, len(tokens), _f(out) if logits else None):
            raise RuntimeError(lib().eo_last_error().decode())
        return out

    def seek(self, position: int):
        """Timing aid: continue at `position` with zeroed K/V rows."""
        if lib().eo_model_seek(self.m, position):
            raise RuntimeError(lib().eo_last_error().decode())

    def last_hidden(self, normed: bool = False) -> np.ndarray:
        out = np.empty(self.hidden, dtype=np.float32)
        (lib().eo_model_last_hidden_normed if normed else lib().eo_model_last_hidden)(self.m, _f(out))
        return out

    @property
    def has_mtp(self) -> bool:
        return bool(lib().eo_model_has_mtp(self.m))

    def mtp_draft(self, hidden, token: int, position: int) -> np.ndarray:
        """Model::mtp_draft (model.cpp:376-397)."""
        h = np.ascontiguousarray(hidden, dtype=np.float32)
        out = np.empty(self.vocab, dtype=np.float32)
        if lib().eo_model_mtp_draft(self.m, _f(h), token, position, _f(out)):
            raise RuntimeError(lib().eo_last_error().decode())
        return out

    def mtp_hidden(self) -> np.ndarray:
        out = np.empty(self.hidden, dtype=np.float32)
        if lib().eo_model_mtp_hidden(self.m, _f(out)):
            raise RuntimeError(lib().eo_last_error().decode())
        return out

    def reset_mtp(self):
        lib().eo_model_reset_mtp(self.m)

    def generate(self, prompt, count: int):
        p = (ctypes.c_int * len(prompt))(*prompt)
        toks = (ctypes.c_int * max(count, 1))()
        margins = np.empty(max(count, 1), dtype=np.float32)
        n = lib().eo_model_generate(self.m, p, len(prompt), count, toks, _f(margins))
        if n < 0:
            raise RuntimeError(lib().eo_last_error().decode())
        return list(toks[:n]), margins[:n].copy()


class RefModel:
    """The reference's own emprise::Model (CPU backend) over a GGUF file, for pinning the
    oracle's model composition and tokenizer; the same method names as Model above."""

    def __init__(self, path: str, context: int = 4096, threads: int = 0):
        self.m = refm().refm_open(str(path).encode(), context, threads)
        if not self.m:
            raise RuntimeError(refm().refm_last_error().decode())
        probe = Model(path, context=8)
        self.vocab, self.hidden = probe.vocab, probe.hidden
        probe.close()
        self._trace = None

    def close(self):
        if self.m:
            refm().refm_close(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc):
        if rc:
            raise RuntimeError(refm().refm_last_error().decode())

    def set_trace(self, store):
        hook = trace_recorder(store) if store is not None else None
        refm().refm_set_trace(self.m, hook if hook else TRACE_FN(), None)
        self._trace = hook

    def reset(self):
        self._check(refm().refm_reset(self.m))

    def evaluate(self, token: int, logits: bool = True):
        out = np.empty(self.vocab, dtype=np.float32) if logits else None
        self._check(refm().refm_evaluate(self.m, token, _f(out) if logits else None, self.vocab))
        return out

    def evaluate_block(self, tokens):
        out = np.empty((len(tokens), self.vocab), dtype=np.float32)
        t = (ctypes.c_int * len(tokens))(*tokens)
        self._check(refm().refm_evaluate_block(self.m, t, len(tokens), _f(out), self.vocab))
        return out

    def prefill(self, tokens):
        out = np.empty(self.vocab, dtype=np.float32)
        t = (ctypes.c_int * len(tokens))(*tokens)
        self._check(refm().refm_prefill(self.m, t, len(tokens), _f(out), self.vocab))
        return out

    def last_hidden(self, normed: bool = False) -> np.ndarray:
        out = np.empty(self.hidden, dtype=np.float32)
        self._check(refm().refm_last_hidden(self.m, 0 if normed else 1, _f(out), self.hidden))
        return out

    def mtp_draft(self, hidden, token: int, position: int):
        h = np.ascontiguousarray(hidden, dtype=np.float32)
        out = np.empty(self.vocab, dtype=np.float32)
        self._check(refm().refm_mtp_draft(self.m, _f(h), h.size, token, position, _f(out), self.vocab))
        return out

    def mtp_hidden(self):
        out = np.empty(self.hidden, dtype=np.float32)
        self._check(refm().refm_mtp_hidden(self.m, _f(out), self.hidden))
        return out

    def reset_mtp(self):
        self._check(refm().refm_reset_mtp(self.m))

    def encode(self, text: str, parse_special: bool = True):
        b = text.encode()
        cap = 4 * len(b) + 16
        ids = (ctypes.c_int * cap)()
        n = refm().refm_encode(self.m, b, len(b), 1 if parse_special else 0, ids, cap)
        if n < 0:
            raise RuntimeError(refm().refm_last_error().decode())
        return list(ids[:n])

    def decode(self, token: int) -> bytes:
        buf = ctypes.create_string_buffer(256)
        n = refm().refm_decode(self.m, token, buf, 256)
        if n < 0:
            raise RuntimeError(refm().refm_last_error().decode())
        return buf.raw[:n]

    def chat_prompt(self, user: str) -> str:
        b = user.encode()
        buf = ctypes.create_string_buffer(len(b) + 256)
        n = refm().refm_chat_prompt(self.m, b, len(b), buf, len(buf))
        if n < 0:
            raise RuntimeError(refm().refm_last_error().decode())
        return buf.raw[:n].decode()
