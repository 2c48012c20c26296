"""The reference-side adapter of INTEGRATION.md section 1, executed: its text, compiled
with the reference's own backend.cpp / quant.cpp / gguf.cpp and linked to
libemprise_hip.so (oracle/Makefile -> oracle/_ref/libemprise_adapter.so, harness
oracle/adapter_check.cpp), run on the GPU next to the reference's cpu_backend().

The sequence is the reference's for a recurrent layer: delta_net once per prompt
position on the layer's slot (model.cpp:301-306 -> :162-183), then recurrent_block on the
same slot (model.cpp:431-440), which continues from the device state the prefill left
(cuda.cpp:934-984). Bars: each output within 1e-4 of max|ref| (the FP32 per-op bar);
with a one-byte weight budget every op falls back to cpu_backend() and must match it bit
for bit (tests/core.cpp:145-147, which checks feed_forward; here delta_net and
recurrent_block as well).
"""
import ctypes
import os
import tempfile
from pathlib import Path

import numpy as np
import pytest

from emprise_amd import NINE_B, TINY, synth_write

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
ADAPTER = ROOT / "oracle" / "_ref" / "libemprise_adapter.so"
TOL = 1e-4


def _lib():
    if not ADAPTER.exists():
        pytest.skip(f"{ADAPTER} not built (oracle/Makefile, where the reference tree is mounted)")
    lib = ctypes.CDLL(str(ADAPTER))
    F = ctypes.POINTER(ctypes.c_float)
    lib.adapter_recurrent_check.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_uint32,
                                            F, F, F, F, ctypes.c_uint64, ctypes.c_char_p, ctypes.c_size_t]
    lib.adapter_ffn_check.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_uint32, F, F,
                                      ctypes.c_uint64, ctypes.c_char_p, ctypes.c_size_t]
    return lib


def _fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _model(cfg, name):
    d = Path(os.environ.get("EMPRISE_BENCH_DIR", tempfile.gettempdir()))
    p = d / name
    if not p.exists():
        tmp = p.with_suffix(".tmp")
        synth_write(tmp, seed=0, **cfg)
        os.replace(tmp, p)
    return str(p)


def _recurrent(cfg, path, budget, positions, seed=5):
    lib = _lib()
    kh, vh, sd, cw, H = cfg["key_heads"], cfg["value_heads"], cfg["state_dim"], cfg["conv_width"], cfg["hidden"]
    vd = vh * sd
    dn_hip, dn_cpu = np.zeros((positions, vd), np.float32), np.zeros((positions, vd), np.float32)
    rb_hip, rb_cpu = np.zeros(H, np.float32), np.zeros(H, np.float32)
    err = ctypes.create_string_buffer(1024)
    rc = lib.adapter_recurrent_check(path.encode(), budget, 0, kh, vh, sd, cw, cfg["eps"], positions, seed,
                                     _fp(dn_hip), _fp(dn_cpu), _fp(rb_hip), _fp(rb_cpu), H, err, len(err))
    assert rc == 0, err.value.decode()
    return dn_hip, dn_cpu, rb_hip, rb_cpu


def _close(got, ref, what):
    e = float(np.max(np.abs(got.astype(np.float64) - ref)))
    bound = TOL * max(float(np.max(np.abs(ref))), 1e-30)
    assert e <= bound, f"{what}: max abs err {e:.3e} > {bound:.3e}"


@pytest.mark.parametrize("cfg,name,positions", [(TINY, "adapter_tiny.gguf", 64), (NINE_B, "emprise_9b_q6k_seed0.gguf", 16)],
                         ids=["tiny", "9b"])
def test_adapter_prefill_delta_net_then_recurrent_block(cfg, name, positions):
    """delta_net per prompt position, then recurrent_block, on one layer slot of the HIP
    adapter (the state on the device) against cpu_backend() (the state in host spans)."""
    path = _model(cfg, name)
    dn_hip, dn_cpu, rb_hip, rb_cpu = _recurrent(cfg, path, 0, positions)
    for t in range(positions):
        _close(dn_hip[t], dn_cpu[t], f"delta_net at position {t}")
    _close(rb_hip, rb_cpu, "recurrent_block after the prefill")


def test_adapter_one_byte_budget_is_the_cpu_backend():
    """Budget of one byte: no weight fits, so linear, delta_net (its F32 parameters do not
    fit either) and recurrent_block all run on cpu_backend(), bit for bit."""
    path = _model(TINY, "adapter_tiny.gguf")
    dn_hip, dn_cpu, rb_hip, rb_cpu = _recurrent(TINY, path, 1, 8)
    assert np.array_equal(dn_hip.view(np.uint32), dn_cpu.view(np.uint32))
    assert np.array_equal(rb_hip.view(np.uint32), rb_cpu.view(np.uint32))


@pytest.mark.parametrize("budget", [0, 1])
def test_adapter_feed_forward(budget):
    """feed_forward through the adapter: on the device within the FP32 bar, and with a
    one-byte budget the CPU fallback, bit for bit (tests/core.cpp:145-147)."""
    lib = _lib()
    path = _model(TINY, "adapter_tiny.gguf")
    H = TINY["hidden"]
    a, b = np.zeros(H, np.float32), np.zeros(H, np.float32)
    err = ctypes.create_string_buffer(1024)
    assert lib.adapter_ffn_check(path.encode(), budget, 0, 9, _fp(a), _fp(b), H, err, len(err)) == 0, err.value.decode()
    if budget == 1:
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    else:
        _close(a, b, "feed_forward")
