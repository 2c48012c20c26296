"""The C-ABI libraries load and export every function their headers declare; host-side
logic that needs no GPU (synthetic GGUF writer, prompt ids, bench guard). CPU only."""
import hashlib
import json
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent


def _declared(header: str):
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(emprise_\w+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", [("emprise_hip.h", "libemprise_hip.so"), ("emprise_host.h", "libemprise_host.so")])
def test_library_exports_every_declared_symbol(header, lib):
    import ctypes
    import emprise_amd
    emprise_amd.hip_lib()
    so = ctypes.CDLL(str(ROOT / "emprise_amd" / lib))
    names = _declared(header)
    assert len(names) > 10
    missing = [n for n in names if not hasattr(so, n)]
    assert not missing, missing


def test_oracle_is_not_linked_by_the_product():
    out = subprocess.run(["ldd", str(ROOT / "emprise_amd" / "libemprise_host.so")], capture_output=True, text=True).stdout
    assert "oracle" not in out and "emprise_ref" not in out
    for src in (ROOT / "emprise_amd").rglob("*"):
        if src.suffix in (".py", ".cpp", ".hpp", ".hip", ".h") and src.is_file():
            assert "oracle" not in src.read_text().replace("oracle/", ""), src


def test_hip_errors_without_device_are_reported():
    """No GPU here: creating a backend fails with a status, not a crash."""
    from emprise_amd import EmpriseError, HipBackend, gpu_available
    if gpu_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(EmpriseError):
        HipBackend(0)


def test_synthetic_gguf_is_deterministic(tmp_path):
    from emprise_amd import TINY, synth_write
    a, b = tmp_path / "a.gguf", tmp_path / "b.gguf"
    synth_write(a, seed=0, **TINY)
    synth_write(b, seed=0, **TINY)
    ha = hashlib.sha256(a.read_bytes()).hexdigest()
    assert ha == hashlib.sha256(b.read_bytes()).hexdigest()
    golden = json.loads((ROOT / "tests" / "golden" / "tiny_generate.json").read_text())
    assert ha == golden["gguf_sha256"]
    c = tmp_path / "c.gguf"
    synth_write(c, seed=1, **TINY)
    assert hashlib.sha256(c.read_bytes()).hexdigest() != ha


def test_synthetic_gguf_distributions(tmp_path):
    """Q6_K sub-scales uniform in [-32, 31], d = fp16(|N| 2e-4); norm weights 1 + 0.02 N."""
    import oracle
    from emprise_amd import TINY, synth_write
    p = tmp_path / "t.gguf"
    synth_write(p, seed=0, **TINY)
    if not oracle.ref_available():
        pytest.skip("reads tensors through the reference loader")
    import ctypes
    R = oracle.ref()
    m = R.ref_open(str(p).encode(), 1 << 30)
    t, nd, nb = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
    shape = (ctypes.c_uint64 * 4)()
    assert R.ref_tensor_info(m, b"blk.0.ffn_gate.weight", ctypes.byref(t), shape, ctypes.byref(nd), ctypes.byref(nb)) == 0
    raw = np.empty(nb.value, np.uint8)
    assert R.ref_tensor_read(m, b"blk.0.ffn_gate.weight", raw.ctypes.data, nb.value) == 0
    blocks = raw.reshape(-1, 210)
    sc = blocks[:, 192:208].view(np.int8)
    assert sc.min() == -32 and sc.max() == 31
    assert abs(sc.mean() + 0.5) < 0.2
    d = blocks[:, 208:210].copy().view(np.float16).astype(np.float64).ravel()
    assert np.all(d >= 0) and abs(d.mean() - 2e-4 * np.sqrt(2 / np.pi)) < 1e-5
    assert R.ref_tensor_info(m, b"blk.0.attn_norm.weight", ctypes.byref(t), shape, ctypes.byref(nd), ctypes.byref(nb)) == 0
    nw = np.empty(nb.value // 4, np.float32)
    assert R.ref_tensor_read(m, b"blk.0.attn_norm.weight", nw.ctypes.data, nb.value) == 0
    assert abs(nw.mean() - 1) < 0.01 and 0.01 < nw.std() < 0.03
    R.ref_close(m)


def test_synth_prompt_ids():
    from emprise_amd import synth_prompt
    ids = synth_prompt(0, 4096, 512)
    assert ids == synth_prompt(0, 4096, 512) and min(ids) >= 0 and max(ids) < 4096
    assert len(set(ids)) > 400


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr


REF_INCLUDE = Path("/root/reference/v1.1/include")


@pytest.mark.skipif(not REF_INCLUDE.exists(), reason="reference tree not mounted")
def test_integration_adapter_compiles(tmp_path):
    """The reference-side adapter in INTEGRATION.md (section 1) compiles against the
    reference's Backend interface (backend.hpp) and this repository's C ABI header."""
    import shutil
    text = (ROOT / "INTEGRATION.md").read_text()
    section = text[text.index("## 1. The adapter"):text.index("## 2. Factory")]
    code = re.search(r"```cpp\n(.*?)```", section, flags=re.S).group(1)
    src = tmp_path / "hip_backend.cpp"
    src.write_text(code)
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("g++ missing")
    r = subprocess.run([gxx, "-std=c++20", "-fsyntax-only", "-Wall", "-Wextra", f"-I{REF_INCLUDE}",
                        f"-I{REF_INCLUDE.parent / 'third_party'}", f"-I{ROOT / 'include'}", str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "delta_net(Gguf& m, const DeltaNet& p) override" in code
