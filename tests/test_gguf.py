"""The host's GGUF reader (emprise_amd/host/gguf.cpp) on files written here byte by byte:
the reference's fixture and reject cases (tests/core.cpp:29-38 the 1-tensor F32 file,
:48-49 sizes that are not whole blocks or overflow, :102-103 a file cut short by one
byte), plus one file per invariant of the format. CPU only (no device needed)."""
import struct

import pytest

from emprise_amd import InvalidArgument, TINY, gguf_inspect, synth_write

MAGIC = 0x46554747


def _string(s: bytes) -> bytes:
    return struct.pack("<Q", len(s)) + s


def _gguf(tensors, kv=b"", n_kv=0, magic=MAGIC, version=3, align=32, data=None, n_tensors=None):
    """tensors: [(name, dims, type, offset)]; data: bytes of the data section."""
    out = struct.pack("<IIQQ", magic, version, len(tensors) if n_tensors is None else n_tensors, n_kv) + kv
    for name, dims, wtype, offset in tensors:
        out += _string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", wtype, offset)
    out += b"\0" * (-len(out) % align)
    return out + (data if data is not None else b"")


FIXTURE = _gguf([(b"matrix", (2, 2), 0, 0)], data=struct.pack("<4f", 1, 2, -3, 4))


def _inspect(tmp_path, blob, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(blob)
    return gguf_inspect(p)


def test_reference_fixture_reads(tmp_path):
    """core.cpp:29-38: one 2x2 F32 tensor, no metadata."""
    assert _inspect(tmp_path, FIXTURE) == (1, 0)


def test_truncated_file_rejected(tmp_path):
    """core.cpp:102-103: the same file one byte short."""
    with pytest.raises(InvalidArgument, match="past the end"):
        _inspect(tmp_path, FIXTURE[:-1])


def test_block_rows_must_be_whole_blocks(tmp_path):
    """core.cpp:48: 255 Q6_K values are not a whole 256-value block (also for Q4_K), and a
    row of 255 values in a 2-row tensor (510 values, not a multiple of 256 either)."""
    for wtype in (14, 12):
        with pytest.raises(InvalidArgument, match="256-value"):
            _inspect(tmp_path, _gguf([(b"w", (255,), wtype, 0)], data=b"\0" * 256))
        # 512 values in total but rows of 128: every row splits a block
        with pytest.raises(InvalidArgument, match="split a 256-value block"):
            _inspect(tmp_path, _gguf([(b"w", (128, 4), wtype, 0)], data=b"\0" * 420))


def test_size_overflow_rejected(tmp_path):
    """core.cpp:49: an element count whose byte size overflows 64 bits."""
    with pytest.raises(InvalidArgument, match="overflows"):
        _inspect(tmp_path, _gguf([(b"w", (1 << 62, 8), 0, 0)], data=b"\0" * 64))


@pytest.mark.parametrize("blob,what", [
    (_gguf([(b"m", (2, 2), 0, 0)], magic=0x46554748, data=b"\0" * 16), "magic"),
    (_gguf([(b"m", (2, 2), 0, 0)], version=4, data=b"\0" * 16), "version"),
    (_gguf([(b"m", (2, 2), 0, 4)], data=b"\0" * 32), "alignment"),
    (_gguf([(b"a", (4,), 0, 0), (b"b", (4,), 0, 0)], data=b"\0" * 32), "overlap"),
    (_gguf([(b"a", (4,), 0, 0), (b"a", (4,), 0, 32)], data=b"\0" * 64), "repeats"),
    (_gguf([(b"m", (), 0, 0)], data=b"\0" * 16), "rank"),
    (_gguf([(b"m", (1, 1, 1, 1, 1), 0, 0)], data=b"\0" * 16), "rank"),
    (_gguf([(b"m", (2, 0), 0, 0)], data=b"\0" * 16), "empty dimension"),
    (_gguf([(b"m", (32,), 7, 0)], data=b"\0" * 64), "encoding"),
    (_gguf([(b"m", (2, 2), 0, 0)], n_tensors=1 << 40, data=b"\0" * 16), "counts"),
    (_gguf([], kv=_string(b"general.alignment") + struct.pack("<II", 4, 3), n_kv=1), "power of two"),
    (_gguf([], kv=_string(b"k") + struct.pack("<IB", 7, 2), n_kv=1), "boolean"),
    (_gguf([], kv=_string(b"k") + struct.pack("<II", 13, 0), n_kv=1), "undefined"),
    (_gguf([], kv=_string(b"k") + struct.pack("<IB", 0, 1) + _string(b"k") + struct.pack("<IB", 0, 2), n_kv=2),
     "repeated key"),
    (struct.pack("<IIQQ", MAGIC, 3, 0, 1) + struct.pack("<Q", 1 << 40), "string"),
    (struct.pack("<III", MAGIC, 3, 0), "header"),
])
def test_corrupt_files_rejected(tmp_path, blob, what):
    with pytest.raises(InvalidArgument, match=what):
        _inspect(tmp_path, blob)


def test_synthetic_model_reads(tmp_path):
    """The synthetic tiny qwen35 GGUF that the tests and the benchmark use."""
    p = tmp_path / "tiny.gguf"
    synth_write(p, seed=0, **TINY)
    n_tensors, n_meta = gguf_inspect(p)
    # token_embd, output, output_norm + 3 GDN layers of 14 tensors (2 norms, 3 FFN, qkv, gate,
    # alpha, beta, out, conv1d, a, dt bias, ssm norm) + 1 attention layer of 11
    assert n_tensors == 3 + 3 * 14 + 11
    assert n_meta >= 15
