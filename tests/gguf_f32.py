"""Writes small qwen35 GGUF files whose tensors are all F32 and chosen by the test, so
that model paths can be reduced to closed forms (CPU tests of the oracle)."""
import struct

import numpy as np

_MAGIC = 0x46554747


def _string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, value) -> bytes:
    if isinstance(value, str):
        return _string(key) + struct.pack("<I", 8) + _string(value)
    if isinstance(value, float):
        return _string(key) + struct.pack("<If", 6, value)
    return _string(key) + struct.pack("<II", 4, value)


def write(path, meta: dict, tensors: dict, align: int = 32):
    """meta: qwen35 keys without the prefix (plus tokenizer.ggml.eos_token_id under 'eos');
    tensors: name -> float32 array whose numpy shape is the GGUF shape reversed (a matrix
    of `rows` outputs over `cols` inputs is (rows, cols))."""
    kvs = [("general.architecture", "qwen35"), ("general.alignment", align)]
    kvs += [(("tokenizer.ggml.eos_token_id" if k == "eos" else "qwen35." + k), v) for k, v in meta.items()]
    out = struct.pack("<IIQQ", _MAGIC, 3, len(tensors), len(kvs)) + b"".join(_kv(k, v) for k, v in kvs)
    offset, blobs = 0, []
    for name, a in tensors.items():
        a = np.ascontiguousarray(a, dtype=np.float32)
        dims = a.shape[::-1]
        out += _string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", 0, offset)
        blobs.append((offset, a.tobytes()))
        offset = (offset + a.nbytes + align - 1) // align * align
    out += b"\0" * (-len(out) % align)
    data = bytearray(offset)
    for o, b in blobs:
        data[o:o + len(b)] = b
    with open(path, "wb") as f:
        f.write(out + bytes(data))
