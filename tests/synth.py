"""Seeded synthetic GGUF blocks for the op-level tests (config 1 of the benchmark
spec): Q6_K codes and Q4_K nibbles uniform bytes, Q6_K int8 sub-scales uniform in
[-32, 31], Q6_K d = fp16(|N(0,1)| * 2e-4), Q4_K 6-bit scales/mins uniform and
d, dmin = fp16(|N(0,1)| * 1e-3)."""
from __future__ import annotations

import numpy as np


def q6k_blocks(rng: np.random.Generator, nblocks: int, d_scale: float = 2e-4) -> np.ndarray:
    b = rng.integers(0, 256, size=(nblocks, 210), dtype=np.uint8)
    b[:, 192:208] = rng.integers(-32, 32, size=(nblocks, 16), dtype=np.int8).view(np.uint8)
    d = (np.abs(rng.standard_normal(nblocks)) * d_scale).astype(np.float16)
    b[:, 208:210] = d.view(np.uint8).reshape(nblocks, 2)
    return b


def q4k_blocks(rng: np.random.Generator, nblocks: int, d_scale: float = 1e-3) -> np.ndarray:
    b = rng.integers(0, 256, size=(nblocks, 144), dtype=np.uint8)
    d = (np.abs(rng.standard_normal((nblocks, 2))) * d_scale).astype(np.float16)
    b[:, 0:4] = d.view(np.uint8).reshape(nblocks, 4)
    return b


def matrix(rng: np.random.Generator, wtype: int, rows: int, cols: int) -> bytes:
    """GGUF bytes of a rows x cols matrix (row-major, rows of whole blocks)."""
    from emprise_amd import BF16, F16, F32, Q4_K, Q6_K
    if wtype == Q6_K:
        return q6k_blocks(rng, rows * cols // 256).tobytes()
    if wtype == Q4_K:
        return q4k_blocks(rng, rows * cols // 256).tobytes()
    w = rng.standard_normal(rows * cols).astype(np.float32) * 0.05
    if wtype == F32:
        return w.tobytes()
    if wtype == F16:
        return w.astype(np.float16).tobytes()
    if wtype == BF16:
        return (w.view(np.uint32) >> 16).astype(np.uint16).tobytes()
    raise ValueError(wtype)


def encode_q6k_block(q: np.ndarray, scales: np.ndarray, d_bits: int) -> np.ndarray:
    """Independent Q6_K encoder (the reverse of quant.cpp:25-40) for 256 6-bit codes."""
    b = np.zeros(210, dtype=np.uint8)
    for i in range(256):
        half, local = divmod(i, 128)
        seg, lane = divmod(local, 32)
        b[half * 64 + (seg % 2) * 32 + lane] |= (int(q[i]) & 15) << (seg // 2 * 4)
        b[128 + half * 32 + lane] |= (int(q[i]) >> 4) << (seg * 2)
    b[192:208] = np.asarray(scales, dtype=np.int8).view(np.uint8)
    b[208:210] = np.array([d_bits], dtype=np.uint16).view(np.uint8)
    return b


def decode_q4k_block(b: np.ndarray) -> np.ndarray:
    """Independent float64 Q4_K decoder following the GGUF definition (quant.cpp:41-61)."""
    d = float(np.frombuffer(b[0:2].tobytes(), dtype=np.float16)[0])
    dmin = float(np.frombuffer(b[2:4].tobytes(), dtype=np.float16)[0])
    s = b[4:16].astype(np.int64)
    out = np.zeros(256)
    for j in range(8):
        if j < 4:
            sc, mn = s[j] & 63, s[j + 4] & 63
        else:
            sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4)
            mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
        chunk, hi = divmod(j, 2)
        qs = b[16 + chunk * 32: 16 + chunk * 32 + 32].astype(np.int64)
        codes = (qs >> 4) if hi else (qs & 15)
        out[j * 32:(j + 1) * 32] = d * sc * codes - dmin * mn
    return out


def decode_q6k_block(b: np.ndarray) -> np.ndarray:
    """Independent float64 Q6_K decoder (quant.cpp:25-40)."""
    d = float(np.frombuffer(b[208:210].tobytes(), dtype=np.float16)[0])
    sc = b[192:208].view(np.int8).astype(np.int64)
    out = np.zeros(256)
    for i in range(256):
        half, local = divmod(i, 128)
        g, l = divmod(local, 32)
        low = (int(b[half * 64 + (g & 1) * 32 + l]) >> (4 if g >= 2 else 0)) & 15
        high = (int(b[128 + half * 32 + l]) >> (2 * g)) & 3
        out[i] = d * sc[i // 16] * ((low | high << 4) - 32)
    return out


def quantize_like_reference(x):
    """core.cpp:119-125: x' = round(x/s) * fp16(s) per 32, s = amax/127."""
    q = np.empty_like(x)
    for s0 in range(0, x.size, 32):
        blk = x[s0:s0 + 32]
        s = np.float32(np.max(np.abs(blk)) / np.float32(127))
        if s == 0:
            q[s0:s0 + 32] = 0
            continue
        r = np.round(blk / s)
        r = np.where(np.abs(blk / s - np.trunc(blk / s)) == 0.5, np.trunc(blk / s) + np.sign(blk), r)
        q[s0:s0 + 32] = r.astype(np.float32) * np.float32(np.float16(s))
    return q
