#!/usr/bin/env python3
"""Decode benchmark: 9B-shape qwen35, Q6_K weights, batch-1 greedy decode on one MI355X.

Workload (benchmark config 3): a deterministic synthetic GGUF with the 9B shape (hidden
4096, 32 layers as [GDN,GDN,GDN,attention] x 8, FFN 12288, vocab 151936, Q6_K
matrices, random init), a seeded 512-token prompt, then 128 greedy tokens at context
4096. A "step" is one decoded token. Throughput follows the reference's definition
(chat.cpp:71, :81): (emitted - 1) / (t_last - t_first), with token completion times from
HIP events on the backend stream; the prompt prefill is outside the timed region.

Also reported on the same JSON line:
  roofline      the dominant kernel (by share of step time) from an event-traced eager
                step: algorithmic bytes per launch / mean launch duration vs 8 TB/s
  cpu_baseline  the reference CPU path (the C oracle restating it, OpenMP) decoding a
                bounded sample of the same model on this host's cores
  hbm_measured  the HBM bandwidth a plain read stream and a device copy reach on this GPU,
                and the decode's weight stream as a fraction of the read figure
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def model_file(kind: str, seed: int) -> Path:
    import emprise_amd as ea
    d = Path(os.environ.get("EMPRISE_BENCH_DIR", tempfile.gettempdir()))
    path = d / f"emprise_{kind}_seed{seed}.gguf"
    if not path.exists():
        t = time.time()
        tmp = path.with_suffix(".tmp")
        if kind == "9b_q6k":
            ea.synth_write(tmp, seed=seed, **ea.NINE_B)
        elif kind == "9b_q4km":
            ea.synth_write(tmp, seed=seed, q4_k_m_mix=True, **ea.NINE_B)
        elif kind == "tiny":
            ea.synth_write(tmp, seed=seed, **ea.TINY)
        else:
            raise ValueError(kind)
        os.replace(tmp, path)
        log(f"wrote {path} ({path.stat().st_size / 1e9:.2f} GB) in {time.time() - t:.1f}s")
    return path


def dominant_kernel(trace):
    """Groups traced launches by kernel; returns the one with the largest total time."""
    agg = {}
    for name, nbytes, ms in trace:
        a = agg.setdefault(name, [0, 0, 0.0])
        a[0] += 1
        a[1] += nbytes
        a[2] += ms
    name, (launches, nbytes, ms) = max(agg.items(), key=lambda kv: kv[1][2])
    total_ms = sum(v[2] for v in agg.values())
    return name, launches, nbytes / launches, ms / launches, ms / total_ms, agg


def cpu_info():
    """CPU model name and physical core count of this host (from /proc/cpuinfo)."""
    model, cores = "unknown", set()
    phys = core = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            k, _, val = line.partition(":")
            k, val = k.strip(), val.strip()
            if k == "model name" and model == "unknown":
                model = val
            elif k == "physical id":
                phys = val
            elif k == "core id":
                core = val
            elif not k and phys is not None and core is not None:
                cores.add((phys, core))
                phys = core = None
        if phys is not None and core is not None:
            cores.add((phys, core))
    except OSError:
        pass
    return model, len(cores) or (os.cpu_count() or 1)


def cpu_baseline(path: Path, seconds: float, context: int, position: int):
    """The reference's OpenMP CPU decode (restated in oracle/) on a bounded sample of the
    GPU run's positions: a 4-token prompt, then the model jumps to `position` (zeroed K/V
    rows there, so attention spans position + 1 rows as after the GPU run's prompt) and
    decodes greedily for ~`seconds`."""
    import oracle
    threads = min(16, os.cpu_count() or 1)  # the reference default, model.cpp:51-52
    m = oracle.Model(str(path), context=context, threads=threads)
    import emprise_amd as ea
    prompt = ea.synth_prompt(0, m.vocab, 4)
    logits = None
    for t in prompt:
        logits = m.evaluate(t)
    m.seek(position)
    arrivals, tok = [], int(logits.argmax())
    t0 = time.perf_counter()
    while True:
        logits = m.evaluate(tok)
        tok = int(logits.argmax())
        arrivals.append(time.perf_counter())
        if arrivals[-1] - t0 > seconds and len(arrivals) >= 3:
            break
    m.close()
    rate = (len(arrivals) - 1) / (arrivals[-1] - arrivals[0])
    model, phys = cpu_info()
    return {"value": round(rate, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "cpu_model": model, "physical_cores": phys,
            "sample": f"{len(arrivals)} greedy decode steps of the same 9B-shape model at positions "
                      f"{position}-{position + len(arrivals) - 1} (the GPU run's), oracle/ C restatement of the "
                      f"reference CPU path, OpenMP {threads} threads (the reference's default min(16, hardware "
                      f"threads)) on {model}, {phys} physical cores"}


def copy_probe(mib: int):
    """One device-to-device copy of `mib` MiB through the HIP runtime's copy kernel: the
    known-size reference that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    n = mib << 20
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    for p in (src, dst):
        if hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(n)) != 0:
            raise RuntimeError("hipMalloc failed")
    if hip.hipMemset(src, 1, ctypes.c_size_t(n)) != 0 or hip.hipDeviceSynchronize() != 0:
        raise RuntimeError("hipMemset failed")
    for _ in range(3):
        if hip.hipMemcpy(dst, src, ctypes.c_size_t(n), 3) != 0:  # hipMemcpyDeviceToDevice
            raise RuntimeError("hipMemcpy failed")
    hip.hipDeviceSynchronize()
    hip.hipFree(src)
    hip.hipFree(dst)
    log(f"copied {mib} MiB device to device 3 times")


def hbm_measured() -> dict:
    """Achievable HBM bandwidth measured on this GPU, for a fraction against what the part
    delivers rather than its 8 TB/s peak: the library's plain read stream
    (emprise_hip_stream_read: non-temporal 16-byte loads over 4 GiB, one 8-wave workgroup
    per CU, replayed from a graph, the mean of 12 launches) and the HIP runtime's device-to-device copy of
    2 GiB (read + write bytes, the best of 5, HIP events)."""
    import ctypes
    import emprise_amd as ea
    be = ea.HipBackend(0)
    n = 4 << 30
    buf, sink = be.alloc(n), be.alloc(4096 * 4)
    be.fill(buf, 1.0, n // 4)
    ms = _graph_time_ms(be, lambda: be.stream_read(buf, n, sink), n=4, reps=3)
    read = n / (ms * 1e-3) / 1e9
    be.free(buf)
    be.free(sink)
    be.close()
    hip = ctypes.CDLL("libamdhip64.so")
    n = 2 << 30
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    ev = [ctypes.c_void_p(), ctypes.c_void_p()]
    for p in (src, dst):
        if hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(n)) != 0:
            raise RuntimeError("hipMalloc failed")
    for e in ev:
        if hip.hipEventCreate(ctypes.byref(e)) != 0:
            raise RuntimeError("hipEventCreate failed")
    if hip.hipMemset(src, 1, ctypes.c_size_t(n)) != 0 or hip.hipDeviceSynchronize() != 0:
        raise RuntimeError("hipMemset failed")
    best = float("inf")
    for _ in range(5):
        t = ctypes.c_float()
        if (hip.hipEventRecord(ev[0], None) or hip.hipMemcpyAsync(dst, src, ctypes.c_size_t(n), 3, None) or
                hip.hipEventRecord(ev[1], None) or hip.hipEventSynchronize(ev[1]) or
                hip.hipEventElapsedTime(ctypes.byref(t), ev[0], ev[1])):
            raise RuntimeError("timed copy failed")
        best = min(best, t.value)
    for e in ev:
        hip.hipEventDestroy(e)
    hip.hipFree(src)
    hip.hipFree(dst)
    return {"read_GBps": round(read, 1), "copy_GBps": round(2 * n / (best * 1e-3) / 1e9, 1),
            "how": "read: emprise_hip_stream_read over 4 GiB (non-temporal 16-byte loads, 8 waves per CU), "
                   "graph-replayed, mean of 12; copy: hipMemcpyAsync device to device, 2 GiB, read + write bytes, "
                   "best of 5"}


def traffic_from_profiles(model: str, kernel: str):
    """HBM bytes per launch of `kernel` on `model` measured by the rocprofv3 FETCH_SIZE and
    WRITE_SIZE passes committed under profiles/ (scaled by the copy-kernel calibration),
    or None when no such measurement is committed."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    rec = json.loads(path.read_text()).get(model, {}).get(kernel)
    return None if rec is None else rec.get("bytes_per_launch")


def attention_probe(kv_len: int, calls: int = 40):
    """Eager decode attention at the 9B shape (16 Q / 4 KV heads x 256, RoPE 64) over a
    KV cache of kv_len positions, `calls` launches from the host, for profilers (counters
    per dispatch): one attention + merge per call, seeded synthetic caches and inputs."""
    import numpy as np
    import emprise_amd as ea
    be = ea.HipBackend(0)
    rng = np.random.default_rng(2)
    heads, kv, hd, rot, context = 16, 4, 256, 64, 4096
    kvd = kv * hd
    keys = be.to_device(rng.standard_normal((context, kvd)).astype(np.float32))
    values = be.to_device(rng.standard_normal((context, kvd)).astype(np.float32))
    qkv = be.to_device(rng.standard_normal(heads * hd * 2 + 2 * kvd).astype(np.float32))
    qn, kn = be.vector(np.ones(hd, np.float32)), be.vector(np.ones(hd, np.float32))
    ao = be.alloc(heads * hd * 4)
    pos = be.to_device(np.array([kv_len - 1], np.int32))
    pa = ea.AttentionParams(heads, kv, hd, rot, context, 1e-6, 1e7, qn, kn, keys, values, pos)
    for _ in range(calls):
        be.attention(pa, qkv, ao)
    be.sync()
    be.close()
    log(f"{calls} attention calls at {kv_len} positions")


def gemm_probe(tokens: int, calls: int = 10):
    """Batched projection of `tokens` positions through a 12288 x 4096 Q6_K matrix (the
    9B FFN gate shape) -- the prefill GEMM (fp16 pieces on the matrix cores) -- `calls`
    times, for profilers; seeded synthetic weights and inputs."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "tests"))
    from synth import matrix
    import emprise_amd as ea
    be = ea.HipBackend(0)
    rng = np.random.default_rng(5)
    rows, cols = 12288, 4096
    w = be.upload_weight(ea.Q6_K, cols, rows, matrix(rng, ea.Q6_K, rows, cols))
    x = be.to_device(rng.standard_normal((tokens, cols)).astype(np.float32))
    y = be.alloc(tokens * rows * 4)
    for _ in range(calls):
        be.linear_batch(w, x, y, tokens)
    be.sync()
    be.close()
    log(f"{calls} batched projections of {tokens} tokens through {rows} x {cols} Q6_K")


def prefill_probe(tokens: int):
    """Two batched prefills of a `tokens`-token seeded prompt through the 9B Q4_K_M mix
    (C4a's workload), for profilers."""
    import emprise_amd as ea
    path = model_file("9b_q4km", seed=0)
    model = ea.Model(path, context=4096)
    prompt = ea.synth_prompt(1, model.info.vocab, tokens + 1)
    for _ in range(2):
        _, arr = model.generate(prompt, 1)
        log(f"prefill of {tokens} tokens: {arr[0]:.4f} s")
    model.close()


def _graph_time_ms(be, fn, n=20, reps=5):
    """Mean duration of `fn`'s launches, replayed n times per graph, reps graphs."""
    fn()
    be.sync()
    be.graph_begin()
    for _ in range(n):
        fn()
    g = be.graph_end()
    be.graph_launch(g)
    be.sync()
    be.event_record(0)
    for _ in range(reps):
        be.graph_launch(g)
    be.event_record(1)
    ms = be.event_elapsed(0, 1) / (n * reps)
    be.graph_destroy(g)
    return ms


def suite(args):
    """The benchmark spec's other configurations, one JSON line each on stdout:
    C1 standalone matvecs (Q6_K, Q4_K, Q8 activations) and small batches of 2-4 inputs,
    C2 GDN step and attention at the 9B shape, C4a batched prefill of 2048 tokens, a
    draft-verification block against decode steps, and C4b fast-q8 decode on the
    Q4_K_M-mix model. Synthetic seeded inputs as in the tests (tests/synth.py)."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "tests"))
    from synth import matrix
    import emprise_amd as ea

    def emit(rec):
        print(json.dumps(rec), flush=True)

    shapes = [(4096, 4096), (12288, 4096), (4096, 12288), (151936, 4096)]
    for q8 in (False, True):
        be = ea.HipBackend(0, quantize_activations=q8)
        for wtype in ((ea.Q6_K,) if q8 else (ea.Q6_K, ea.Q4_K)):
            for rows, cols in shapes:
                rng = np.random.default_rng(rows + cols)
                raw = matrix(rng, wtype, rows, cols)
                w = be.upload_weight(wtype, cols, rows, raw)
                x = be.to_device(rng.standard_normal(cols).astype(np.float32))
                y = be.alloc(rows * 4)
                ms = _graph_time_ms(be, lambda: be.linear(w, x, y))
                gbs = len(raw) / (ms * 1e-3) / 1e9
                emit({"config": "C1", "op": "matvec", "weights": "Q6_K" if wtype == ea.Q6_K else "Q4_K",
                      "activations": "q8" if q8 else "f32", "rows": rows, "cols": cols, "bytes": len(raw),
                      "us": round(ms * 1e3, 2), "GBps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
                be.free(x)
                be.free(y)
                be.weight_free(w)
        be.close()

    # a7 small batches: K inputs through one matrix, the weights read once per launch
    be = ea.HipBackend(0)
    for wtype in (ea.Q6_K, ea.Q4_K):
        for rows, cols in ((12288, 4096), (4096, 12288)):
            rng = np.random.default_rng(rows + cols + 5)
            raw = matrix(rng, wtype, rows, cols)
            w = be.upload_weight(wtype, cols, rows, raw)
            for K in (2, 3, 4):
                X = be.to_device(rng.standard_normal((K, cols)).astype(np.float32))
                Y = be.alloc(K * rows * 4)
                ms = _graph_time_ms(be, lambda: be.linear_batch(w, X, Y, K))
                emit({"config": "C1-batch", "op": "linear_batch (small-batch matvec)",
                      "weights": "Q6_K" if wtype == ea.Q6_K else "Q4_K", "rows": rows, "cols": cols, "K": K,
                      "us": round(ms * 1e3, 2), "us_per_input": round(ms * 1e3 / K, 2),
                      "weight_GBps": round(len(raw) / (ms * 1e-3) / 1e9, 1)})
                be.free(X)
                be.free(Y)
            be.weight_free(w)
    be.close()

    be = ea.HipBackend(0)
    rng = np.random.default_rng(2)
    kh, vh, sd, cw = 16, 32, 128, 4
    ch, vd = 2 * kh * sd + vh * sd, vh * sd
    conv = be.vector((rng.standard_normal(ch * cw) * 0.3).astype(np.float32))
    a = be.vector((-np.exp(rng.standard_normal(vh))).astype(np.float32))
    dt = be.vector((rng.standard_normal(vh) * 0.5).astype(np.float32))
    nw = be.vector((1 + 0.02 * rng.standard_normal(sd)).astype(np.float32))
    bufs = [be.to_device(rng.standard_normal(n).astype(np.float32)) for n in (ch, vd, vh, vh)]
    cs, rs, out = be.alloc(ch * cw * 4), be.alloc(vh * sd * sd * 4), be.alloc(vd * 4)
    be.fill(cs, 0.0, ch * cw)
    be.fill(rs, 0.0, vh * sd * sd)
    p = ea.DeltaNetParams(kh, vh, sd, cw, 1e-6, bufs[0], bufs[1], bufs[2], bufs[3], conv, a, dt, nw, cs, rs, out)
    ms = _graph_time_ms(be, lambda: be.delta_net(p))
    nbytes = 2 * vh * sd * sd * 4 + 2 * ch * cw * 4 + (ch + vd + 2 * vh + vd) * 4
    emit({"config": "C2a", "op": "gdn_step (conv1d + delta rule, 32 v-heads x 128^2 state)", "bytes": nbytes,
          "us": round(ms * 1e3, 2), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)})
    heads, kv, hd, rot, context = 16, 4, 256, 64, 4096
    kvd = kv * hd
    keys = be.to_device(rng.standard_normal((context, kvd)).astype(np.float32))
    values = be.to_device(rng.standard_normal((context, kvd)).astype(np.float32))
    qkv = be.to_device(rng.standard_normal(heads * hd * 2 + 2 * kvd).astype(np.float32))
    qn, kn = be.vector(np.ones(hd, np.float32)), be.vector(np.ones(hd, np.float32))
    ao = be.alloc(heads * hd * 4)
    for L in (512, 2048, 4096):
        pos = be.to_device(np.array([L - 1], np.int32))
        pa = ea.AttentionParams(heads, kv, hd, rot, context, 1e-6, 1e7, qn, kn, keys, values, pos)
        ms = _graph_time_ms(be, lambda: be.attention(pa, qkv, ao))
        nbytes = 8192 * L
        emit({"config": "C2b", "op": "attention (16Q/4KV x 256, RoPE 64, gate)", "kv_len": L, "bytes": nbytes,
              "us": round(ms * 1e3, 2), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)})
        be.free(pos)
    be.close()

    path = model_file("9b_q4km", seed=0)
    model = ea.Model(path, context=4096)
    info = model.info
    prompt = ea.synth_prompt(1, info.vocab, 2049)
    model.generate(prompt[:80], 2)
    t0 = time.perf_counter()
    _, arr = model.generate(prompt, 1)
    wall = time.perf_counter() - t0
    # weights applied per prompt token: every matrix but the output head, plus one embedding row
    per_tok = info.token_weight_bytes
    emit({"config": "C4a", "op": "batched prefill, Q4_K_M mix, projections on fp16 MFMA (exact fp16 pieces, FP32 sums)",
          "prompt_tokens": 2048, "seconds": round(arr[0], 4), "tok_per_s": round(2048 / arr[0], 1),
          "host_wall_s": round(wall, 3), "token_weight_bytes": per_tok})
    model.close()
    # MTP draft verification: a block of positions in one batched pass against one decode
    # step per position (Model::evaluate_block, model.cpp:274-354)
    model = ea.Model(path, context=4096)
    model.prefill(prompt[:512], logits=False)
    at = 512
    for K in (2, 3, 4):
        block, steps = [], []
        for rep in range(6):  # the first repetition warms up and is not counted
            t0 = time.perf_counter()
            model.evaluate_block(prompt[at:at + K])
            block.append(time.perf_counter() - t0)
            t0 = time.perf_counter()
            for t in prompt[at + K:at + 2 * K]:
                model.evaluate(t)
            steps.append(time.perf_counter() - t0)
            at += 2 * K
        emit({"config": "verify", "op": "evaluate_block (one batched pass) vs K decode steps, Q4_K_M mix, "
              "all logits to the host, median of 5", "K": K,
              "block_ms": round(statistics.median(block[1:]) * 1e3, 3),
              "steps_ms": round(statistics.median(steps[1:]) * 1e3, 3)})
    model.close()
    model = ea.Model(path, context=4096, fast_q8=True)
    model.generate(prompt[:8], 4)
    tokens, arr = model.generate(prompt[:512], 257)
    rate = 256 / (arr[-1] - arr[0])
    emit({"config": "C4b", "op": "fast-q8 greedy decode, Q4_K_M mix", "tokens": 256, "tok_per_s": round(rate, 2),
          "token_weight_bytes": info.token_weight_bytes,
          "hbm_roofline_fraction": round(rate * info.token_weight_bytes / 1e9 / HBM_PEAK_GBS, 4)})
    model.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=127, help="timed decode steps (tokens after the first)")
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--context", type=int, default=4096)
    ap.add_argument("--model", default="9b_q6k", choices=["9b_q6k", "9b_q4km", "tiny"])
    ap.add_argument("--fast-q8", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--trace-steps", type=int, default=3)
    ap.add_argument("--no-graph", action="store_true",
                    help="launch every kernel from the host instead of replaying the step graph (for profilers)")
    ap.add_argument("--copy-probe", type=int, metavar="MIB",
                    help="only run a device-to-device copy of MIB MiB (counter calibration) and exit")
    ap.add_argument("--attention-probe", type=int, metavar="KV_LEN",
                    help="only run 40 eager 9B-shape attention calls over KV_LEN positions (for profilers) and exit")
    ap.add_argument("--gemm-probe", type=int, metavar="TOKENS",
                    help="only run 10 batched 12288x4096 Q6_K projections of TOKENS positions (for profilers) and exit")
    ap.add_argument("--prefill-probe", type=int, metavar="TOKENS",
                    help="only run two batched prefills of TOKENS positions on the 9B Q4_K_M mix (for profilers)")
    ap.add_argument("--suite", action="store_true",
                    help="only run the other benchmark configurations (C1, C2, C4), one JSON line each")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); multi-GPU decode is not part of "
              "this build", file=sys.stderr)
        sys.exit(2)
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gemm_probe:
        gemm_probe(args.gemm_probe)
        return
    if args.prefill_probe:
        prefill_probe(args.prefill_probe)
        return
    if args.attention_probe:
        attention_probe(args.attention_probe)
        return
    if args.suite:
        suite(args)
        return

    import emprise_amd as ea
    path = model_file(args.model, seed=0)
    t = time.time()
    model = ea.Model(path, context=args.context, fast_q8=args.fast_q8, graph=not args.no_graph)
    info = model.info
    log(f"loaded {path.name}: {info.weight_bytes / 1e9:.3f} GB on device in {time.time() - t:.1f}s "
        f"({model.backend_name}); {info.token_weight_bytes / 1e9:.4f} GB streamed per token")
    prompt = ea.synth_prompt(0, info.vocab, args.prompt)

    # warmup: instantiates the step graphs and touches every weight once
    model.generate(prompt[:8], max(args.warmup, 2))
    log("warmup done")

    count = args.steps + 1
    t0 = time.perf_counter()
    tokens, arrivals = model.generate(prompt, count)
    wall = time.perf_counter() - t0
    if len(tokens) != count:
        raise RuntimeError(f"generation stopped early ({len(tokens)} of {count} tokens)")
    decode_s = arrivals[-1] - arrivals[0]
    value = args.steps / decode_s
    log(f"prefill {args.prompt} tokens in {arrivals[0]:.3f}s, {args.steps} decode steps in {decode_s:.4f}s "
        f"-> {value:.1f} tok/s (host wall {wall:.3f}s; "
        f"{'per-op launches, no graph' if args.no_graph else 'per-op step graph'})")

    # per-kernel timing of eager steps right after the timed region (same positions range)
    trace = []
    tok = tokens[-1]
    for _ in range(args.trace_steps):
        trace += model.trace_step(tok)
    roofline, per_kernel = None, None
    if trace:
        name, launches, bpl, mspl, share, agg = dominant_kernel(trace)
        achieved = bpl / (mspl * 1e-3) / 1e9
        per_kernel = {k: {"launches": v[0] // args.trace_steps, "ms_per_step": round(v[2] / args.trace_steps, 4),
                          "GBps": round(v[1] / (v[2] * 1e-3) / 1e9, 1) if v[2] > 0 else None}
                      for k, v in sorted(agg.items(), key=lambda kv: -kv[1][2])}
        log(f"dominant kernel {name}: {launches // args.trace_steps} launches/step, {bpl / 1e6:.2f} MB and "
            f"{mspl * 1e3:.2f} us per launch -> {achieved:.0f} GB/s ({share * 100:.0f}% of traced step time)")
        log("per kernel: " + json.dumps(per_kernel))
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(args.model, name),
                    "kernel": name, "bytes_per_launch": int(bpl), "us_per_launch": round(mspl * 1e3, 3),
                    "launches_per_step": launches // args.trace_steps}
    model.close()

    e2e_gbs = value * info.token_weight_bytes / 1e9
    hbm = hbm_measured()
    log(f"measured HBM: a plain read stream reaches {hbm['read_GBps']:.0f} GB/s, a device copy moves "
        f"{hbm['copy_GBps']:.0f} GB/s; the decode streams {e2e_gbs:.0f} GB/s")
    cpu = None
    if not args.no_cpu and args.model.startswith("9b"):
        log(f"cpu baseline: ~{args.cpu_seconds:.0f}s sample")
        cpu = cpu_baseline(path, args.cpu_seconds, args.context, args.prompt)
        log(f"cpu baseline {cpu['value']} tok/s on {cpu['cores']} threads")

    workload = {"9b_q6k": "9B-shape qwen35 Q6_K greedy decode, batch 1",
                "9b_q4km": "9B-shape qwen35 Q4_K_M-mix greedy decode, batch 1",
                "tiny": "tiny qwen35 Q6_K greedy decode, batch 1"}[args.model]
    line = {
        # the headline metric, worded exactly as quoted; other models name their weights
        "metric": {"9b_q6k": "decode tok/s, 9B-shape Q6_K batch 1, 1×MI355X; % of HBM roofline",
                   "9b_q4km": "decode tok/s, 9B-shape Q4_K_M-mix batch 1, 1×MI355X; % of HBM roofline",
                   "tiny": "decode tok/s, tiny qwen35 Q6_K batch 1, 1×MI355X"}[args.model],
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000.0 / value, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8" if args.fast_q8 else "f32",
        "data": "synthetic (seeded random-init GGUF and prompt ids)",
        "config": {"workload": workload + (" (--fast-q8)" if args.fast_q8 else ""), "prompt_tokens": args.prompt,
                   "generated_tokens": count, "context": args.context, "hidden": info.hidden, "layers": info.layers,
                   "vocab": info.vocab, "token_weight_bytes": info.token_weight_bytes,
                   "step": "per-op launches" if args.no_graph else "per-op graph",
                   "parallelism": "single GPU"},
        "hbm_roofline_fraction": round(e2e_gbs / HBM_PEAK_GBS, 4),
        "hbm_measured": hbm,
        "measured_roofline_fraction": round(e2e_gbs / hbm["read_GBps"], 4),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": per_kernel,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
