#!/usr/bin/env python3
"""Decode benchmark of the forword MI355X path.

Default workload: Llama-3-8B-shaped random-init GGUF (Q4_0 linears, Q8_0
embedding/output), 512-token random prompt, then greedy decode at positions
528..783 (after 16 warm-up steps).  One step = one token forward
(transformer_forward) plus the greedy pick, run device-resident through the
C ABI; the persistent step kernel runs up to 64 steps per launch.

Prints one JSON line:
  value        decode tok/s (weights and KV already in HBM)
  roofline     the dominant kernel (the persistent step kernel, all of the
               decode time): algorithmic bytes of the steps one launch runs
               (weights + embedding row + norm weights + KV read/write) over
               its mean duration, timed with HIP events on the handle's stream
  microbench   quant_matvec GB/s per weight type and shape (>= 1 GiB of
               rotating weight copies so the 256 MB last-level cache cannot
               serve repeats)
  cpu_baseline the oracle (CPU restatement of forword.c) on one core, bounded sample

Other modes: --config lc (8B shape at 32K context, KV rows 0..32767 written
with N(0,1) through kv_write, then greedy decode), --config 70b, --mode decode
(just the timed decode, for profilers), --mode copy (device-to-device copy of
known size: calibrates the memory-traffic counters), --mode micro (only the
quant_matvec microbenchmark, for profiling k_gemv).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "forword.c_amd"))
import fwgpu  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "decode tok/s (8B-shape Q4_0, 1 GPU) + quant-matvec HBM GB/s % of peak"
STEPS_PER_LAUNCH = 64


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Hip:
    """The few HIP runtime calls the timing needs (events on a given stream, D2D copy)."""

    def __init__(self):
        fwgpu.gpu_lib()   # loads libamdhip64 as a dependency
        for name in ("libamdhip64.so", "libamdhip64.so.7", "/opt/rocm/lib/libamdhip64.so"):
            try:
                self.L = C.CDLL(name)
                break
            except OSError:
                continue
        L = self.L
        fwgpu._sig(L, "hipEventCreate", C.c_int, [C.POINTER(C.c_void_p)])
        fwgpu._sig(L, "hipEventRecord", C.c_int, [C.c_void_p, C.c_void_p])
        fwgpu._sig(L, "hipEventSynchronize", C.c_int, [C.c_void_p])
        fwgpu._sig(L, "hipEventElapsedTime", C.c_int, [C.POINTER(C.c_float), C.c_void_p, C.c_void_p])
        fwgpu._sig(L, "hipStreamSynchronize", C.c_int, [C.c_void_p])
        fwgpu._sig(L, "hipMemcpyAsync", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p])
        vpp = C.POINTER(C.c_void_p)
        fwgpu._sig(L, "hipStreamCreate", C.c_int, [vpp])
        fwgpu._sig(L, "hipStreamDestroy", C.c_int, [C.c_void_p])
        fwgpu._sig(L, "hipStreamBeginCapture", C.c_int, [C.c_void_p, C.c_int])
        fwgpu._sig(L, "hipStreamEndCapture", C.c_int, [C.c_void_p, vpp])
        fwgpu._sig(L, "hipGraphInstantiate", C.c_int, [vpp, C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t])
        fwgpu._sig(L, "hipGraphLaunch", C.c_int, [C.c_void_p, C.c_void_p])
        fwgpu._sig(L, "hipGraphExecDestroy", C.c_int, [C.c_void_p])
        fwgpu._sig(L, "hipGraphDestroy", C.c_int, [C.c_void_p])

    def event(self):
        e = C.c_void_p()
        assert self.L.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.L.hipEventRecord(e, stream) == 0

    def ms(self, a, b):
        assert self.L.hipEventSynchronize(b) == 0
        t = C.c_float()
        assert self.L.hipEventElapsedTime(C.byref(t), a, b) == 0
        return float(t.value)

    def sync(self, stream):
        assert self.L.hipStreamSynchronize(stream) == 0

    def stream(self):
        s = C.c_void_p()
        assert self.L.hipStreamCreate(C.byref(s)) == 0
        return s

    def graph_of(self, stream, enqueue):
        """enqueue(stream) captured (thread-local mode) as an executable graph."""
        assert self.L.hipStreamBeginCapture(stream, 1) == 0
        enqueue(stream)
        g, ex = C.c_void_p(), C.c_void_p()
        assert self.L.hipStreamEndCapture(stream, C.byref(g)) == 0
        assert self.L.hipGraphInstantiate(C.byref(ex), g, None, None, 0) == 0
        return g, ex


def step_bytes(cfg, pos, linear_bb=18, embd_bb=34, out_bb=34, mix_bb=None):
    """Algorithmic bytes of one token step at position pos: weights, embedding row, norm
    weights, KV read (rows 0..pos incl. the one just written) and KV write.  mix_bb:
    bytes per 32 values of attn_v and ffn_down in the even layers (Q4_K_M layout)."""
    n, ff, L, hd, kv = cfg.n_embd, cfg.n_ff, cfg.n_layer, cfg.head_dim, cfg.n_head_kv
    n_in = 2 if cfg.use_ffn_gate else 1                 # gate and up, or up alone
    lin = L * ((n // 32) * linear_bb * (2 * n + 2 * kv * hd + n_in * ff) + (ff // 32) * linear_bb * n)
    if mix_bb is not None:
        lin += ((L + 1) // 2) * (mix_bb - linear_bb) * ((n // 32) * kv * hd + (ff // 32) * n)
    head = (n // 32) * out_bb * cfg.n_vocab
    embd = (n // 32) * embd_bb
    norms = 4 * n * (2 * L + 1)
    kvb = L * 2 * kv * hd * 4 * (pos + 1) + L * 2 * kv * hd * 4
    return lin + head + embd + norms + kvb


def linear_shapes(cfg):
    """(rows, cols) of every layer linear (q, k, v, o, gate, up, down)."""
    n, ff, kvd = cfg.n_embd, cfg.n_ff, cfg.n_head_kv * cfg.head_dim
    ffn = [(ff, n), (ff, n), (n, ff)] if cfg.use_ffn_gate else [(ff, n), (n, ff)]
    return ([(n, n), (kvd, n), (kvd, n), (n, n)] + ffn) * cfg.n_layer


def timed_decode(hip, gm, steps):
    """Continue the greedy loop for `steps` steps in launches of STEPS_PER_LAUNCH, each
    bracketed by HIP events on the handle's stream.  Returns (total ms, [(ms, n)])."""
    stream = gm.stream
    launches = []
    done = 0
    hip.sync(stream)
    t_start = hip.event()
    hip.record(t_start, stream)
    while done < steps:
        n = min(STEPS_PER_LAUNCH, steps - done)
        e0, e1 = hip.event(), hip.event()
        hip.record(e0, stream)
        gm.decode(n, copy_out=False)
        hip.record(e1, stream)
        launches.append((e0, e1, n))
        done += n
    t_end = hip.event()
    hip.record(t_end, stream)
    hip.sync(stream)
    total = hip.ms(t_start, t_end)
    return total, [(hip.ms(a, b), n) for a, b, n in launches]


def microbench(hip, min_bytes=1 << 30, reps=48):
    """quant_matvec (operator entry point) GB/s at the microbenchmark shapes: `reps`
    calls over rotating weight copies (>= 1 GiB, so the 256 MB last-level cache cannot
    serve repeats), timed with one event pair around all of them, once as plain
    back-to-back launches and once replayed from a captured graph (fewer launch gaps)."""
    L = fwgpu.gpu_lib()
    out = []
    x = fwgpu.DeviceBuffer.from_array(fwgpu.randn(7, 14336))
    y = fwgpu.DeviceBuffer(14336 * 4)
    st = hip.stream()
    for t in (fwgpu.GGML_Q4_0, fwgpu.GGML_Q5_0, fwgpu.GGML_Q8_0):
        for rows, cols in ((4096, 4096), (14336, 4096), (4096, 14336)):
            w = fwgpu.synth_matrix(t, rows, cols, seed=100 + t)
            copies = max(2, -(-min_bytes // w.nbytes))
            bufs = [fwgpu.DeviceBuffer.from_array(w) for _ in range(copies)]
            algo = w.nbytes + 4 * cols + 4 * rows

            def enqueue(stream, n=reps):
                for i in range(n):
                    assert L.forword_gpu_quant_matvec(bufs[i % copies].ptr, w.nbytes, t, x.ptr, y.ptr,
                                                      cols, rows, stream) == 0

            enqueue(st, copies)                                     # warm-up pass
            hip.sync(st)
            e0, e1 = hip.event(), hip.event()
            hip.record(e0, st)
            enqueue(st)
            hip.record(e1, st)
            us_launch = hip.ms(e0, e1) * 1e3 / reps
            g, ex = hip.graph_of(st, enqueue)
            assert hip.L.hipGraphLaunch(ex, st) == 0                # warm-up replay
            hip.sync(st)
            hip.record(e0, st)
            assert hip.L.hipGraphLaunch(ex, st) == 0
            hip.record(e1, st)
            us = hip.ms(e0, e1) * 1e3 / reps
            hip.L.hipGraphExecDestroy(ex)
            hip.L.hipGraphDestroy(g)
            for b in bufs:
                b.free()
            gbs = algo / (us_launch * 1e-6) / 1e9
            out.append({"type": fwgpu.TYPE_NAMES[t], "rows": rows, "cols": cols, "bytes": algo,
                        "us_per_call": round(us_launch, 2), "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                        "us_per_call_graph": round(us, 2)})
            log(f"microbench {fwgpu.TYPE_NAMES[t]} {rows}x{cols}: {us_launch:.2f} us per call back to back "
                f"({us:.2f} replayed from a graph), {gbs:.0f} GB/s")
    hip.L.hipStreamDestroy(st)
    x.free()
    y.free()
    return out


def host_cpu():
    """CPU model name and the number of cores this process may use."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, len(os.sched_getaffinity(0))


def cpu_baseline(host, budget_s, p0):
    """The oracle (same fp32 arithmetic as forword.c, Q4_0 added) on one pinned core,
    timed at the decode positions p0, p0+1, ...: KV rows 0..p0-1 are filled first
    (N(0,1)), so every timed forward attends over as many rows as a decode step."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import fw_cpu
    model, ncpu = host_cpu()
    keep = os.sched_getaffinity(0)
    core = min(keep)
    os.sched_setaffinity(0, {core})
    try:
        fw_cpu.set_threads(1)
        om = fw_cpu.OracleModel(host)
        c = host.cfg
        kvd = c.n_head_kv * c.head_dim
        rng = np.random.default_rng(11)
        k = rng.standard_normal((p0, kvd), dtype=np.float32)
        v = rng.standard_normal((p0, kvd), dtype=np.float32)
        for layer in range(c.n_layer):
            om.set_kv(layer, 0, k, v)
        done, t0 = 0, time.perf_counter()
        while True:
            om.forward(3 + done, p0 + done)
            done += 1
            el = time.perf_counter() - t0
            log(f"cpu baseline: {done} forwards at positions {p0}.. in {el:.1f}s")
            if el + el / done > budget_s or done >= 64:
                break
        om.close()
    finally:
        os.sched_setaffinity(0, keep)
    return done / el, done, el, model, ncpu, core


def copy_gbs(hip, mb=1024, reps=8):
    """Device-to-device copy rate (bytes read + written per second) of an mb MiB
    buffer: the practical ceiling of a pure streaming kernel on this GPU."""
    n = mb << 20
    a, b = fwgpu.DeviceBuffer(n), fwgpu.DeviceBuffer(n)
    assert hip.L.hipMemcpyAsync(b.ptr, a.ptr, n, 3, None) == 0
    hip.sync(None)
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, None)
    for _ in range(reps):
        assert hip.L.hipMemcpyAsync(b.ptr, a.ptr, n, 3, None) == 0
    hip.record(e1, None)
    hip.sync(None)
    ms = hip.ms(e0, e1)
    a.free()
    b.free()
    return 2.0 * n * reps / (ms / 1e3) / 1e9


def copy_calibration(hip, mb):
    """Device-to-device copies of a known size, for memory-counter calibration."""
    n = mb << 20
    a, b = fwgpu.DeviceBuffer(n), fwgpu.DeviceBuffer(n)
    for _ in range(3):
        assert hip.L.hipMemcpyAsync(b.ptr, a.ptr, n, 3, None) == 0
    hip.sync(None)
    print(json.dumps({"copy_bytes": n, "copies": 3}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--config", default="8b", choices=["8b", "8b-k", "8b-km", "lc", "70b", "qwen2-7b", "phi2", "gpt2-xl", "tiny"])
    ap.add_argument("--mode", default="full", choices=["full", "decode", "copy", "micro"])
    ap.add_argument("--copy-mb", type=int, default=1024)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-microbench", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this decode path runs on one GPU; --gpus {args.gpus} is not supported "
              "(the path is built for one GPU; sharding across GPUs is a design, not code)", file=sys.stderr)
        sys.exit(2)
    hip = Hip()
    if args.mode == "copy":
        copy_calibration(hip, args.copy_mb)
        return
    if args.mode == "micro":
        print(json.dumps({"microbench": microbench(hip)}), flush=True)
        return

    lc = args.config == "lc"
    lc_pos = 32768
    n_ctx = (lc_pos if lc else args.prompt) + args.warmup + args.steps + 1
    if args.config in ("8b", "lc"):
        sp = fwgpu.spec_8b(n_ctx=max(768, n_ctx))
        workload = ("Llama-3-8B-shape Q4_0 greedy decode at 32K context (Q8_0 embedding/output)" if lc else
                    "Llama-3-8B-shape Q4_0 greedy decode (Q8_0 embedding/output)")
    elif args.config == "8b-k":
        sp = fwgpu.spec_8b(n_ctx=max(768, n_ctx), linear_type=fwgpu.GGML_Q4_K, embd_type=fwgpu.GGML_Q4_K,
                           output_type=fwgpu.GGML_Q6_K)
        workload = "Llama-3-8B-shape Q4_K greedy decode (Q4_K embedding, Q6_K output)"
    elif args.config == "8b-km":
        sp = fwgpu.spec_8b(n_ctx=max(768, n_ctx), linear_type=fwgpu.GGML_Q4_K, embd_type=fwgpu.GGML_Q4_K,
                           output_type=fwgpu.GGML_Q6_K, mix_type=fwgpu.GGML_Q6_K)
        workload = ("Llama-3-8B-shape Q4_K_M-layout greedy decode (Q4_K linears, attn_v and ffn_down Q6_K "
                    "in even layers, Q4_K embedding, Q6_K output)")
    elif args.config == "70b":
        sp = fwgpu.spec_70b(n_ctx=max(384, n_ctx))
        workload = "Llama-3-70B-shape Q4_0 greedy decode (Q8_0 embedding/output)"
    elif args.config == "qwen2-7b":
        sp = fwgpu.spec_qwen2_7b(n_ctx=max(768, n_ctx))
        workload = "Qwen2-7B-shape Q4_0 greedy decode (q/k/v biases, GQA group 7; Q8_0 embedding/output)"
    elif args.config == "gpt2-xl":
        sp = fwgpu.spec_gpt2_xl(n_ctx=max(768, n_ctx))
        workload = "GPT-2-XL-shape Q8_0 greedy decode (learned positions, fused QKV, LayerNorm, no RoPE)"
    elif args.config == "phi2":
        sp = fwgpu.spec_phi2(n_ctx=max(768, n_ctx))
        workload = "Phi-2-shape Q4_0 greedy decode (LayerNorm, parallel residual, NEOX RoPE, hd 80)"
    else:
        sp = fwgpu.spec_tiny()
        sp.n_ctx = max(sp.n_ctx, n_ctx)
        workload = "tiny llama Q8_0 greedy decode"
    t0 = time.perf_counter()
    host = fwgpu.HostModel(synth=sp, max_ctx=n_ctx)
    log(f"model generated in {time.perf_counter() - t0:.1f}s ({host.data_size / 1e9:.2f} GB of tensors)")
    t0 = time.perf_counter()
    gm = fwgpu.GpuModel(host)
    gm_persistent = gm.persistent
    step_impl = "persistent kernel" if gm_persistent else "per-phase kernels (hipGraph)"
    log(f"uploaded to HBM in {time.perf_counter() - t0:.1f}s; token step: {step_impl}")
    cfg = host.cfg

    first, prefill_s, prefill_b_s, first_b = None, None, None, None
    if lc:
        # KV rows 0..lc_pos-1 of every layer from N(0,1), written through kv_write
        kvd = cfg.n_head_kv * cfg.head_dim
        rng = np.random.default_rng(4)
        t0 = time.perf_counter()
        chunk = 4096
        kbuf = rng.standard_normal((chunk, kvd), dtype=np.float32)
        vbuf = rng.standard_normal((chunk, kvd), dtype=np.float32)
        for layer in range(cfg.n_layer):
            for c0 in range(0, lc_pos, chunk):
                sh = (layer * 131 + c0) % chunk
                gm.kv_write(layer, c0, np.roll(kbuf, sh, axis=0), np.roll(vbuf, sh, axis=0))
        log(f"KV rows 0..{lc_pos - 1} of {cfg.n_layer} layers written in {time.perf_counter() - t0:.1f}s")
        gm.decode_from(7, lc_pos, args.warmup)
        p0 = lc_pos + args.warmup
    else:
        prompt = np.random.default_rng(512).integers(3, cfg.n_vocab, args.prompt).astype(np.uint32)
        # batched prefill of the same prompt (one pass per layer, matrix-core GEMMs);
        # the token-by-token prefill below rewrites the same KV rows
        gm.prefill_argmax(prompt)                                     # first call: scratch, code objects
        t0 = time.perf_counter()
        first_b = gm.prefill_argmax(prompt)
        prefill_b_s = time.perf_counter() - t0
        flops = 2.0 * args.prompt * sum(int(r) * int(c) for r, c in linear_shapes(cfg))
        log(f"batched prefill {args.prompt} tokens in {prefill_b_s * 1e3:.1f} ms -> "
            f"{args.prompt / prefill_b_s:.0f} tok/s, linears {flops / prefill_b_s / 1e12:.1f} TFLOP/s (fp32)")
        t0 = time.perf_counter()
        first = gm.generate_greedy(prompt, 1)
        prefill_s = time.perf_counter() - t0
        log(f"prefill {args.prompt} tokens (token-by-token, as the reference) in {prefill_s:.2f}s")
        gm.decode(args.warmup)
        p0 = args.prompt + args.warmup
    hip.sync(gm.stream)

    total_ms, launches = timed_decode(hip, gm, args.steps)
    gm.status()                     # raises if a launch gave up at a bounded wait: no number from it
    tok_s = args.steps / (total_ms / 1e3)
    bb = {"8b-k": dict(linear_bb=18, embd_bb=18, out_bb=26.25),                      # per 32 values
          "8b-km": dict(linear_bb=18, embd_bb=18, out_bb=26.25, mix_bb=26.25),
          "gpt2-xl": dict(linear_bb=34)}.get(args.config, {})
    byte_list = [step_bytes(cfg, p, **bb) for p in range(p0, p0 + args.steps)]
    avg_bytes = float(np.mean(byte_list))
    log(f"decode: {args.steps} steps at positions {p0}..{p0 + args.steps - 1} in {total_ms:.2f} ms "
        f"-> {tok_s:.1f} tok/s, {avg_bytes * tok_s / 1e9:.0f} GB/s effective")
    if args.mode == "decode":
        gm.close()                  # handle, stream and pinned buffers released before the process exits
        host.close()
        print(json.dumps({"tok_s": round(tok_s, 2), "steps": args.steps, "ms": round(total_ms, 3)}), flush=True)
        return
    if gm.persistent and os.environ.get("FORWORD_GPU_PHASE_TIMES") == "1":
        pt, L = gm.phase_times(), cfg.n_layer
        names = ["qkv", "attn", "wo", "ffn", "down"]
        per = {nm: float(np.mean(pt[i:5 * L:5])) for i, nm in enumerate(names)}
        log("phase us (mean over layers, last launch): " + ", ".join(f"{k} {v:.2f}" for k, v in per.items())
            + f", head {pt[-1]:.2f}; step {pt.sum():.1f}")

    # roofline of the dominant kernel: the full-size launches of the timed decode
    n_l = max(n for _, n in launches)
    i0, per_bytes, per_ms = 0, [], []
    for ms, n in launches:
        if n == n_l:
            per_bytes.append(sum(byte_list[i0:i0 + n]))
            per_ms.append(ms)
        i0 += n
    launch_bytes = float(np.mean(per_bytes))
    launch_ms = float(np.mean(per_ms))
    achieved = launch_bytes / (launch_ms / 1e3) / 1e9
    log(f"persistent launch: {n_l} steps, {launch_bytes / 1e9:.2f} GB, {launch_ms:.2f} ms -> {achieved:.0f} GB/s")

    micro = None
    if not args.no_microbench and args.config == "8b":
        micro = microbench(hip)
    gm.close()
    copy = copy_gbs(hip)
    log(f"device-to-device copy: {copy:.0f} GB/s (read + write)")

    cpu = None
    if not args.no_cpu and args.config == "8b":
        v, n, el, model, ncpu, core = cpu_baseline(host, args.cpu_seconds, p0)
        cpu = {"value": round(v, 4), "unit": "tok/s", "cores": 1, "kind": "port",
               "sample": f"{n} forwards of the same model at decode positions {p0}..{p0 + n - 1} "
                         f"(KV rows 0..{p0 - 1} filled), 1 thread pinned to core {core} of {ncpu} "
                         f"({model}), {el:.1f} s (oracle/fw_cpu.c: forword.c's fp32 order, Q4_0 added)"}
    host.close()

    cfg_out = {"workload": workload, "step_impl": step_impl,
               "decode_positions": [p0, p0 + args.steps - 1], "kv_cache": "fp32 in HBM",
               "step_bytes_avg": int(avg_bytes), "step_gbs": round(avg_bytes * tok_s / 1e9, 1),
               "step_roofline_frac": round(avg_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4)}
    if lc:
        cfg_out["kv_prefill"] = f"rows 0..{lc_pos - 1} N(0,1) via forword_gpu_kv_write"
    else:
        cfg_out["prompt_tokens"] = args.prompt
        cfg_out["prefill_tok_s"] = round(args.prompt / prefill_s, 1)
        cfg_out["prefill_batched_tok_s"] = round(args.prompt / prefill_b_s, 1)
        cfg_out["prefill_batched_same_first_token"] = bool(int(first_b) == int(first[0]))
        cfg_out["first_token"] = int(first[0])
    traffic, traffic_src, traffic_ratio = None, None, None
    tf = os.path.join(ROOT, "profiles", "k_decode_8b_q4_0_traffic.json")
    if args.config == "8b" and gm_persistent and os.path.exists(tf):
        # HBM bytes per step from the committed FETCH_SIZE / WRITE_SIZE runs of this
        # workload, scaled to the steps of the launch timed here
        t = json.load(open(tf))
        traffic = int(t["traffic_bytes_per_step"] * n_l)
        traffic_ratio = round(t["traffic_bytes_per_step"] / t["algorithmic_bytes_per_step"], 4)
        traffic_src = t["source"]
    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(total_ms / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded random-init GGUF, random prompt ids)",
        "config": cfg_out,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_vs_algorithmic": traffic_ratio, "traffic_source": traffic_src,
                     "copy_gbs": round(copy, 1), "frac_of_copy": round(achieved / copy, 4),
                     "kernel": (f"k_decode (persistent token step, {n_l} steps per launch)" if gm_persistent
                                else f"per-phase step kernels replayed from a hipGraph, {n_l} steps per timing"),
                     "bytes_per_launch": int(launch_bytes), "avg_ms_per_launch": round(launch_ms, 3)},
        "microbench": micro,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
