#!/usr/bin/env python3
"""Decode benchmark of the forword MI355X path: Llama-3-8B-shaped random-init
Q4_0 GGUF (Q8_0 embedding/output), 512-token random prompt, then greedy decode
at positions 512..767.  One step = one token forward (transformer_forward) plus
the greedy pick, run device-resident through the C ABI.

Prints one JSON line:
  value        decode tok/s (weights and KV already in HBM)
  roofline     the dominant kernel (fused gate/up Q4_0 GEMV + SiLU*up, 54% of each
               layer's weight bytes) timed with HIP events over >= 1 GiB of
               rotating weight copies; achieved = algorithmic bytes / duration
  cpu_baseline the oracle (CPU restatement of forword.c) on one core, bounded sample
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


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Hip:
    """The few HIP runtime calls the timing needs (events on a given stream)."""

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
        fwgpu._sig(L, "hipEventDestroy", C.c_int, [C.c_void_p])
        fwgpu._sig(L, "hipStreamSynchronize", C.c_int, [C.c_void_p])

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


def step_bytes(cfg, pos, linear_bb=18, embd_bb=34, out_bb=34):
    """Algorithmic bytes of one token step at position pos: weights, embedding row,
    norm weights, KV read (rows 0..pos incl. the one just written) and KV write."""
    n, ff, L, hd, kv = cfg.n_embd, cfg.n_ff, cfg.n_layer, cfg.head_dim, cfg.n_head_kv
    lin = L * ((n // 32) * linear_bb * (2 * n + 2 * kv * hd + 2 * ff) + (ff // 32) * linear_bb * n)
    head = (n // 32) * out_bb * cfg.n_vocab
    embd = (n // 32) * embd_bb
    norms = 4 * n * (2 * L + 1)
    kvb = L * 2 * kv * hd * 4 * (pos + 1) + L * 2 * kv * hd * 4
    return lin + head + embd + norms + kvb


def time_dominant_kernel(hip, stream, n_in, n_ff, reps_min=64):
    """Fused gate/up Q4_0 GEMV at the layer shape, cycling through >= 1 GiB of
    distinct weight copies so the 256 MB last-level cache cannot serve repeats."""
    per = fwgpu.BLOCK_BYTES[fwgpu.GGML_Q4_0] * (n_in // 32) * n_ff
    copies = max(2, -(-(1 << 30) // (2 * per)))
    w = fwgpu.synth_matrix(fwgpu.GGML_Q4_0, n_ff, n_in, seed=123)
    bufs = [(fwgpu.DeviceBuffer.from_array(w), fwgpu.DeviceBuffer.from_array(w)) for _ in range(copies)]
    x = fwgpu.DeviceBuffer.from_array(fwgpu.randn(7, n_in))
    h = fwgpu.DeviceBuffer(n_ff * 4)
    reps = max(reps_min, 2 * copies)
    for i in range(copies):                                  # warm-up pass
        fwgpu.ops.ffn_swiglu(bufs[i][0], bufs[i][1], fwgpu.GGML_Q4_0, x, h, n_in, n_ff, stream, sync=False)
    hip.sync(stream)
    ev = [hip.event() for _ in range(reps + 1)]
    for i in range(reps):
        hip.record(ev[i], stream)
        g, u = bufs[i % copies]
        fwgpu.ops.ffn_swiglu(g, u, fwgpu.GGML_Q4_0, x, h, n_in, n_ff, stream, sync=False)
    hip.record(ev[reps], stream)
    hip.sync(stream)
    per_launch = [hip.ms(ev[i], ev[i + 1]) for i in range(reps)]
    total = hip.ms(ev[0], ev[reps])
    for b in bufs:
        b[0].free()
        b[1].free()
    algo = 2 * per + 4 * n_in + 4 * n_ff
    return algo, float(np.mean(per_launch)), total / reps, copies


def cpu_baseline(host, budget_s):
    """The oracle (same fp32 arithmetic as forword.c, Q4_0 added) on one core."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import fw_cpu
    fw_cpu.set_threads(1)
    om = fw_cpu.OracleModel(host)
    done, t0 = 0, time.perf_counter()
    while True:
        om.forward(3 + done, done)
        done += 1
        el = time.perf_counter() - t0
        log(f"cpu baseline: {done} forwards in {el:.1f}s")
        if el + el / done > budget_s or done >= 64:
            break
    om.close()
    return done / el, done, el


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--config", default="8b", choices=["8b", "70b", "tiny"])
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this decode path runs on one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is design-only, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    n_ctx = args.prompt + args.warmup + args.steps + 1
    if args.config == "8b":
        sp = fwgpu.spec_8b(n_ctx=max(768, n_ctx))
        workload = "Llama-3-8B-shape Q4_0 greedy decode (Q8_0 embedding/output)"
    elif args.config == "70b":
        sp = fwgpu.spec_70b(n_ctx=max(384, n_ctx))
        workload = "Llama-3-70B-shape Q4_0 greedy decode (Q8_0 embedding/output)"
    else:
        sp = fwgpu.spec_tiny()
        sp.n_ctx = max(sp.n_ctx, n_ctx)
        workload = "tiny llama Q8_0 greedy decode"
    t0 = time.perf_counter()
    host = fwgpu.HostModel(synth=sp, max_ctx=n_ctx)
    log(f"model generated in {time.perf_counter() - t0:.1f}s ({host.data_size / 1e9:.2f} GB of tensors)")
    hip = Hip()
    t0 = time.perf_counter()
    gm = fwgpu.GpuModel(host)
    step_impl = "persistent kernel" if gm.persistent else "per-phase kernels (hipGraph)"
    log(f"uploaded to HBM in {time.perf_counter() - t0:.1f}s; token step: {step_impl}")
    stream = gm.stream
    prompt = np.random.default_rng(512).integers(3, host.cfg.n_vocab, args.prompt).astype(np.uint32)

    t0 = time.perf_counter()
    first = gm.generate_greedy(prompt, 1)
    prefill_s = time.perf_counter() - t0
    log(f"prefill {args.prompt} tokens (token-by-token, as the reference) in {prefill_s:.2f}s")
    gm.decode(args.warmup)
    hip.sync(stream)
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, stream)
    gm.decode(args.steps, copy_out=False)
    hip.record(e1, stream)
    hip.sync(stream)
    ms = hip.ms(e0, e1)
    tok_s = args.steps / (ms / 1e3)
    p0 = args.prompt + args.warmup
    avg_bytes = float(np.mean([step_bytes(host.cfg, p) for p in range(p0, p0 + args.steps)]))
    log(f"decode: {args.steps} steps in {ms:.2f} ms -> {tok_s:.1f} tok/s, "
        f"{avg_bytes * tok_s / 1e9:.0f} GB/s effective")
    if gm.persistent and os.environ.get("FORWORD_GPU_PHASE_TIMES") == "1":
        pt, L = gm.phase_times(), host.cfg.n_layer
        names = ["qkv", "attn", "wo", "ffn", "down"]
        per = {nm: float(np.mean(pt[i:5 * L:5])) for i, nm in enumerate(names)}
        log("phase us (mean over layers, last launch): " + ", ".join(f"{k} {v:.2f}" for k, v in per.items())
            + f", head {pt[-1]:.2f}; step {pt.sum():.1f}")

    algo, dur_ms, dur_ms_total, copies = time_dominant_kernel(hip, stream, host.cfg.n_embd, host.cfg.n_ff)
    achieved = algo / (dur_ms / 1e3) / 1e9
    log(f"dominant kernel: {algo} B per launch, {dur_ms * 1e3:.2f} us avg -> {achieved:.0f} GB/s")
    gm.close()

    cpu = None
    if not args.no_cpu:
        v, n, el = cpu_baseline(host, args.cpu_seconds)
        cpu = {"value": round(v, 4), "unit": "tok/s", "cores": 1, "kind": "port",
               "sample": f"{n} forwards of the same model at positions 0..{n - 1}, 1 thread, "
                         f"{el:.1f} s (oracle/fw_cpu.c: forword.c's fp32 order, Q4_0 added)"}
    host.close()

    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded random-init GGUF, random prompt ids)",
        "config": {"workload": workload, "prompt_tokens": args.prompt, "step_impl": step_impl,
                   "decode_positions": [p0, p0 + args.steps - 1], "kv_cache": "fp32 in HBM",
                   "step_bytes_avg": int(avg_bytes), "step_gbs": round(avg_bytes * tok_s / 1e9, 1),
                   "step_roofline_frac": round(avg_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4),
                   "prefill_tok_s": round(args.prompt / prefill_s, 1), "first_token": int(first[0])},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "k_qmv<Q4_0, SWIGLU> (fused gate/up GEMV + SiLU*up), "
                               f"{host.cfg.n_ff}x{host.cfg.n_embd} x2, {copies} rotating copies",
                     "bytes_per_launch": algo, "avg_us": round(dur_ms * 1e3, 3),
                     "avg_us_back_to_back": round(dur_ms_total * 1e3, 3)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
