"""Writes the golden fixtures under tests/golden/ from forword.c's own compiled code.

Runs only where the reference sources exist (the build container): it builds
oracle/_ref/ with oracle/ref.mk, generates the inputs with this repository's
seeded writer (forword.c_amd/host), runs oracle/_ref/ref_driver on them and
stores inputs' SHA-256 plus the reference's outputs.  The tests regenerate the
inputs from the same seeds, check the SHA-256, and compare against the stored
outputs, so the reference itself is never needed at test time.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
GOLD = os.path.join(ROOT, "tests", "golden")
DRIVER = os.path.join(ROOT, "oracle", "_ref", "ref_driver")
sys.path.insert(0, os.path.join(ROOT, "forword.c_amd"))
import fwgpu  # noqa: E402
import golden_specs as gs  # noqa: E402  (tests/golden/golden_specs.py)


def sha(b) -> str:
    return hashlib.sha256(memoryview(b).cast("B")).hexdigest()


def run(args):
    r = subprocess.run([DRIVER] + [str(a) for a in args], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"ref_driver {args[0]} failed rc={r.returncode}: {r.stdout} {r.stderr}")
    return r.stdout


def gen_model(name, tmp, manifest):
    m = gs.MODELS[name]
    sp = m["spec"]()
    path = os.path.join(tmp, f"{name}.gguf")
    if fwgpu.host_lib().fwh_synth_write_file(sp, path.encode()) != 0:
        raise RuntimeError("synth write failed")
    img = open(path, "rb").read()
    prompt = gs.prompt(name)
    ppath = os.path.join(tmp, f"{name}.prompt.u32")
    prompt.tofile(ppath)
    od = os.path.join(tmp, name)
    os.makedirs(od, exist_ok=True)
    n_fwd = prompt.size + m["n_gen"] - 1
    lsteps, tsteps = gs.logit_steps(name), gs.trace_steps(name)
    out = run(["gen", path, m["max_ctx"], ppath, m["n_gen"], od, ",".join(map(str, lsteps)),
               ",".join(map(str, tsteps))])
    arrays = {
        "tokens": np.fromfile(os.path.join(od, "tokens.u32"), np.uint32),
        "stats": np.fromfile(os.path.join(od, "stats.f64"), np.float64).reshape(n_fwd, 5),
    }
    for f in lsteps:
        arrays[f"logits_{f}"] = np.fromfile(os.path.join(od, f"logits_{f}.f32"), np.float32)
    for f in tsteps:
        arrays[f"trace_{f}"] = np.fromfile(os.path.join(od, f"trace_{f}.f32"), np.float32)
    np.savez_compressed(os.path.join(GOLD, f"model_{name}.npz"), **arrays)
    manifest["models"][name] = {"gguf_sha256": sha(img), "gguf_bytes": len(img), "driver": out.strip(),
                                "prompt": prompt.tolist(), "n_gen": m["n_gen"], "max_ctx": m["max_ctx"]}


def gen_matvec(tmp, manifest):
    arrays = {}
    for (t, rows, cols) in gs.MATVEC_CASES:
        w = gs.matvec_weights(t, rows, cols)
        x = gs.matvec_x(t, rows, cols)
        wp, xp, yp = (os.path.join(tmp, f) for f in ("w.bin", "x.bin", "y.bin"))
        w.tofile(wp)
        x.tofile(xp)
        run(["qmv", t, cols, rows, wp, xp, yp])
        key = gs.matvec_key(t, rows, cols)
        arrays[key] = np.fromfile(yp, np.float32)
        manifest["matvec"][key] = {"w_sha256": sha(w), "x_sha256": sha(x)}
    np.savez_compressed(os.path.join(GOLD, "matvec.npz"), **arrays)


def gen_dequant(tmp, manifest):
    arrays = {}
    for t in (fwgpu.GGML_Q8_0, fwgpu.GGML_Q5_0):
        blocks = gs.dequant_blocks(t)
        bp, op = os.path.join(tmp, "b.bin"), os.path.join(tmp, "o.bin")
        blocks.tofile(bp)
        n = blocks.size // fwgpu.BLOCK_BYTES[t]
        run(["getrow", t, 32, n, bp, op])
        arrays[f"getrow_{t}"] = np.fromfile(op, np.float32)
        arrays[f"blocks_{t}"] = blocks
        if t == fwgpu.GGML_Q8_0:
            run(["q8dec", blocks.size, bp, op])
            arrays["q8dec"] = np.fromfile(op, np.float32)
    np.savez_compressed(os.path.join(GOLD, "dequant.npz"), **arrays)


def gen_kquant(tmp, manifest):
    arrays = {}
    for t in gs.KQ_TYPES:
        blocks = gs.kquant_blocks(t)
        bp, op = os.path.join(tmp, "b.bin"), os.path.join(tmp, "o.bin")
        blocks.tofile(bp)
        n = blocks.size // fwgpu.BLOCK_BYTES[t]
        run(["getrow", t, 256, n, bp, op])
        arrays[f"getrow_{t}"] = np.fromfile(op, np.float32)
        arrays[f"blocks_{t}"] = blocks
    manifest["kquant"] = {}
    for (t, rows, cols) in gs.KQ_MATVEC_CASES:
        w = gs.matvec_weights(t, rows, cols)
        x = gs.matvec_x(t, rows, cols)
        wp, xp, yp = (os.path.join(tmp, f) for f in ("w.bin", "x.bin", "y.bin"))
        w.tofile(wp)
        x.tofile(xp)
        run(["qmv", t, cols, rows, wp, xp, yp])
        key = gs.matvec_key(t, rows, cols)
        arrays[key] = np.fromfile(yp, np.float32)
        manifest["kquant"][key] = {"w_sha256": sha(w), "x_sha256": sha(x)}
    np.savez_compressed(os.path.join(GOLD, "kquant.npz"), **arrays)


def gen_sampler(tmp, manifest):
    arrays = {}
    for name, lg, hist in gs.sample_cases():
        arrays[f"logits_{name}"] = lg
        arrays[f"hist_{name}"] = hist
        res = []
        for (temp, top_p, pen) in gs.SAMPLE_SETTINGS:
            for seed in gs.SAMPLE_SEEDS:
                lp, hp, op = (os.path.join(tmp, f) for f in ("l.bin", "h.bin", "o.bin"))
                lg.tofile(lp)
                hist.tofile(hp)
                run(["sample", lg.size, repr(temp), repr(top_p), repr(pen), seed, hist.size, lp, hp, op])
                raw = np.fromfile(op, np.uint8)
                res.append((int(raw[:4].view(np.uint32)[0]), int(raw[4:12].view(np.uint64)[0])))
        arrays[f"tok_{name}"] = np.array([r[0] for r in res], np.uint32)
        arrays[f"rng_{name}"] = np.array([r[1] for r in res], np.uint64)
    np.savez_compressed(os.path.join(GOLD, "sampler.npz"), **arrays)


def gen_ops(tmp, manifest):
    arrays = {}
    p = lambda f: os.path.join(tmp, f)  # noqa: E731
    for n in gs.NORM_SIZES:
        x, w = gs.norm_inputs(n)
        x.tofile(p("x"))
        w.tofile(p("w"))
        run(["rmsnorm", n, repr(gs.NORM_EPS), p("x"), p("w"), p("o")])
        arrays[f"rmsnorm_{n}"] = np.fromfile(p("o"), np.float32)
    for (nctx, hd, base) in gs.ROPE_TABLES:
        run(["ropetab", nctx, hd, repr(base), p("o")])
        arrays[f"ropetab_{nctx}_{hd}_{int(base)}"] = np.fromfile(p("o"), np.float32)
    for (pos, nh, hd, nctx, base, neox) in gs.ROPE_CASES:
        qk = gs.rope_input(nh, hd)
        qk.tofile(p("qk"))
        run(["rope", pos, nh, hd, nctx, repr(base), neox, p("qk"), p("o")])
        arrays[f"rope_{pos}_{nh}_{hd}_{int(base)}_{neox}"] = np.fromfile(p("o"), np.float32)
    x = gs.silu_input()
    x.tofile(p("x"))
    run(["silu", x.size, p("x"), p("o")])
    arrays["silu"] = np.fromfile(p("o"), np.float32)
    dots = []
    for n in gs.DOT_SIZES:
        a, b = gs.dot_inputs(n)
        a.tofile(p("a"))
        b.tofile(p("b"))
        run(["dot", n, p("a"), p("b"), p("o")])
        dots.append(np.fromfile(p("o"), np.float32)[0])
    arrays["dot"] = np.array(dots, np.float32)
    am = []
    for case in gs.argmax_cases():
        case.tofile(p("x"))
        run(["argmax", case.size, p("x"), p("o")])
        am.append(np.fromfile(p("o"), np.uint32)[0])
    arrays["argmax"] = np.array(am, np.uint32)
    np.savez_compressed(os.path.join(GOLD, "ops.npz"), **arrays)


def main():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "-f", "ref.mk"], check=True)
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "forword.c_amd"), "host"], check=True)
    only = sys.argv[2] if len(sys.argv) > 2 and sys.argv[1] == "--only" else None
    if only:                                   # regenerate one fixture file, keep the others
        with open(os.path.join(GOLD, "manifest.json")) as f:
            manifest = json.load(f)
        with tempfile.TemporaryDirectory() as tmp:
            if only.startswith("model:"):      # --only model:<name>
                gen_model(only[6:], tmp, manifest)
            else:
                {"kquant": gen_kquant, "sampler": gen_sampler, "matvec": gen_matvec, "dequant": gen_dequant,
                 "ops": gen_ops}[only](tmp, manifest)
        with open(os.path.join(GOLD, "manifest.json"), "w") as f:
            json.dump(manifest, f, indent=1, sort_keys=True)
        print("fixture", only, "written to", GOLD)
        return
    manifest = {"generator": "tests/golden/make_golden.py", "reference_build": "oracle/ref.mk",
                "models": {}, "matvec": {}}
    with tempfile.TemporaryDirectory() as tmp:
        for name in gs.MODELS:
            gen_model(name, tmp, manifest)
        gen_matvec(tmp, manifest)
        gen_dequant(tmp, manifest)
        gen_kquant(tmp, manifest)
        gen_sampler(tmp, manifest)
        gen_ops(tmp, manifest)
    with open(os.path.join(GOLD, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print("fixtures written to", GOLD)


if __name__ == "__main__":
    main()
