"""Benchmark of the denoiser step on one MI355X.

Default workload: Flux.2-Klein-4B-shaped denoiser (5 double + 20 single
blocks, hidden 3072, 24 heads x 128, SwiGLU x3), 1024x1024 image = 64x64
latent tokens of 128 channels (4096 image tokens) + 512 text tokens of 7680
dims, 4-step official schedule, batch 1, random-init bf16 weights, synthetic
inputs. A step = one transformer forward + the Euler update, with latent, text
and weights resident in HBM (captured hipGraph replay + update kernel).

Prints one JSON line (see the fields below). `value` is images/s (4 steps per
image); ms_per_step is per denoise step. `roofline` is the dominant kernel (the
single-block fused QKV+SwiGLU GEMM, 20 launches per step) timed with HIP
events; `cpu_baseline` times the oracle (C restatement of the reference's
`make blas` path, OpenBLAS) on one double and one single block at the same
shape, extrapolated to a step.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import iris_testlib as tl  # noqa: E402

PEAK_BF16 = 2.5e15          # MI355X dense bf16 MFMA, FLOP/s
PEAK_HBM = 8.0e12           # B/s

CONFIGS = {
    # name: hidden, heads, n_double, n_single, text_dim, latent h, w, txt, steps, refs, batch
    "ns": dict(h=3072, H=24, nd=5, ns=20, td=7680, ih=64, iw=64, T=512, steps=4, refs=[], B=1,
               workload="Flux.2-Klein-4B-shaped denoise, 1024x1024 (4096 img + 512 txt tokens), 4 steps"),
    "c2": dict(h=3072, H=24, nd=5, ns=20, td=7680, ih=32, iw=32, T=512, steps=4, refs=[], B=1,
               workload="Flux.2-Klein-4B-shaped denoise, 512x512 (1024 img + 512 txt tokens), 4 steps"),
    "c3": dict(h=3072, H=24, nd=5, ns=20, td=7680, ih=64, iw=64, T=512, steps=4, refs=[(64, 64, 1), (64, 64, 2)],
               B=1, workload="Flux.2-Klein-4B-shaped, 1024x1024 + 2 references (T offsets 1, 2), 12800 tokens"),
    "c4": dict(h=4096, H=32, nd=8, ns=24, td=12288, ih=64, iw=64, T=512, steps=50, refs=[], B=2,
               workload="Flux.2-Klein-9B-base-shaped, 1024x1024, CFG 4.0 as batch 2, 50-step schedule"),
}


def step_flops(c):
    """Algorithmic FLOP per step: 2MNK per linear, attention 4 S^2 h (QK^T + PV)."""
    h, mlp, T = c["h"], 3 * c["h"], c["T"]
    I0 = c["ih"] * c["iw"]
    I = I0 + sum(a * b for a, b, _ in c["refs"])
    S = I + T
    blk = 2 * S * h * (3 * h + h + 2 * mlp + mlp) + 4 * S * S * h
    f = (c["nd"] + c["ns"]) * blk
    f += 2 * I * 128 * h + 2 * T * c["td"] * h + 2 * I0 * h * 128
    f *= c["B"]
    attn = (c["nd"] + c["ns"]) * 4 * S * S * h * c["B"]
    return f, attn


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=12)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="ns", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is design-only, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    c = CONFIGS[args.config]
    lib = tl.hip()
    t0 = time.time()
    tf = ctypes.c_void_p(lib.iris_transformer_create_synthetic(c["h"], c["H"], c["nd"], c["ns"], c["td"], 128, 3.0,
                                                               2000.0, 20250101))
    assert tf, lib.iris_hip_last_error().decode()
    t_load = time.time() - t0
    I0 = c["ih"] * c["iw"]
    lib.iris_init_noise.argtypes = [ctypes.c_int] * 4 + [ctypes.c_int64]
    zp = lib.iris_init_noise(1, 128, c["ih"], c["iw"], 42)
    z = np.ctypeslib.as_array(ctypes.cast(zp, tl.FP), shape=(128 * I0,)).copy()
    txt = tl.synth_f32((c["B"], c["T"], c["td"]), 7)
    refs_np = [tl.synth_f32((128, rh, rw), 100 + i) for i, (rh, rw, _) in enumerate(c["refs"])]
    refs = (tl.IrisRef * max(1, len(refs_np)))(*[tl.IrisRef(tl.fptr(r), rh, rw, to) for r, (rh, rw, to)
                                                 in zip(refs_np, c["refs"])])
    nref = len(refs_np)
    assert lib.iris_flux_prepare(tf, c["ih"], c["iw"], refs if nref else None, nref, c["T"], c["B"]) == 0
    assert lib.iris_flux_upload(tf, tl.fptr(z), refs if nref else None, tl.fptr(txt)) == 0
    lib.iris_official_schedule.argtypes = [ctypes.c_int, ctypes.c_int]
    sp = lib.iris_official_schedule(c["steps"], I0)
    sched = np.ctypeslib.as_array(ctypes.cast(sp, tl.FP), shape=(c["steps"] + 1,)).copy()
    g = 4.0 if c["B"] == 2 else 0.0

    def step(i):
        j = i % c["steps"]
        assert lib.iris_flux_step(tf, float(sched[j]), float(sched[j + 1]), g) == 0, lib.iris_hip_last_error()

    for i in range(args.warmup):
        step(i)
    assert lib.iris_hip_sync() == 0
    lib.iris_hip_event_record(0)
    t1 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    lib.iris_hip_event_record(1)
    assert lib.iris_hip_sync() == 0
    wall = time.perf_counter() - t1
    ms_event = lib.iris_hip_event_elapsed_ms(0, 1)
    ms_step = ms_event / args.steps
    flops, attn_flops = step_flops(c)
    images_per_s = 1000.0 / (ms_step * c["steps"]) * c["B"] / c["B"]

    # dominant kernel: the single-block fused projection (QKV -> bf16, gate/up ->
    # SwiGLU), same shapes, buffers and weights as inside the step
    h, mlp = c["h"], 3 * c["h"]
    S = I0 + sum(a * b for a, b, _ in c["refs"]) + c["T"]
    BS = c["B"] * S
    a_buf = lib.iris_flux_device_buffer(tf, b"a")
    qkv_buf = lib.iris_flux_device_buffer(tf, b"qkv")
    cat_buf = lib.iris_flux_device_buffer(tf, b"cat")
    wdev = tl.Dev((3 * h + 2 * mlp) * h * 2)
    wdev.put(tl.to_bf16(tl.synth_f32(((3 * h + 2 * mlp) * h,), 9, 0, 0.02)))
    P = tl.GemmProblem
    probs = (P * 2)(P(a_buf, wdev.ptr, qkv_buf, None, BS, 3 * h, h, h, h, 3 * h, 1),
                    P(a_buf, wdev.ptr + 3 * h * h * 2, cat_buf + h * 2, None, BS, 2 * mlp, h, h, h, h + mlp, 3))
    n_launch = 50
    for _ in range(3):
        lib.iris_hip_gemm(probs, 2)
    lib.iris_hip_event_record(2)
    for _ in range(n_launch):
        lib.iris_hip_gemm(probs, 2)
    lib.iris_hip_event_record(3)
    assert lib.iris_hip_sync() == 0
    k_ms = lib.iris_hip_event_elapsed_ms(2, 3) / n_launch
    k_flops = 2.0 * BS * h * (3 * h + 2 * mlp)
    k_achieved = k_flops / (k_ms * 1e-3)
    # traffic (algorithmic): A read + W read + outputs
    k_bytes = BS * h * 2 + (3 * h + 2 * mlp) * h * 2 + BS * 3 * h * 2 + BS * mlp * 2

    result = {
        "metric": "ms per denoise step + images/s @4B-shape 1024^2; % of bf16 MFMA peak",
        "value": round(images_per_s, 4),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "ms_per_image": round(ms_step * c["steps"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random-init bf16 weights, N(0,1) text embeddings, seeded noise latent)",
        "config": {"workload": c["workload"], "hidden": c["h"], "heads": c["H"], "double_blocks": c["nd"],
                   "single_blocks": c["ns"], "image_tokens": I0, "text_tokens": c["T"], "seq": S,
                   "batch": c["B"], "steps_per_image": c["steps"]},
        "step_tflop": round(flops / 1e12, 3),
        "mfma_frac_step": round(flops / (ms_step * 1e-3) / PEAK_BF16, 4),
        "achieved_tflops_step": round(flops / (ms_step * 1e-3) / 1e12, 1),
        "wall_ms_per_step": round(wall * 1000 / args.steps, 4),
        "model_create_s": round(t_load, 1),
        "roofline": {"kernel": "gemm_bf16_kernel (single-block fused QKV + gate/up with SwiGLU epilogue)",
                     "bound": "mfma", "achieved": round(k_achieved / 1e12, 1), "peak": PEAK_BF16 / 1e12,
                     "unit": "TFLOP/s", "frac": round(k_achieved / PEAK_BF16, 4), "traffic": None,
                     "launch_ms": round(k_ms, 4), "flop_per_launch": k_flops, "algorithmic_bytes": k_bytes},
        "device": lib.iris_hip_device_name().decode(),
    }
    wdev.close()
    lib.iris_transformer_free(tf)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(c)
    print(json.dumps(result))


def cpu_baseline(c):
    """Oracle (C restatement of the reference f32 BLAS path) on the host cores:
    one double and one single block at the benchmark's shape, timed once each,
    extrapolated to one step (n_double x double + n_single x single)."""
    orc = tl.oracle()
    threads = int(os.environ.get("IRIS_ORACLE_THREADS", min(os.cpu_count() or 1, 16)))
    tl.bind_blas(orc, threads)
    h, T, I0 = c["h"], c["T"], c["ih"] * c["iw"]
    I = I0 + sum(a * b for a, b, _ in c["refs"])
    m = ctypes.c_void_p(orc.orc_flux_create_synth(h, c["H"], 1, 1, c["td"], 128, 3.0, 2000.0, 20250101))
    ic, is_ = np.zeros(I * 128, np.float32), np.zeros(I * 128, np.float32)
    orc.orc_rope_img(tl.fptr(ic), tl.fptr(is_), c["ih"], c["iw"], 32, ctypes.c_float(2000.0), 0)
    tc, ts = np.zeros(T * 128, np.float32), np.zeros(T * 128, np.float32)
    orc.orc_rope_txt(tl.fptr(tc), tl.fptr(ts), T, 32, ctypes.c_float(2000.0))
    img, txt = tl.synth_f32((I, h), 1), tl.synth_f32((T, h), 2)
    mi, mt = tl.synth_f32((6 * h,), 3, 0, 0.1), tl.synth_f32((6 * h,), 4, 0, 0.1)
    t0 = time.perf_counter()
    orc.orc_flux_double_block(m, 0, tl.fptr(img), tl.fptr(txt), tl.fptr(mi), tl.fptr(mt), tl.fptr(ic), tl.fptr(is_),
                              tl.fptr(tc), tl.fptr(ts), I, T)
    t_d = time.perf_counter() - t0
    x, temb = tl.synth_f32((T + I, h), 5), tl.synth_f32((h,), 6)
    t0 = time.perf_counter()
    orc.orc_flux_single_block(m, 0, tl.fptr(x), tl.fptr(temb), tl.fptr(ic), tl.fptr(is_), tl.fptr(tc), tl.fptr(ts),
                              T + I, T)
    t_s = time.perf_counter() - t0
    orc.orc_flux_free(m)
    ms_step = (c["nd"] * t_d + c["ns"] * t_s) * 1000 * c["B"]
    return {"value": round(1000.0 / (ms_step * c["steps"]), 6), "unit": "images/s", "cores": threads,
            "kind": "port", "ms_per_step": round(ms_step, 1),
            "sample": f"oracle (C restatement of the reference make-blas path, "
                      f"{orc.orc_blas_info().decode()}): 1 double block {t_d:.2f} s + 1 single block {t_s:.2f} s "
                      f"at S={T + I}, h={h}, extrapolated x{c['nd']} + x{c['ns']} per step"}


if __name__ == "__main__":
    main()
