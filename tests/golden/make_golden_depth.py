"""Writes the full-size oracle goldens of tests/test_gpu_depth.py.

The oracle (oracle/liboracle.so, the C restatement of the reference's f32
`make blas` path, pinned to the reference build at small sizes and on a
4B-shaped block by tests/test_oracle.py) runs here on OpenBLAS; the
reference's own generic build multiplies with single-threaded loop nests and
would take hours at these sizes. Every input is a pure function of seeds:
weights from iris_synth (include/iris_synth.h), noise from the reference's
iris_init_noise (the oracle reproduces it bit for bit), schedules from the
reference build (reference_small.npz), text / caption rows iris_synth f32
N(0, 1).

Targets (python tests/golden/make_golden_depth.py [c2|ns|c3|zimage] ...):

  c2      oracle_4b_c2_sample.npz: Flux.2-Klein-4B-shaped denoiser at full
          depth (5 double + 20 single blocks, hidden 3072, 24 heads, text
          7680), 512x512 (32x32 latent = 1024 image + 512 text tokens),
          iris_official_schedule(4, 1024), noise seed 42, model seed 4242,
          text seed 4243. About 2-7 minutes on 8 cores.
  ns      oracle_4b_ns_sample.npz: the same denoiser at 1024x1024 (64x64
          latent = 4096 image + 512 text tokens), iris_official_schedule(4,
          4096), noise seed 42, model seed 20250101, text seed 7 -- the
          inputs the benchmark's default workload uses. About 10 minutes.
  c3      oracle_4b_c3_refs.npz: one forward of the 4B-width denoiser with
          1 double + 2 single blocks, a 64x64 target and two 64x64 reference
          latents at T offsets 1 and 2 (12800 joint tokens), t = 0.85, model
          seed 77; plus the same forward without the references. About 2
          minutes; needs about 20 GB of host memory (the BLAS path
          materialises every head's 12800 x 12800 scores).
  zimage  oracle_zimage_turbo_sample.npz: the Z-Image-Turbo-6B-shaped S3-DiT
          at full depth (2 noise refiners, 2 context refiners, 30 layers,
          dim 3840, 30 heads, FFN 10240, caption 2560), 1024x1024 (16x128x128
          latent = 4096 image patches + 512 caption tokens), the reference's
          8-step iris_zimage_schedule(8, 4096), noise iris_init_noise(1, 16,
          128, 128, 42), model seed 20250101, caption seed 7 -- the
          benchmark's Z-Image workload. About 15 minutes; about 30 GB of
          host memory (f32 weights).

Sample goldens store the velocity of every step on the oracle's trajectory
(Flux: z_{i+1} = z_i + (t_{i+1} - t_i) v_i, iris_sample.c:359; Z-Image:
z_{i+1} = z_i + (s_{i+1} - s_i) (-v_i) at timestep 1 - s_i,
iris_sample.c:449-470, both in float32) and the SHA-256 of the final latent,
which the test recomputes from those velocities.
"""
import ctypes
import hashlib
import os
import sys
import time

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import iris_testlib as tl  # noqa: E402

FLUX_4B = {"hidden": 3072, "heads": 24, "n_double": 5, "n_single": 20, "text_dim": 7680, "text_tokens": 512}
TARGETS = {
    "c2": dict(FLUX_4B, latent=[128, 32, 32], sched="sched_official_4_1024", model_seed=4242, noise_seed=42,
               text_seed=4243, out="oracle_4b_c2_sample.npz"),
    "ns": dict(FLUX_4B, latent=[128, 64, 64], sched="sched_official_4_4096", model_seed=20250101, noise_seed=42,
               text_seed=7, out="oracle_4b_ns_sample.npz"),
    "c3": dict(FLUX_4B, n_double=1, n_single=2, latent=[128, 64, 64], refs=[(64, 64, 1, 173), (64, 64, 2, 174)],
               t=0.85, model_seed=77, latent_seed=171, text_seed=172, out="oracle_4b_c3_refs.npz"),
    "zimage": dict(dim=3840, heads=30, layers=30, refiners=2, cap_dim=2560, in_ch=16, ps=2, theta=256.0,
                   axes=[32, 48, 48], ffn=10240, t_mid=1024, latent=[16, 128, 128], cap_len=512,
                   sched="sched_zimage_8", model_seed=20250101, noise_seed=42, cap_seed=7,
                   out="oracle_zimage_turbo_sample.npz"),
}


def sha256(a):
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()


def schedule(name):
    G = np.load(os.path.join(tl.GOLDEN, "reference_small.npz"), allow_pickle=False)
    return G[name].astype(np.float32)


def flux_model(orc, c):
    m = ctypes.c_void_p(orc.orc_flux_create_synth(c["hidden"], c["heads"], c["n_double"], c["n_single"],
                                                  c["text_dim"], 128, 3.0, 2000.0, c["model_seed"]))
    assert m.value
    return m


def flux_sample(orc, c, t0):
    sched = schedule(c["sched"])
    m = flux_model(orc, c)
    C, lh, lw = c["latent"]
    n = C * lh * lw
    z = tl.take_f32(orc, orc.orc_init_noise(1, C, lh, lw, ctypes.c_int64(c["noise_seed"])), n)
    txt = tl.synth_f32((c["text_tokens"], c["text_dim"]), c["text_seed"])
    print(f"model {time.time() - t0:.0f} s, {orc.orc_blas_info().decode()}", flush=True)
    res = {"schedule": sched, "noise": z.copy()}
    for i in range(len(sched) - 1):
        v = tl.take_f32(orc, orc.orc_flux_forward(m, tl.fptr(z), lh, lw, tl.fptr(txt), c["text_tokens"],
                                                  ctypes.c_float(sched[i])), n)
        res[f"velocity_{i}"] = v
        z = z + np.float32(sched[i + 1] - sched[i]) * v
        print(f"step {i} done {time.time() - t0:.0f} s", flush=True)
    orc.orc_flux_free(m)
    return res, z


class OrcRef(ctypes.Structure):
    _fields_ = [("latent", tl.FP), ("h", ctypes.c_int), ("w", ctypes.c_int), ("t_offset", ctypes.c_int)]


def flux_refs(orc, c, t0):
    m = flux_model(orc, c)
    C, lh, lw = c["latent"]
    n = C * lh * lw
    lat = tl.synth_f32((C, lh, lw), c["latent_seed"])
    txt = tl.synth_f32((c["text_tokens"], c["text_dim"]), c["text_seed"])
    rl = [tl.synth_f32((C, rh, rw), s) for rh, rw, _, s in c["refs"]]
    orefs = (OrcRef * len(rl))(*[OrcRef(tl.fptr(r), rh, rw, to) for r, (rh, rw, to, _) in zip(rl, c["refs"])])
    print(f"model {time.time() - t0:.0f} s, {orc.orc_blas_info().decode()}", flush=True)
    v = tl.take_f32(orc, orc.orc_flux_forward_refs(m, tl.fptr(lat), lh, lw, orefs, len(rl), tl.fptr(txt),
                                                   c["text_tokens"], ctypes.c_float(c["t"])), n)
    print(f"forward with references {time.time() - t0:.0f} s", flush=True)
    plain = tl.take_f32(orc, orc.orc_flux_forward(m, tl.fptr(lat), lh, lw, tl.fptr(txt), c["text_tokens"],
                                                  ctypes.c_float(c["t"])), n)
    print(f"forward without {time.time() - t0:.0f} s", flush=True)
    orc.orc_flux_free(m)
    return {"velocity": v, "velocity_without_refs": plain}


def zimage_sample(orc, c, t0):
    orc.orc_zi_create_synth.argtypes = [ctypes.c_int] * 7 + [ctypes.c_float, ctypes.c_void_p, ctypes.c_int,
                                                             ctypes.c_int, ctypes.c_uint64]
    orc.orc_zi_forward.argtypes = [ctypes.c_void_p, tl.FP, ctypes.c_int, ctypes.c_int, ctypes.c_float, tl.FP,
                                   ctypes.c_int]
    orc.orc_zi_set_reference_aliasing(0)
    axes = (ctypes.c_int * 3)(*c["axes"])
    m = ctypes.c_void_p(orc.orc_zi_create_synth(c["dim"], c["heads"], c["layers"], c["refiners"], c["cap_dim"],
                                                c["in_ch"], c["ps"], c["theta"], axes, c["ffn"], c["t_mid"],
                                                c["model_seed"]))
    assert m.value
    sched = schedule(c["sched"])
    C, lh, lw = c["latent"]
    n = C * lh * lw
    z = tl.take_f32(orc, orc.orc_init_noise(1, C, lh, lw, ctypes.c_int64(c["noise_seed"])), n)
    cap = tl.synth_f32((c["cap_len"], c["cap_dim"]), c["cap_seed"])
    print(f"model {time.time() - t0:.0f} s, {orc.orc_blas_info().decode()}", flush=True)
    res = {"schedule": sched, "noise": z.copy()}
    for i in range(len(sched) - 1):
        v = tl.take_f32(orc, orc.orc_zi_forward(m, tl.fptr(z), lh, lw, ctypes.c_float(1.0 - sched[i]),
                                                tl.fptr(cap), c["cap_len"]), n)
        res[f"velocity_{i}"] = v
        z = z + np.float32(sched[i + 1] - sched[i]) * (-v)
        print(f"step {i} done {time.time() - t0:.0f} s", flush=True)
    orc.orc_zi_free(m)
    return res, z


def main(names):
    orc = tl.oracle()
    for name in names:
        c = TARGETS[name]
        t0 = time.time()
        if name == "c3":
            res = flux_refs(orc, c, t0)
        else:
            res, z = (zimage_sample if name == "zimage" else flux_sample)(orc, c, t0)
            if name == "c2":            # the first golden keeps its original layout
                res["final_latent"] = z
            else:
                res["noise_sha256"] = np.array(sha256(res.pop("noise")))
                res["final_latent_sha256"] = np.array(sha256(z))
        out = os.path.join(tl.GOLDEN, c["out"])
        np.savez_compressed(out, **res)
        print(f"wrote {out} {sorted(res)} in {time.time() - t0:.0f} s", flush=True)


if __name__ == "__main__":
    main(sys.argv[1:] or ["c2"])
