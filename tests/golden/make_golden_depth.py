"""Writes tests/golden/oracle_4b_c2_sample.npz: the oracle's 4-step sample of
the Flux.2-Klein-4B-shaped denoiser at full depth (5 double + 20 single
blocks, hidden 3072, 24 heads, text 7680) on a 512x512 image (32x32 latent,
1024 image tokens + 512 text tokens).

The oracle (oracle/liboracle.so, the C restatement of the reference's f32
`make blas` path, pinned to the reference build at small sizes and on a
4B-shaped block by tests/test_oracle.py) runs here on OpenBLAS; the
reference's own generic build multiplies with single-threaded loop nests and
would take hours at this size. Inputs are pure functions of seeds:

  * weights: iris_synth (include/iris_synth.h), model seed 4242;
  * noise: the reference's iris_init_noise(1, 128, 32, 32, seed 42), which the
    oracle reproduces bit for bit;
  * schedule: the reference build's iris_official_schedule(4, 1024)
    (sched_official_4_1024 of reference_small.npz);
  * text: iris_synth f32 N(0, 1) [512, 7680], seed 4243.

Stored: the velocity of every step on the oracle's trajectory (z_{i+1} =
z_i + (t_{i+1} - t_i) v_i in float32, iris_sample.c:359) and the final latent.

    python tests/golden/make_golden_depth.py      (about 7 minutes on 8 cores)
"""
import ctypes
import os
import sys
import time

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import iris_testlib as tl  # noqa: E402

CFG = {"hidden": 3072, "heads": 24, "n_double": 5, "n_single": 20, "text_dim": 7680, "latent": [128, 32, 32],
       "text_tokens": 512, "model_seed": 4242, "noise_seed": 42, "text_seed": 4243}
OUT = os.path.join(tl.GOLDEN, "oracle_4b_c2_sample.npz")


def main():
    orc = tl.oracle()
    G = np.load(os.path.join(tl.GOLDEN, "reference_small.npz"), allow_pickle=False)
    sched = G["sched_official_4_1024"].astype(np.float32)
    c = CFG
    t0 = time.time()
    m = ctypes.c_void_p(orc.orc_flux_create_synth(c["hidden"], c["heads"], c["n_double"], c["n_single"],
                                                  c["text_dim"], 128, 3.0, 2000.0, c["model_seed"]))
    assert m.value
    C, lh, lw = c["latent"]
    n = C * lh * lw
    z = tl.take_f32(orc, orc.orc_init_noise(1, C, lh, lw, ctypes.c_int64(c["noise_seed"])), n)
    txt = tl.synth_f32((c["text_tokens"], c["text_dim"]), c["text_seed"])
    print(f"model {time.time() - t0:.0f} s, {orc.orc_blas_info().decode()}", flush=True)
    res = {"schedule": sched, "noise": z.copy()}
    for i in range(4):
        v = tl.take_f32(orc, orc.orc_flux_forward(m, tl.fptr(z), lh, lw, tl.fptr(txt), c["text_tokens"],
                                                  ctypes.c_float(sched[i])), n)
        res[f"velocity_{i}"] = v
        z = z + np.float32(sched[i + 1] - sched[i]) * v
        print(f"step {i} done {time.time() - t0:.0f} s", flush=True)
    res["final_latent"] = z
    orc.orc_flux_free(m)
    np.savez_compressed(OUT, **res)
    print("wrote", OUT, sorted(res))


if __name__ == "__main__":
    main()
