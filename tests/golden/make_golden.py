"""Writes the golden fixtures of tests/golden/ by running the reference itself.

Run where the reference tree exists (it is compiled by `make -C oracle ref` from
the sources where they lie, generic backend, the reference's own CFLAGS):

    python tests/golden/make_golden.py [--skip-c1]

Every input is a pure function of a seed (include/iris_synth.h), so the
fixtures hold only seeds, shapes and the reference's outputs. Large outputs are
stored as fingerprints (strided subsample + moments); tables that must be
bit-exact are stored as SHA-256 digests of their bytes.
"""
import argparse
import ctypes
import json
import os
import sys
import tempfile

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import iris_testlib as tl  # noqa: E402

FLUX_TINY = {"heads": 2, "n_double": 2, "n_single": 2, "text_dim": 256, "latent_ch": 128,
             "mlp_ratio": 3.0, "theta": 2000.0, "seed": 1234}
ZI_TINY = {"dim": 256, "heads": 2, "layers": 2, "refiners": 1, "cap_dim": 128, "in_ch": 16, "ps": 2,
           "theta": 256.0, "axes": [32, 48, 48], "ffn": 768, "t_mid": 256, "seed": 4321}
ZI_TRIU_CASES = [(12, 20, 0.4, (31, 34)), (16, 32, 0.9, (35, 36)), (8, 7, 0.05, (37, 38))]
C1 = {"heads": 24, "n_double": 1, "n_single": 1, "text_dim": 7680, "latent_ch": 128, "mlp_ratio": 3.0,
      "theta": 2000.0, "seed": 777}


def tables(lib, fn, n, *args):
    c = np.zeros(n, np.float32)
    s = np.zeros(n, np.float32)
    getattr(lib, fn)(tl.fptr(c), tl.fptr(s), *args)
    return c, s


def rope_goldens(r):
    out = {}
    f = ctypes.c_float
    for (ph, pw, t) in [(8, 8, 0), (8, 8, 1), (4, 6, 2), (16, 16, 0), (32, 32, 0), (64, 64, 0), (64, 64, 1),
                        (64, 64, 2), (64, 64, 10)]:
        c, s = tables(r, "ref_rope_img", ph * pw * 128, ph, pw, 32, f(2000.0), t)
        out[f"img_{ph}x{pw}_t{t}"] = tl.sha(c, s)
    for T in [32, 128, 512]:
        c, s = tables(r, "ref_rope_txt", T * 128, T, 32, f(2000.0))
        out[f"txt_{T}"] = tl.sha(c, s)
    for t in [0.0, 0.25, 0.958085, 1.0]:
        sc = np.zeros(256, np.float32)
        r.ref_timestep_sincos(tl.fptr(sc), f(t * 1000.0), 256, f(10000.0))
        out[f"tsincos_{t}"] = tl.sha(sc)
    return out


def flux_goldens(r, d, res):
    cfg = FLUX_TINY
    tl.write_flux_model(d, cfg, cfg["seed"])
    tf = r.iris_transformer_load_safetensors(d.encode())
    assert tf, "reference failed to load the synthetic model"
    tf = ctypes.c_void_p(tf)
    h, f = 256, ctypes.c_float
    t_emb = np.zeros(h, np.float32)
    r.ref_time_embed(tf, f(0.7), tl.fptr(t_emb))
    res["flux_t_emb"] = t_emb
    dimg, dtxt = np.zeros(6 * h, np.float32), np.zeros(6 * h, np.float32)
    sgl, fin = np.zeros(3 * h, np.float32), np.zeros(2 * h, np.float32)
    r.ref_modulation(tf, tl.fptr(t_emb), tl.fptr(dimg), tl.fptr(dtxt), tl.fptr(sgl), tl.fptr(fin))
    res.update(flux_mod_dimg=dimg, flux_mod_dtxt=dtxt, flux_mod_single=sgl, flux_mod_final=fin)
    I, T = 64, 32
    ic, is_ = tables(r, "ref_rope_img", I * 128, 8, 8, 32, f(2000.0), 0)
    tc, ts = tables(r, "ref_rope_txt", T * 128, T, 32, f(2000.0))
    img = tl.synth_f32((I, h), 11)
    txt = tl.synth_f32((T, h), 12)
    mod_i = tl.synth_f32((6 * h,), 13, 0.0, 0.5)
    mod_t = tl.synth_f32((6 * h,), 14, 0.0, 0.5)
    r.ref_double_block(tf, 1, tl.fptr(img), tl.fptr(txt), tl.fptr(mod_i), tl.fptr(mod_t),
                       tl.fptr(ic), tl.fptr(is_), tl.fptr(tc), tl.fptr(ts), I, T)
    res.update(flux_dbl1_img=img, flux_dbl1_txt=txt)
    x = tl.synth_f32((T + I, h), 15)
    temb = tl.synth_f32((h,), 16)
    r.ref_single_block(tf, 1, tl.fptr(x), tl.fptr(temb), tl.fptr(ic), tl.fptr(is_), tl.fptr(tc),
                       tl.fptr(ts), T + I, T)
    res["flux_sgl1_x"] = x
    lat = tl.synth_f32((128, 8, 8), 21)
    temb_txt = tl.synth_f32((T, 256), 22)
    p = r.iris_transformer_forward(tf, tl.fptr(lat), 8, 8, tl.fptr(temb_txt), T, f(0.8))
    res["flux_fwd"] = tl.take_f32(r, p, 128 * 64)

    class Ref(ctypes.Structure):
        _fields_ = [("latent", tl.FP), ("h", ctypes.c_int), ("w", ctypes.c_int), ("t_offset", ctypes.c_int)]
    r1 = tl.synth_f32((128, 8, 8), 23)
    r2 = tl.synth_f32((128, 4, 6), 24)
    refs = (Ref * 2)(Ref(tl.fptr(r1), 8, 8, 1), Ref(tl.fptr(r2), 4, 6, 2))
    p = r.iris_transformer_forward_with_multi_refs(tf, tl.fptr(lat), 8, 8, refs, 2, tl.fptr(temb_txt), T, f(0.6))
    res["flux_fwd_refs"] = tl.take_f32(r, p, 128 * 64)
    # SREF RoPE band control on the reference keys (iris_transformer_set_sref_bands)
    r.iris_transformer_set_sref_bands.argtypes = [ctypes.c_void_p, ctypes.c_float, ctypes.c_float]
    r.iris_transformer_set_sref_bands(tf, 0.0, 8.0)
    p = r.iris_transformer_forward_with_multi_refs(tf, tl.fptr(lat), 8, 8, refs, 2, tl.fptr(temb_txt), T, f(0.6))
    res["flux_fwd_refs_sref_bands"] = tl.take_f32(r, p, 128 * 64)
    r.iris_transformer_set_sref_bands(tf, 1.0, 1.0)
    # LoRA on every adapted linear (lora_apply at the reference's call sites)
    r.iris_transformer_set_lora.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    r.iris_transformer_set_lora(tf, tl.make_lora(cfg, seed=5, std=0.2))
    p = r.iris_transformer_forward(tf, tl.fptr(lat), 8, 8, tl.fptr(temb_txt), T, f(0.8))
    res["flux_fwd_lora"] = tl.take_f32(r, p, 128 * 64)
    # a LoRA of a trained adapter's size: rank 16, A and B entries of std
    # 0.0125, so scale * B A is about 1 % of W (entries of std 1/sqrt(fan_in))
    r.iris_transformer_set_lora(tf, tl.make_lora(cfg, seed=6, rank=16, std=0.0125))
    p = r.iris_transformer_forward(tf, tl.fptr(lat), 8, 8, tl.fptr(temb_txt), T, f(0.8))
    res["flux_fwd_lora_r16"] = tl.take_f32(r, p, 128 * 64)
    r.iris_transformer_set_lora(tf, None)
    # CSD style delta on the time embedding (iris_transformer_set_csd_delta)
    r.iris_transformer_set_csd_delta.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    r.iris_transformer_set_csd_delta(tf, tl.c_floats(tl.synth_f32((256,), 61, 0.0, 0.5)))
    p = r.iris_transformer_forward(tf, tl.fptr(lat), 8, 8, tl.fptr(temb_txt), T, f(0.8))
    res["flux_fwd_csd"] = tl.take_f32(r, p, 128 * 64)
    r.iris_transformer_set_csd_delta(tf, None)
    # 2-step Euler sample from the reference's own noise and schedule
    sched = r.iris_official_schedule(2, 64)
    sched_arr = np.ctypeslib.as_array(ctypes.cast(sched, tl.FP), shape=(3,)).copy()
    noise = r.iris_init_noise(1, 128, 8, 8, ctypes.c_int64(42))
    noise_arr = np.ctypeslib.as_array(ctypes.cast(noise, tl.FP), shape=(128 * 64,)).copy()
    r.iris_sample_euler.argtypes = [ctypes.c_void_p, ctypes.c_void_p, tl.FP, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, tl.FP, ctypes.c_int, tl.FP, ctypes.c_int,
                                    ctypes.c_void_p]
    p = r.iris_sample_euler(tf, None, tl.fptr(noise_arr), 1, 128, 8, 8, tl.fptr(temb_txt), T,
                            tl.fptr(sched_arr), 2, None)
    res["flux_sample2"] = tl.take_f32(r, p, 128 * 64)
    res["flux_sample2_sched"] = sched_arr
    res["flux_noise42"] = noise_arr
    # the reference-image samplers: one reference (T offset 1), two references,
    # CFG over both references with equal text lengths, CFG over one
    # reference with an uncond text of 20 tokens
    V, I_ = ctypes.c_void_p, ctypes.c_int
    r.iris_sample_euler_with_refs.argtypes = [V, V, tl.FP, I_, I_, I_, I_, tl.FP, I_, I_, I_, tl.FP, I_, tl.FP, I_, V]
    r.iris_sample_euler_with_multi_refs.argtypes = [V, V, tl.FP, I_, I_, I_, I_, V, I_, tl.FP, I_, tl.FP, I_, V]
    r.iris_sample_euler_cfg_with_multi_refs.argtypes = [V, V, tl.FP, I_, I_, I_, I_, V, I_, tl.FP, I_, tl.FP, I_,
                                                        ctypes.c_float, tl.FP, I_, V]
    r.iris_sample_euler_cfg_with_refs.argtypes = [V, V, tl.FP, I_, I_, I_, I_, tl.FP, I_, I_, I_, tl.FP, I_, tl.FP,
                                                  I_, ctypes.c_float, tl.FP, I_, V]
    for fn in ("iris_sample_euler_with_refs", "iris_sample_euler_with_multi_refs",
               "iris_sample_euler_cfg_with_multi_refs", "iris_sample_euler_cfg_with_refs"):
        getattr(r, fn).restype = V
    txt_u = tl.synth_f32((T, 256), 25)
    txt_u20 = tl.synth_f32((20, 256), 26)
    p = r.iris_sample_euler_with_refs(tf, None, tl.fptr(noise_arr), 1, 128, 8, 8, tl.fptr(r1), 8, 8, 1,
                                      tl.fptr(temb_txt), T, tl.fptr(sched_arr), 2, None)
    res["flux_sample2_ref1"] = tl.take_f32(r, p, 128 * 64)
    p = r.iris_sample_euler_with_multi_refs(tf, None, tl.fptr(noise_arr), 1, 128, 8, 8, refs, 2, tl.fptr(temb_txt), T,
                                            tl.fptr(sched_arr), 2, None)
    res["flux_sample2_refs"] = tl.take_f32(r, p, 128 * 64)
    p = r.iris_sample_euler_cfg_with_multi_refs(tf, None, tl.fptr(noise_arr), 1, 128, 8, 8, refs, 2,
                                                tl.fptr(temb_txt), T, tl.fptr(txt_u), T, 4.0, tl.fptr(sched_arr), 2,
                                                None)
    res["flux_sample2_cfg_refs"] = tl.take_f32(r, p, 128 * 64)
    p = r.iris_sample_euler_cfg_with_refs(tf, None, tl.fptr(noise_arr), 1, 128, 8, 8, tl.fptr(r2), 4, 6, 2,
                                          tl.fptr(temb_txt), T, tl.fptr(txt_u20), 20, 3.0, tl.fptr(sched_arr), 2,
                                          None)
    res["flux_sample2_cfg_ref1_t20"] = tl.take_f32(r, p, 128 * 64)
    # the ancestral (eta 0.6, noise from the global generator seeded with
    # 1234) and Heun samplers, iris_sample.c:990-1145, over 3 steps
    sched3 = r.iris_official_schedule(3, 64)
    sched3_arr = np.ctypeslib.as_array(ctypes.cast(sched3, tl.FP), shape=(4,)).copy()
    r.iris_sample_euler_ancestral.argtypes = [V, tl.FP, I_, I_, I_, I_, tl.FP, I_, tl.FP, I_, ctypes.c_float, V]
    r.iris_sample_heun.argtypes = [V, tl.FP, I_, I_, I_, I_, tl.FP, I_, tl.FP, I_, V]
    r.iris_sample_euler_ancestral.restype = V
    r.iris_sample_heun.restype = V
    r.iris_rng_seed.argtypes = [ctypes.c_uint64]
    r.iris_rng_seed(1234)
    p = r.iris_sample_euler_ancestral(tf, tl.fptr(noise_arr), 1, 128, 8, 8, tl.fptr(temb_txt), T,
                                      tl.fptr(sched3_arr), 3, 0.6, None)
    res["flux_sample3_ancestral"] = tl.take_f32(r, p, 128 * 64)
    p = r.iris_sample_heun(tf, tl.fptr(noise_arr), 1, 128, 8, 8, tl.fptr(temb_txt), T, tl.fptr(sched3_arr), 3, None)
    res["flux_sample3_heun"] = tl.take_f32(r, p, 128 * 64)
    res["flux_sample3_sched"] = sched3_arr
    r.iris_transformer_free(tf)


def zimage_goldens(r, d, res, hashes):
    cfg = ZI_TINY
    tl.write_zimage_model(d, cfg, cfg["seed"])
    axes = (ctypes.c_int * 3)(*cfg["axes"])
    r.zi_transformer_load_safetensors.argtypes = [ctypes.c_char_p] + [ctypes.c_int] * 7 + [ctypes.c_float,
                                                                                           ctypes.c_void_p]
    tf = r.zi_transformer_load_safetensors(d.encode(), cfg["dim"], cfg["heads"], cfg["layers"], cfg["refiners"],
                                           cfg["cap_dim"], cfg["in_ch"], cfg["ps"], cfg["theta"], axes)
    assert tf, "reference failed to load the synthetic Z-Image model"
    tf = ctypes.c_void_p(tf)
    for ax, dd in enumerate(cfg["axes"]):
        c, s = tables(r, "ref_zi_rope_table", 1024 * dd // 2, tf, ax)
        hashes[f"zi_rope_axis{ax}"] = tl.sha(c, s)
    lat = tl.synth_f32((16, 12, 12), 31)
    pt = np.zeros(36 * 64, np.float32)
    r.ref_zi_patchify(tl.fptr(pt), tl.fptr(lat), 16, 12, 12, 2)
    hashes["zi_patchify_16x12x12"] = tl.sha(pt)
    temb = np.zeros(256, np.float32)
    r.ref_zi_t_embed(tf, ctypes.c_float(0.3), tl.fptr(temb))
    res["zi_t_emb"] = temb
    # block-level: a main layer over a padded unified sequence (36 img -> 64, 20 cap -> 32)
    seq = 96
    x = tl.synth_f32((seq, 256), 32)
    pos = np.zeros((seq, 3), np.int32)
    for i in range(36):
        pos[i] = (33, i // 6, i % 6)
    for s in range(32):
        pos[64 + s] = (1 + s, 0, 0)
    mask = np.array([1 if (i < 36 or 64 <= i < 84) else 0 for i in range(seq)], np.int32)
    res["zi_blk_in_pos"] = pos
    res["zi_blk_in_mask"] = mask
    r.ref_zi_block(tf, 2, 1, tl.fptr(x), pos.ctypes.data_as(tl.IP), mask.ctypes.data_as(tl.IP), tl.fptr(temb), seq)
    res["zi_layer1"] = x
    xc = tl.synth_f32((32, 256), 33)
    r.ref_zi_block(tf, 1, 0, tl.fptr(xc), pos[64:].ctypes.data_as(tl.IP), mask[64:].ctypes.data_as(tl.IP),
                   None, 32)
    res["zi_ctx0"] = xc
    cap = tl.synth_f32((20, 128), 34)
    p = r.zi_transformer_forward(tf, tl.fptr(lat), 12, 12, ctypes.c_float(0.4), tl.fptr(cap), 20)
    res["zi_fwd_12x12_cap20"] = tl.take_f32(r, p, 16 * 144)
    lat2 = tl.synth_f32((16, 16, 16), 35)
    cap2 = tl.synth_f32((32, 128), 36)
    p = r.zi_transformer_forward(tf, tl.fptr(lat2), 16, 16, ctypes.c_float(0.9), tl.fptr(cap2), 32)
    res["zi_fwd_16x16_cap32"] = tl.take_f32(r, p, 16 * 256)
    r.zi_transformer_free(tf)


def zimage_triu_goldens(r, d, res):
    """Same tiny model with upper-triangular attention output projections: the
    reference CPU path's in-place projection then equals the out-of-place one,
    so these outputs are the model's out-of-place forward."""
    cfg = ZI_TINY
    tl.write_zimage_model(d, cfg, cfg["seed"], triu_out=True)
    axes = (ctypes.c_int * 3)(*cfg["axes"])
    tf = r.zi_transformer_load_safetensors(d.encode(), cfg["dim"], cfg["heads"], cfg["layers"], cfg["refiners"],
                                           cfg["cap_dim"], cfg["in_ch"], cfg["ps"], cfg["theta"], axes)
    assert tf, "reference failed to load the synthetic Z-Image model"
    tf = ctypes.c_void_p(tf)
    for hw, cap_len, t, seeds in ZI_TRIU_CASES:
        lat = tl.synth_f32((16, hw, hw), seeds[0])
        cap = tl.synth_f32((cap_len, 128), seeds[1])
        p = r.zi_transformer_forward(tf, tl.fptr(lat), hw, hw, ctypes.c_float(t), tl.fptr(cap), cap_len)
        res[f"zi_triu_fwd_{hw}x{hw}_cap{cap_len}"] = tl.take_f32(r, p, 16 * hw * hw)
    r.zi_transformer_free(tf)


def fast_expf_golden(r, res):
    r.ref_fast_expf.restype = ctypes.c_float
    xs = np.linspace(-90.0, 90.0, 2001).astype(np.float32)
    res["fast_expf_x"] = xs
    res["fast_expf_y"] = np.array([r.ref_fast_expf(ctypes.c_float(v)) for v in xs], np.float32)


def sampler_goldens(r, res, hashes):
    for n, seq in [(4, 1024), (4, 4096), (50, 4096)]:
        p = r.iris_official_schedule(n, seq)
        res[f"sched_official_{n}_{seq}"] = tl.take_f32(r, p, n + 1)
    os.environ.pop("IRIS_ZIMAGE_SHIFT", None)
    p = r.iris_zimage_schedule(8, 4096)
    res["sched_zimage_8"] = tl.take_f32(r, p, 9)
    for (c, hh, ww, seed) in [(128, 64, 64, 42), (128, 32, 32, 7), (16, 128, 128, 3)]:
        p = r.iris_init_noise(1, c, hh, ww, ctypes.c_int64(seed))
        hashes[f"noise_{c}x{hh}x{ww}_s{seed}"] = tl.sha(tl.take_f32(r, p, c * hh * ww))


def c1_golden(r, d, res):
    cfg = C1
    tl.write_flux_model(d, cfg, cfg["seed"])
    tf = r.iris_transformer_load_safetensors(d.encode())
    assert tf
    tf = ctypes.c_void_p(tf)
    f = ctypes.c_float
    T, I, h = 128, 256, 3072
    ic, is_ = tables(r, "ref_rope_img", I * 128, 16, 16, 32, f(2000.0), 0)
    tc, ts = tables(r, "ref_rope_txt", T * 128, T, 32, f(2000.0))
    x = tl.synth_f32((T + I, h), 41)
    temb = tl.synth_f32((h,), 42)
    x0 = x.copy()
    r.ref_single_block(tf, 0, tl.fptr(x), tl.fptr(temb), tl.fptr(ic), tl.fptr(is_), tl.fptr(tc), tl.fptr(ts),
                       T + I, T)
    fp = tl.fingerprint(x)
    fd = tl.fingerprint(x - x0)
    res["c1_out_sub"], res["c1_out_sum"], res["c1_out_sumsq"] = fp["sub"], fp["sum"], fp["sumsq"]
    res["c1_delta_sub"], res["c1_delta_sum"], res["c1_delta_sumsq"] = fd["sub"], fd["sum"], fd["sumsq"]
    r.iris_transformer_free(tf)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--skip-c1", action="store_true")
    args = ap.parse_args()
    r = tl.ref()
    res, hashes = {}, {}
    hashes.update(rope_goldens(r))
    with tempfile.TemporaryDirectory() as d:
        flux_goldens(r, d, res)
    with tempfile.TemporaryDirectory() as d:
        zimage_goldens(r, d, res, hashes)
    with tempfile.TemporaryDirectory() as d:
        zimage_triu_goldens(r, d, res)
    sampler_goldens(r, res, hashes)
    fast_expf_golden(r, res)
    np.savez_compressed(os.path.join(tl.GOLDEN, "reference_small.npz"), **res)
    if not args.skip_c1:
        c1 = {}
        with tempfile.TemporaryDirectory() as d:
            c1_golden(r, d, c1)
        np.savez_compressed(os.path.join(tl.GOLDEN, "reference_c1_single_block.npz"), **c1)
    def schedule_lanes():
        """the vector lane plan of this host's -march=native reference build
        (16-wide with AVX-512 F + VL, else 8-wide with AVX2 + FMA)"""
        flags = next((ln.split(":", 1)[1].split() for ln in open("/proc/cpuinfo") if ln.startswith("flags")), [])
        if "avx512f" in flags and "avx512vl" in flags:
            return "avx512"
        return "avx2" if "avx2" in flags and "fma" in flags else "scalar"

    manifest = {
        "generator": "tests/golden/make_golden.py",
        "reference_build": "oracle/Makefile `ref`: gcc -O3 -march=native -ffast-math -DGENERIC_BUILD",
        "flux_tiny": FLUX_TINY, "zimage_tiny": ZI_TINY, "zimage_triu_cases": ZI_TRIU_CASES, "c1": C1,
        "inputs": "iris_synth f32 N(0,1) by seed (see make_golden.py); weights bf16 via iris_synth_seed(name)",
        "schedule_lanes": schedule_lanes(),
        "sha256": hashes,
    }
    with open(os.path.join(tl.GOLDEN, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print("wrote", sorted(res), len(hashes), "hashes")


if __name__ == "__main__":
    main()
