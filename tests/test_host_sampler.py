"""Sampler inputs of the product (libiris_hip.so host code, no GPU needed):
schedules, seeded noise and the timestep sinusoid, bit for bit.

* Against the reference build's own outputs committed in tests/golden/
  (made by tests/golden/make_golden.py from the reference compiled with its
  own -O3 -march=native -ffast-math flags): assert_array_equal / SHA-256.
* Against the reference build itself where oracle/_ref exists (this
  container): every schedule function over 1..70 steps and several sequence
  lengths and resolutions, bit for bit, including the IRIS_ZIMAGE_SHIFT path.
* Against float64 closed forms of the source formulas (iris_sample.c:61-244),
  which pin the schedules without the reference build.

The reference build's vectorized schedule lanes divide through the CPU's
reciprocal estimate (rcpps, or vrcp14ps in 16-wide AVX-512 blocks) and one
Newton step, in blocks whose widths follow the host's vector ISA; the product
uses the same instructions and the same blocks, so these equalities hold on a
host of the model that made the goldens (run with that host's lane plan,
recorded in manifest.json) and against the reference build on the host that
runs the tests.
"""
import ctypes
import json
import os

import numpy as np
import pytest

import iris_testlib as tl

G = np.load(os.path.join(tl.GOLDEN, "reference_small.npz"), allow_pickle=False)
MAN = json.load(open(os.path.join(tl.GOLDEN, "manifest.json")))
F = ctypes.c_float
libc = ctypes.CDLL(None)


@pytest.fixture(scope="module")
def prod():
    if not os.path.exists(tl.HIP_SO):
        pytest.fail(f"{tl.HIP_SO} is not built")
    lib = ctypes.CDLL(tl.HIP_SO)          # host functions only: nothing here touches a GPU
    for fn in ("iris_linear_schedule", "iris_power_schedule", "iris_sigmoid_schedule", "iris_resolution_schedule",
               "iris_official_schedule", "iris_zimage_schedule", "iris_init_noise"):
        getattr(lib, fn).restype = ctypes.c_void_p
    lib.iris_init_noise.argtypes = [ctypes.c_int] * 4 + [ctypes.c_int64]
    lib.iris_timestep_sincos.argtypes = [tl.FP, F, ctypes.c_int, F]
    return lib


def take(p, n):
    assert p
    out = np.ctypeslib.as_array(ctypes.cast(p, tl.FP), shape=(n,)).copy()
    libc.free(ctypes.c_void_p(p))
    return out


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.fixture
def golden_lanes(monkeypatch):
    """the schedule lane plan of the host that made the goldens (the product
    can narrow its plan to it; a wider one than this CPU runs is skipped)"""
    plan = MAN.get("schedule_lanes", "avx2")
    flags = next((ln.split(":", 1)[1].split() for ln in open("/proc/cpuinfo") if ln.startswith("flags")), [])
    have = {"scalar": True, "avx2": "avx2" in flags and "fma" in flags,
            "avx512": "avx512f" in flags and "avx512vl" in flags}
    if not have[plan]:
        pytest.skip(f"the goldens' schedules come from {plan} lanes, which this CPU lacks")
    monkeypatch.setenv("IRIS_SCHEDULE_ISA", plan)
    return plan


@pytest.mark.parametrize("n,seq", [(4, 1024), (4, 4096), (50, 4096)])
def test_official_schedule_equals_reference_golden(prod, golden_lanes, n, seq):
    got = take(prod.iris_official_schedule(n, seq), n + 1)
    np.testing.assert_array_equal(bits(got), bits(G[f"sched_official_{n}_{seq}"]))


def test_zimage_schedule_equals_reference_golden(prod, golden_lanes, monkeypatch):
    monkeypatch.delenv("IRIS_ZIMAGE_SHIFT", raising=False)
    got = take(prod.iris_zimage_schedule(8, 4096), 9)
    np.testing.assert_array_equal(bits(got), bits(G["sched_zimage_8"]))
    # and the reference's own test goldens (debug/test_zimage_scheduler.c:71-79, tol 1e-5)
    gold3 = [1.0, 0.947542489, 0.882787704, 0.800837338, 0.693793058, 0.548045635, 0.337972105, 0.008928538, 0.0]
    assert np.abs(got - gold3).max() <= 1e-5
    monkeypatch.setenv("IRIS_ZIMAGE_SHIFT", "3.16")
    gold316 = [1.0, 0.950074732, 0.888080359, 0.809038460, 0.704796433, 0.561017215, 0.349943727, 0.009896723, 0.0]
    assert np.abs(take(prod.iris_zimage_schedule(8, 4096), 9) - gold316).max() <= 1e-5


@pytest.mark.parametrize("c,h,w,seed", [(128, 64, 64, 42), (128, 32, 32, 7), (16, 128, 128, 3)])
def test_init_noise_equals_reference_digest(prod, c, h, w, seed):
    got = take(prod.iris_init_noise(1, c, h, w, seed), c * h * w)
    assert tl.sha(got) == MAN["sha256"][f"noise_{c}x{h}x{w}_s{seed}"]


def test_noise_small_latent_is_subsampled_field(prod):
    """Below 112x112 the noise is a nearest-neighbour subsample of the seed's
    112x112 field (iris_sample.c:1155-1184), so one seed gives one image at
    every size."""
    big = take(prod.iris_init_noise(1, 4, 112, 112, 9), 4 * 112 * 112).reshape(4, 112, 112)
    small = take(prod.iris_init_noise(1, 4, 28, 56, 9), 4 * 28 * 56).reshape(4, 28, 56)
    ys, xs = np.arange(28) * 112 // 28, np.arange(56) * 112 // 56
    np.testing.assert_array_equal(small, big[:, ys][:, :, xs])


@pytest.mark.parametrize("t", [0.0, 0.25, 0.958085, 1.0])
def test_timestep_sincos_equals_reference_digest(prod, t):
    sc = np.zeros(256, np.float32)
    prod.iris_timestep_sincos(tl.fptr(sc), F(np.float32(t) * np.float32(1000.0)), 256, F(10000.0))
    assert tl.sha(sc) == MAN["sha256"][f"tsincos_{t}"]


SCHED_CASES = ([("iris_linear_schedule", ())] +
               [("iris_official_schedule", (s,)) for s in (256, 1024, 4096, 4300, 4301, 16384)] +
               [("iris_zimage_schedule", (4096,))] +
               [("iris_power_schedule", (F(a),)) for a in (2.0, 1.7)] +
               [("iris_sigmoid_schedule", (F(s),)) for s in (0.0, 0.3)] +
               [("iris_resolution_schedule", hw) for hw in ((1024, 1024), (512, 768), (256, 256))])


def closed_form(fn, n, args):
    """float64 statement of iris_sample.c:61-244"""
    i = np.arange(n + 1, dtype=np.float64)
    t = i / n
    if fn == "iris_linear_schedule":
        return 1 - t
    if fn == "iris_power_schedule":
        return 1 - t ** args[0].value
    if fn == "iris_sigmoid_schedule":
        s = 1 - 1 / (1 + np.exp(-((t - 0.5) * 10 + args[0].value)))
        s[0], s[n] = 1, 0
        return s
    if fn == "iris_resolution_schedule":
        px = args[0] * args[1]
        return 1 - t ** (1 + 0.5 * (1.0 if px >= 1 << 20 else 0.5 if px >= 1 << 18 else 0.0))
    if fn == "iris_official_schedule":
        seq = args[0]
        a1, b1, a2, b2 = 8.73809524e-05, 1.89833333, 0.00016927, 0.45666666
        if seq > 4300:
            mu = a2 * seq + b2
        else:
            m200, m10 = a2 * seq + b2, a1 * seq + b1
            a = (m200 - m10) / 190
            mu = a * n + (m200 - 200 * a)
        tt = 1 - t
        with np.errstate(divide="ignore"):
            return np.where(tt <= 0, 0, np.where(tt >= 1, 1, np.exp(mu) / (np.exp(mu) + 1 / np.maximum(tt, 1e-30) - 1)))
    shift = 3.0
    smin = shift * 1e-3 / (1 + (shift - 1) * 1e-3)
    raw = 1 + (smin - 1) * (np.arange(n) / max(n - 1, 1))
    return np.append(shift * raw / (1 + (shift - 1) * raw), 0.0)


@pytest.mark.parametrize("fn,args", SCHED_CASES, ids=lambda v: str(v))
def test_schedules_closed_form(prod, fn, args, monkeypatch):
    monkeypatch.delenv("IRIS_ZIMAGE_SHIFT", raising=False)
    for n in (1, 2, 3, 4, 5, 7, 8, 9, 12, 20, 28, 50):
        got = take(getattr(prod, fn)(n, *args), n + 1).astype(np.float64)
        # the float32 evaluation of mu alone moves the official schedule by ~1e-5
        tol = 4e-5 if fn == "iris_official_schedule" else 2e-6
        np.testing.assert_allclose(got, closed_form(fn, n, args), rtol=0, atol=tol, err_msg=f"{fn} n={n}")


SCALAR_NS = (1, 2, 3, 4, 5, 7, 8, 9, 12, 20, 28, 50)


def test_schedules_scalar_path_closed_form(tmp_path):
    """The schedules on a CPU without AVX2 / FMA (forced with
    IRIS_SCHEDULE_SCALAR=1 in a fresh process: the choice is made once per
    process) take the scalar formulas for every element: within the
    closed-form tolerances, and within 2e-6 of the vector lanes where those
    run (their divisions go through a refined reciprocal estimate)."""
    import subprocess
    import sys
    out = tmp_path / "scalar.npz"
    script = (
        "import ctypes, numpy as np, sys\n"
        f"sys.path.insert(0, {os.path.dirname(os.path.abspath(__file__))!r})\n"
        "import test_host_sampler as t\n"
        f"lib = ctypes.CDLL({tl.HIP_SO!r})\n"
        "res = {}\n"
        "for k, (fn, args) in enumerate(t.SCHED_CASES):\n"
        "    getattr(lib, fn).restype = ctypes.c_void_p\n"
        "    for n in t.SCALAR_NS:\n"
        "        res[f'{k}_{n}'] = t.take(getattr(lib, fn)(n, *args), n + 1)\n"
        f"np.savez({str(out)!r}, **res)\n")
    env = dict(os.environ, IRIS_SCHEDULE_SCALAR="1")
    env.pop("IRIS_ZIMAGE_SHIFT", None)
    subprocess.run([sys.executable, "-c", script], check=True, env=env, timeout=120)
    got = np.load(out)
    lib = ctypes.CDLL(tl.HIP_SO)
    for k, (fn, args) in enumerate(SCHED_CASES):
        getattr(lib, fn).restype = ctypes.c_void_p
        for n in SCALAR_NS:
            a = got[f"{k}_{n}"]
            tol = 4e-5 if fn == "iris_official_schedule" else 2e-6
            np.testing.assert_allclose(a.astype(np.float64), closed_form(fn, n, args), rtol=0, atol=tol,
                                       err_msg=f"{fn} n={n} (scalar)")
            v = take(getattr(lib, fn)(n, *args), n + 1)
            d = np.abs(a.astype(np.float64) - v.astype(np.float64)).max()
            assert d <= 2e-6, (fn, n, d)


@pytest.mark.skipif(not os.path.exists(tl.REF_SO), reason="reference build (oracle/_ref) not present")
@pytest.mark.parametrize("fn,args", SCHED_CASES, ids=lambda v: str(v))
def test_schedules_equal_reference_build(prod, fn, args, monkeypatch):
    """The product's schedule == the reference build's on this host, bit for
    bit, across the 8-wide / 4-wide / scalar lane splits of 1..70 steps."""
    monkeypatch.delenv("IRIS_ZIMAGE_SHIFT", raising=False)
    ref = ctypes.CDLL(tl.REF_SO)
    getattr(ref, fn).restype = ctypes.c_void_p
    for n in list(range(1, 71)) + [128, 256]:
        a = take(getattr(prod, fn)(n, *args), n + 1)
        b = take(getattr(ref, fn)(n, *args), n + 1)
        np.testing.assert_array_equal(bits(a), bits(b), err_msg=f"{fn} n={n}")
    if fn == "iris_zimage_schedule":
        for v in ("3.16", "1.5", "7"):
            monkeypatch.setenv("IRIS_ZIMAGE_SHIFT", v)
            for n in range(1, 40):
                np.testing.assert_array_equal(bits(take(prod.iris_zimage_schedule(n, 1), n + 1)),
                                              bits(take(ref.iris_zimage_schedule(n, 1), n + 1)))


def test_factored_rope_axis_reproduces_tables(prod):
    """The attention prologue's factored RoPE (iris_rope_axis: one axis's
    per-pair cos / sin by position) against the full per-row tables of
    iris_rope_img / iris_rope_txt (4 axes of 32 dims, theta 2000): every
    image row's H and W pairs and T pairs (T-offset 2) and every text row's
    L pairs are the axis table's entries at the row's positions, bit for bit,
    and the identity axes (position 0) are the table's row 0."""
    prod.iris_rope_axis.argtypes = [tl.FP, tl.FP, ctypes.c_int, ctypes.c_int, F]
    prod.iris_rope_img.argtypes = [tl.FP, tl.FP, ctypes.c_int, ctypes.c_int, ctypes.c_int, F, ctypes.c_int]
    prod.iris_rope_txt.argtypes = [tl.FP, tl.FP, ctypes.c_int, ctypes.c_int, F]
    ph, pw, T, L = 24, 40, 77, 80
    ac, as_ = np.zeros((L, 16), np.float32), np.zeros((L, 16), np.float32)
    prod.iris_rope_axis(tl.fptr(ac), tl.fptr(as_), L, 32, F(2000.0))
    ic, is_ = np.zeros((ph * pw, 128), np.float32), np.zeros((ph * pw, 128), np.float32)
    prod.iris_rope_img(tl.fptr(ic), tl.fptr(is_), ph, pw, 32, F(2000.0), 2)
    tc, ts = np.zeros((T, 128), np.float32), np.zeros((T, 128), np.float32)
    prod.iris_rope_txt(tl.fptr(tc), tl.fptr(ts), T, 32, F(2000.0))
    y, x = np.arange(ph * pw) // pw, np.arange(ph * pw) % pw
    for tab, full in ((ac, ic), (as_, is_)):
        pairs = full[:, 0::2]
        np.testing.assert_array_equal(pairs[:, 0:16].view(np.uint32), np.broadcast_to(tab[2], (ph * pw, 16)).view(np.uint32))
        np.testing.assert_array_equal(pairs[:, 16:32].view(np.uint32), tab[y].view(np.uint32))
        np.testing.assert_array_equal(pairs[:, 32:48].view(np.uint32), tab[x].view(np.uint32))
        np.testing.assert_array_equal(pairs[:, 48:64].view(np.uint32), np.broadcast_to(tab[0], (ph * pw, 16)).view(np.uint32))
    for tab, full in ((ac, tc), (as_, ts)):
        pairs = full[:, 0::2]
        np.testing.assert_array_equal(pairs[:, 48:64].view(np.uint32), tab[np.arange(T)].view(np.uint32))
        np.testing.assert_array_equal(pairs[:, 0:48].view(np.uint32),
                                      np.tile(tab[0], (T, 3)).reshape(T, 48).view(np.uint32))
