"""Z-Image S3-DiT denoiser parity: HIP build vs the oracle.

The oracle runs the reference algorithm (iris_transformer_zimage.c) with the
attention output projection computed out of place, as the model defines it
and as the reference's GPU path computes it; the reference CPU path runs that
product in place over its own input, which the oracle reproduces only for
pinning it to the reference goldens (test_oracle.py). Bars: RoPE tables
bit-exact; velocities within rel-L2 1e-2 and cosine >= 0.999.
"""
import ctypes
import json
import os
import tempfile

import numpy as np
import pytest

import iris_testlib as tl

pytestmark = pytest.mark.gpu
F = ctypes.c_float
MAN = json.load(open(os.path.join(tl.GOLDEN, "manifest.json")))
TINY = MAN["zimage_tiny"]


def axes_arr(axes):
    return (ctypes.c_int * 3)(*axes)


@pytest.fixture(scope="module")
def lib():
    return tl.hip()


@pytest.fixture(scope="module")
def orc():
    o = tl.oracle()
    o.orc_zi_load.argtypes = [ctypes.c_char_p] + [ctypes.c_int] * 7 + [ctypes.c_float, ctypes.c_void_p]
    o.orc_zi_create_synth.argtypes = [ctypes.c_int] * 7 + [ctypes.c_float, ctypes.c_void_p, ctypes.c_int,
                                                           ctypes.c_int, ctypes.c_uint64]
    o.orc_zi_set_reference_aliasing(0)
    return o


def tiny_args(cfg=TINY):
    return (cfg["dim"], cfg["heads"], cfg["layers"], cfg["refiners"], cfg["cap_dim"], cfg["in_ch"], cfg["ps"],
            F(cfg["theta"]), axes_arr(cfg["axes"]))


@pytest.fixture(scope="module")
def models(lib, orc):
    with tempfile.TemporaryDirectory() as d:
        tl.write_zimage_model(d, TINY, TINY["seed"])
        tf = lib.zi_transformer_load_safetensors(d.encode(), *tiny_args())
        m = orc.orc_zi_load(d.encode(), *tiny_args())
    assert tf, lib.iris_hip_last_error()
    assert m
    yield ctypes.c_void_p(tf), ctypes.c_void_p(m)
    lib.zi_transformer_free(ctypes.c_void_p(tf))
    orc.orc_zi_free(ctypes.c_void_p(m))


def take(lib, p, n):
    assert p, lib.iris_hip_last_error()
    out = np.ctypeslib.as_array(ctypes.cast(p, tl.FP), shape=(n,)).copy()
    ctypes.CDLL(None).free(ctypes.c_void_p(p))
    return out


def forward(lib, tf, lat, hw, t, cap):
    return take(lib, lib.zi_transformer_forward(tf, tl.fptr(lat), hw, hw, F(t), tl.fptr(cap), cap.shape[0]),
                lat.size)


def oracle_forward(orc, m, lat, hw, t, cap):
    return tl.take_f32(orc, orc.orc_zi_forward(m, tl.fptr(lat), hw, hw, F(t), tl.fptr(cap), cap.shape[0]), lat.size)


@pytest.mark.parametrize("hw,cap_len,t,seeds", [(12, 20, 0.4, (31, 34)), (16, 32, 0.9, (35, 36)),
                                                (8, 7, 0.05, (37, 38))])
def test_forward_vs_oracle(lib, orc, models, hw, cap_len, t, seeds):
    tf, m = models
    lat = tl.synth_f32((16, hw, hw), seeds[0])
    cap = tl.synth_f32((cap_len, TINY["cap_dim"]), seeds[1])
    got = forward(lib, tf, lat, hw, t, cap)
    ref = oracle_forward(orc, m, lat, hw, t, cap)
    assert tl.rel_l2(got, ref) < 1e-2 and tl.cosine(got, ref) > 0.999


@pytest.mark.parametrize("case", range(3))
def test_forward_vs_reference_goldens(lib, case):
    """Against the reference's own outputs on a model whose output projections
    are upper triangular (there the reference CPU path's in-place projection
    equals the out-of-place product)."""
    hw, cap_len, t, seeds = MAN["zimage_triu_cases"][case]
    G = np.load(os.path.join(tl.GOLDEN, "reference_small.npz"), allow_pickle=False)
    with tempfile.TemporaryDirectory() as d:
        tl.write_zimage_model(d, TINY, TINY["seed"], triu_out=True)
        tf = lib.zi_transformer_load_safetensors(d.encode(), *tiny_args())
    assert tf, lib.iris_hip_last_error()
    tf = ctypes.c_void_p(tf)
    lat = tl.synth_f32((16, hw, hw), seeds[0])
    cap = tl.synth_f32((cap_len, TINY["cap_dim"]), seeds[1])
    got = forward(lib, tf, lat, hw, t, cap)
    lib.zi_transformer_free(tf)
    want = G[f"zi_triu_fwd_{hw}x{hw}_cap{cap_len}"]
    assert tl.rel_l2(got, want) < 1e-2 and tl.cosine(got, want) > 0.999


def test_rope_tables_resident_bit_exact(lib, orc, models):
    """Per-row tables of the unified [image | caption] sequence == the oracle's
    per-axis tables gathered at the reference's position ids."""
    tf, m = models
    hw, cap_len = 12, 20
    lat = tl.synth_f32((16, hw, hw), 31)
    cap = tl.synth_f32((cap_len, TINY["cap_dim"]), 34)
    forward(lib, tf, lat, hw, 0.4, cap)
    I, Ip, Cp = 36, 64, 32
    U = Ip + Cp
    got_c, got_s = [tl.d2h_f32(lib, lib.zi_device_buffer(tf, n.encode()), (U, 128)) for n in ("rope_cos", "rope_sin")]
    axes = TINY["axes"]
    tabs = []
    for ax, dd in enumerate(axes):
        c, s = np.zeros(1024 * dd // 2, np.float32), np.zeros(1024 * dd // 2, np.float32)
        orc.orc_zi_rope_tables(m, tl.fptr(c), tl.fptr(s), ax)
        tabs.append((c.reshape(1024, dd // 2), s.reshape(1024, dd // 2)))
    pos = np.zeros((U, 3), np.int64)
    for i in range(I):
        pos[i] = (Cp + 1, i // 6, i % 6)
    for j in range(Cp):
        pos[Ip + j] = (1 + j, 0, 0)
    want_c, want_s = np.zeros((U, 128), np.float32), np.zeros((U, 128), np.float32)
    off = 0
    for ax, dd in enumerate(axes):
        c, s = tabs[ax]
        want_c[:, off:off + dd] = np.repeat(c[pos[:, ax]], 2, axis=1)
        want_s[:, off:off + dd] = np.repeat(s[pos[:, ax]], 2, axis=1)
        off += dd
    np.testing.assert_array_equal(got_c, want_c)
    np.testing.assert_array_equal(got_s, want_s)


def test_two_step_sample_vs_oracle(lib, orc, models):
    """iris_sample_euler_zimage: v at timestep 1 - sigma, z += dt * (-v)."""
    tf, m = models
    hw, cap_len = 12, 20
    z = tl.synth_f32((16, hw, hw), 41)
    cap = tl.synth_f32((cap_len, TINY["cap_dim"]), 42)
    sched = np.array([1.0, 0.6, 0.0], np.float32)
    got = take(lib, lib.iris_sample_euler_zimage(tf, tl.fptr(z), 1, 16, hw, hw, 2, tl.fptr(cap), cap_len,
                                                 tl.fptr(sched), 2, None), z.size)
    want = z.ravel().copy()
    for i in range(2):
        v = oracle_forward(orc, m, want.reshape(z.shape), hw, 1.0 - float(sched[i]), cap)
        want += np.float32(sched[i + 1] - sched[i]) * (-v)
    assert tl.rel_l2(got, want) < 1e-2 and tl.cosine(got, want) > 0.999


def test_synthetic_equals_safetensors(lib, models):
    """zi_transformer_create_synthetic == loading the written safetensors."""
    tf, _ = models
    tf2 = lib.zi_transformer_create_synthetic(*tiny_args(), TINY["ffn"], TINY["t_mid"], TINY["seed"])
    assert tf2, lib.iris_hip_last_error()
    tf2 = ctypes.c_void_p(tf2)
    lat = tl.synth_f32((16, 12, 12), 61)
    cap = tl.synth_f32((20, TINY["cap_dim"]), 62)
    a = forward(lib, tf, lat, 12, 0.5, cap)
    b = forward(lib, tf2, lat, 12, 0.5, cap)
    lib.zi_transformer_free(tf2)
    np.testing.assert_array_equal(a, b)


def test_full_width_reduced_depth(lib, orc):
    """Z-Image-Turbo widths (dim 3840, 30 heads, caption 2560, FFN 10240) with one
    refiner pair and one main layer, 32x32 latents and 100 caption tokens."""
    args = (3840, 30, 1, 1, 2560, 16, 2, F(256.0), axes_arr([32, 48, 48]), 10240, 1024, 5)
    tf = lib.zi_transformer_create_synthetic(*args)
    assert tf, lib.iris_hip_last_error()
    tf = ctypes.c_void_p(tf)
    m = ctypes.c_void_p(orc.orc_zi_create_synth(*args))
    lat = tl.synth_f32((16, 32, 32), 81)
    cap = tl.synth_f32((100, 2560), 82)
    got = forward(lib, tf, lat, 32, 0.7, cap)
    ref = oracle_forward(orc, m, lat, 32, 0.7, cap)
    lib.zi_transformer_free(tf)
    orc.orc_zi_free(m)
    assert tl.rel_l2(got, ref) < 1e-2 and tl.cosine(got, ref) > 0.999


def test_graph_forward_bitwise(lib):
    """Z-Image-Turbo widths with two refiner pairs and one main layer, 128x128
    latent (4096 image tokens) and 512 caption tokens: the captured forward
    equals the profiled forward (the same launches issued one by one) bit
    for bit, over repeated replays."""
    args = (3840, 30, 1, 2, 2560, 16, 2, F(256.0), axes_arr([32, 48, 48]), 10240, 1024, 7)
    tf = lib.zi_transformer_create_synthetic(*args)
    assert tf, lib.iris_hip_last_error()
    tf = ctypes.c_void_p(tf)
    lat = tl.synth_f32((16, 128, 128), 91)
    cap = tl.synth_f32((512, 2560), 92)
    graph = forward(lib, tf, lat, 128, 0.6, cap)
    assert lib.iris_hip_profile_enable(1) == 0
    seq = forward(lib, tf, lat, 128, 0.6, cap)
    assert lib.iris_hip_profile_enable(0) == 0
    np.testing.assert_array_equal(seq, graph)
    for _ in range(3):
        np.testing.assert_array_equal(forward(lib, tf, lat, 128, 0.6, cap), graph)
    lib.zi_transformer_free(tf)
