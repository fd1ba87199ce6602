"""VAE decoder oracle (oracle/orc_vae.c) against the reference's own
iris_vae_decode (iris_vae.c, compiled from its sources into oracle/_ref) on
random-init decoder files in the diffusers layout (Flux.2: z=32, batch-norm
denormalization and post_quant_conv, f32 tensors; Z-Image: z=16,
x / scaling + shift, bf16 tensors), and the front end against a float64 numpy
statement of denormalize -> unpatchify -> post_quant_conv -> conv_in. CPU only."""
import ctypes
import os

import numpy as np
import pytest

import iris_testlib as tl

ZI_SCALE, ZI_SHIFT = 0.3611, 0.1159


@pytest.fixture(scope="module")
def orc():
    return tl.oracle()


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    d = tmp_path_factory.mktemp("vae")
    flux, zi = str(d / "flux_vae.safetensors"), str(d / "zimage_vae.safetensors")
    tl.write_vae_file(flux, z=32, flux=True, seed=1)
    tl.write_vae_file(zi, z=16, flux=False, seed=2, bf16=True)
    return {"flux": (flux, 32, 0.0, 0.0), "zimage": (zi, 16, ZI_SCALE, ZI_SHIFT)}


def latent(z, lh, lw, seed):
    return np.random.default_rng(seed).standard_normal((4 * z, lh, lw)).astype(np.float32)


def oracle_decode(orc, v, lat, stop=-1, channels=3):
    lh, lw = lat.shape[1:]
    rgb = np.zeros((16 * lh, 16 * lw, 3), np.uint8)
    f32 = np.zeros(channels * 256 * lh * lw * 4 if stop >= 0 else 3 * 256 * lh * lw, np.float32)
    rc = orc.orc_vae_decode(v, tl.fptr(np.ascontiguousarray(lat)), lh, lw, rgb.ctypes.data, tl.fptr(f32), stop)
    assert rc >= 0
    return rgb, f32, rc


@pytest.mark.skipif(not os.path.exists(tl.REF_SO), reason="reference build (oracle/_ref) not present")
@pytest.mark.parametrize("kind,lh,lw", [("flux", 2, 3), ("zimage", 3, 2), ("flux", 1, 4)])
def test_oracle_vs_reference(orc, files, kind, lh, lw):
    path, z, sc, sh = files[kind]
    ref = tl.ref()
    sf = ctypes.c_void_p(ref.safetensors_open(path.encode()))
    assert sf.value
    rv = ctypes.c_void_p(ref.iris_vae_load_safetensors_ex(sf, z, sc, sh))
    ref.safetensors_close(sf)
    assert rv.value
    lat = latent(z, lh, lw, 10 * lh + lw)
    img = ref.iris_vae_decode(rv, tl.fptr(lat), 1, lh, lw)
    assert img
    im = img.contents
    assert (im.width, im.height, im.channels) == (16 * lw, 16 * lh, 3)
    want = np.ctypeslib.as_array(im.data, shape=(im.height, im.width, 3)).copy()
    ref.iris_image_free(img)
    ref.iris_vae_free(rv)
    v = ctypes.c_void_p(orc.orc_vae_load(path.encode(), z, sc, sh))
    assert v.value
    got, f32, _ = oracle_decode(orc, v, lat)
    orc.orc_vae_free(v)
    assert 5 < want.std() and 0.02 < np.mean((want > 0) & (want < 255))   # not saturated
    diff = np.abs(got.astype(int) - want.astype(int))
    assert diff.max() <= 1 and diff.mean() < 0.01, (diff.max(), diff.mean())


def np_conv(x, w, b):
    """float64 'same' convolution, x [C][H][W], w [O][C][k][k]"""
    k = w.shape[2]
    p = k // 2
    xp = np.pad(x, ((0, 0), (p, p), (p, p)))
    H, W = x.shape[1:]
    out = np.zeros((w.shape[0], H, W)) + b[:, None, None]
    for ky in range(k):
        for kx in range(k):
            out += np.einsum("oc,chw->ohw", w[:, :, ky, kx], xp[:, ky:ky + H, kx:kx + W])
    return out


@pytest.mark.parametrize("kind", ["flux", "zimage"])
def test_front_end_known_answer(orc, files, kind):
    """Stage 0 (conv_in output, 512 channels at 1/8 resolution) against numpy:
    pins the denormalization branch, the unpatchify channel order and the
    post_quant_conv of the oracle independently of the reference."""
    path, z, sc, sh = files[kind]
    W = read_all(path)
    lh, lw = 3, 4
    lat = latent(z, lh, lw, 5).astype(np.float64)
    if kind == "flux":
        x = lat * np.sqrt(W["bn.running_var"] + 1e-4)[:, None, None] + W["bn.running_mean"][:, None, None]
    else:
        x = lat / ZI_SCALE + ZI_SHIFT
    u = np.zeros((z, 2 * lh, 2 * lw))
    for c in range(z):
        for pi in range(2):
            for pj in range(2):
                u[c, pi::2, pj::2] = x[c * 4 + pi * 2 + pj]
    if kind == "flux":
        u = np_conv(u, W["post_quant_conv.weight"], W["post_quant_conv.bias"])
    want = np_conv(u, W["decoder.conv_in.weight"], W["decoder.conv_in.bias"])
    v = ctypes.c_void_p(orc.orc_vae_load(path.encode(), z, sc, sh))
    _, f32, ch = oracle_decode(orc, v, lat.astype(np.float32), stop=0, channels=512)
    orc.orc_vae_free(v)
    assert ch == 512
    got = f32[:512 * 4 * lh * lw].reshape(512, 2 * lh, 2 * lw)
    assert tl.rel_l2(got, want) < 1e-5


def read_all(path):
    import json
    import struct
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        hdr = json.loads(f.read(n))
        data = f.read()
    out = {}
    for k, v in hdr.items():
        if k == "__metadata__":
            continue
        a, b = v["data_offsets"]
        if v["dtype"] == "F32":
            arr = np.frombuffer(data[a:b], np.float32).astype(np.float64)
        else:
            arr = tl.bf16_to_f32(np.frombuffer(data[a:b], np.uint16)).astype(np.float64)
        out[k] = arr.reshape(v["shape"])
    return out


def test_deterministic_and_synthetic(orc):
    """The synthetic model decodes deterministically to a non-degenerate image."""
    v = ctypes.c_void_p(orc.orc_vae_create_synth(32, 0.0, 0.0, 7))
    assert v.value
    lat = latent(32, 2, 2, 3)
    a, fa, _ = oracle_decode(orc, v, lat)
    b, fb, _ = oracle_decode(orc, v, lat)
    orc.orc_vae_free(v)
    assert np.array_equal(a, b) and np.array_equal(fa, fb)
    assert np.all(np.isfinite(fa)) and a.std() > 5


# ----------------------------------------------------------------- encoder

@pytest.fixture(scope="module")
def enc_files(tmp_path_factory):
    d = tmp_path_factory.mktemp("vae_enc")
    flux, zi = str(d / "flux_vae.safetensors"), str(d / "zimage_vae.safetensors")
    tl.write_vae_file(flux, z=32, flux=True, seed=3, encoder=True)
    tl.write_vae_file(zi, z=16, flux=False, seed=4, bf16=True, encoder=True)
    return {"flux": (flux, 32, 0.0, 0.0), "zimage": (zi, 16, ZI_SCALE, ZI_SHIFT)}


def oracle_encode(orc, v, img, z):
    H, W = img.shape[1:]
    lat = np.zeros((4 * z, H // 16, W // 16), np.float32)
    assert orc.orc_vae_encode(v, tl.fptr(np.ascontiguousarray(img)), H, W, tl.fptr(lat)) == 0
    return lat


def test_encode_golden_checksum(orc, tmp_path):
    """The reference test's own golden value (debug/test_vae.c:292-309): the
    LCG-seeded VAE of its build_vae, a 32x32 input from seed 7, checksum
    sum(latent[i] * (i % 13 + 1)) = 29.091131 +- 0.2."""
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import vae_lcg
    path = str(tmp_path / "lcg_vae.safetensors")
    tl.write_safetensors(path, vae_lcg.build_vae(seed=1, z=32, with_quant=True))
    v = ctypes.c_void_p(orc.orc_vae_load(path.encode(), 32, 0.0, 0.0))
    assert v.value
    lat = oracle_encode(orc, v, vae_lcg.make_input(7, 32, 32), 32)
    orc.orc_vae_free(v)
    assert lat.shape == (128, 2, 2)
    assert abs(vae_lcg.checksum(lat) - vae_lcg.GOLDEN_ENCODE_CHECKSUM) < vae_lcg.GOLDEN_TOL, vae_lcg.checksum(lat)


@pytest.mark.skipif(not os.path.exists(tl.REF_SO), reason="reference build (oracle/_ref) not present")
@pytest.mark.parametrize("kind,H,W", [("flux", 32, 48), ("zimage", 48, 32)])
def test_encode_vs_reference(orc, enc_files, kind, H, W):
    path, z, sc, sh = enc_files[kind]
    ref = tl.ref()
    sf = ctypes.c_void_p(ref.safetensors_open(path.encode()))
    rv = ctypes.c_void_p(ref.iris_vae_load_safetensors_ex(sf, z, sc, sh))
    ref.safetensors_close(sf)
    assert rv.value
    img = np.random.default_rng(H + W).uniform(-1, 1, (3, H, W)).astype(np.float32)
    oh, ow = ctypes.c_int(), ctypes.c_int()
    p = ref.iris_vae_encode(rv, tl.fptr(img), 1, H, W, ctypes.byref(oh), ctypes.byref(ow))
    assert p and (oh.value, ow.value) == (H // 16, W // 16)
    want = np.ctypeslib.as_array(p, shape=(4 * z, oh.value, ow.value)).copy()
    ctypes.CDLL(None).free(ctypes.cast(p, ctypes.c_void_p))
    ref.iris_vae_free(rv)
    v = ctypes.c_void_p(orc.orc_vae_load(path.encode(), z, sc, sh))
    got = oracle_encode(orc, v, img, z)
    orc.orc_vae_free(v)
    assert np.all(np.isfinite(want)) and want.std() > 0.1
    assert tl.rel_l2(got, want) < 1e-4
