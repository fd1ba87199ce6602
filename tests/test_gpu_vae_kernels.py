"""The VAE decoder's kernels through the C ABI against float64 numpy
statements of the same operations on the same bf16-rounded inputs:
the implicit-GEMM 3x3 convolution (padding, fused nearest upsample, ragged
pixel counts, cout below the tile width, split-K, each epilogue, the
GroupNorm sums of its epilogue), GroupNorm
+ swish, the bf16 softmax, the transpose, the latent front end and
conv_out with the uint8 conversion."""
import ctypes

import numpy as np
import pytest

import iris_testlib as tl

pytestmark = pytest.mark.gpu
EPI_F32, EPI_BF16, EPI_ADD = 0, 1, 5
vp = ctypes.c_void_p


Conv = tl.Conv3x3


@pytest.fixture(scope="module")
def lib():
    lib = tl.hip()
    lib.iris_hip_gn_stats.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, ctypes.c_int]
    lib.iris_hip_gn_finalize.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp,
                                         ctypes.c_float, vp]
    lib.iris_hip_gn_apply.argtypes = [vp, ctypes.c_int, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
    lib.iris_hip_vae_front.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, ctypes.c_int, vp,
                                       vp]
    lib.iris_hip_softmax_bf16.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int]
    lib.iris_hip_transpose_bf16.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int]
    lib.iris_hip_softmax_scores.argtypes = [vp, ctypes.c_int, vp, ctypes.c_int] + [ctypes.c_int] * 3 + [
        ctypes.c_float, vp, ctypes.c_int, ctypes.c_int, vp, vp]
    lib.iris_hip_vae_conv_out.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
    return lib


def bf(a):
    return tl.bf16_to_f32(tl.to_bf16(a)).astype(np.float64)


def np_conv3(x, w, b, up):
    """x [h][w][cin] (NHWC), w [cout][9][cin]; output [H][W][cout], H = h << up"""
    if up:
        x = x.repeat(2, 0).repeat(2, 1)
    H, W, _ = x.shape
    xp = np.pad(x, ((1, 1), (1, 1), (0, 0)))
    out = np.zeros((H, W, w.shape[0])) + (b if b is not None else 0.0)
    for tap in range(9):
        dy, dx = tap // 3, tap % 3
        out += xp[dy:dy + H, dx:dx + W, :] @ w[:, tap, :].T
    return out


@pytest.mark.parametrize("H,W,cin,cout,up,splits", [
    (20, 20, 64, 128, 0, 1),      # cout 128: a 128-wide tile, ragged last row tile
    (16, 24, 128, 256, 1, 1),     # fused nearest upsample, 256-wide tiles
    (37, 29, 256, 64, 0, 3),      # odd sizes, half-empty 128-wide tile, split-K over 36 K steps
    (8, 64, 512, 512, 1, 4),      # 512 channels (8 K steps per tap), upsampled, split
    (16, 96, 128, 128, 0, 1),     # cout 128 over several row tiles
    (9, 200, 256, 64, 0, 2),      # half-empty 128-wide tiles, ragged M, split-K
    (8, 160, 128, 128, 1, 1),     # 128-wide tiles through the upsample
    (12, 20, 128, 192, 0, 1),     # cout between the tile widths: one part-empty 256-wide tile
])
def test_conv3x3(lib, H, W, cin, cout, up, splits):
    rng = np.random.default_rng(H * W + cin)
    h, w = H >> up, W >> up
    x = rng.standard_normal((h, w, cin)).astype(np.float32)
    wt = (rng.standard_normal((cout, 9, cin)) / np.sqrt(9 * cin)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    ref = np_conv3(bf(x), bf(wt), b.astype(np.float64), up).reshape(H * W, cout)
    dx, dw, db = tl.Dev.of(tl.to_bf16(x)), tl.Dev.of(tl.to_bf16(wt)), tl.Dev.of(b)
    ws_bytes = max(splits, 1) * H * W * cout * 4
    ws = tl.Dev(ws_bytes)

    def run(out, epi, bias=db.ptr):
        c = Conv(dx.ptr, dw.ptr, out.ptr, bias, H, W, cin, cout, up, cout, epi, splits, ws.ptr, ws_bytes)
        assert lib.iris_hip_conv3x3(ctypes.byref(c)) == 0, lib.iris_hip_last_error()
        assert lib.iris_hip_sync() == 0

    o = tl.Dev(H * W * cout * 4)
    run(o, EPI_F32)
    got = o.get(np.float32, (H * W, cout))
    assert tl.rel_l2(got, ref) < 1e-5
    run(o, EPI_F32)
    assert np.array_equal(got, o.get(np.float32, (H * W, cout)))
    o16 = tl.Dev(H * W * cout * 2)
    run(o16, EPI_BF16)
    assert tl.rel_l2(tl.bf16_to_f32(o16.get(np.uint16, (H * W, cout))), ref) < 4e-3
    x0 = rng.standard_normal((H * W, cout)).astype(np.float32)
    ox = tl.Dev.of(x0)
    run(ox, EPI_ADD)
    assert tl.rel_l2(ox.get(np.float32, (H * W, cout)), x0 + ref) < 1e-5


@pytest.mark.parametrize("H,W,cin,cout,splits", [(16, 24, 128, 128, 1), (5, 7, 256, 256, 1), (4, 4, 512, 512, 4)])
def test_conv3x3_stride2(lib, H, W, cin, cout, splits):
    """up = 2: the encoder's downsample, a (2H) x (2W) input padded by one
    zero row and column on the right and bottom, 3x3 stride 2."""
    rng = np.random.default_rng(H * W * cin)
    x = rng.standard_normal((2 * H, 2 * W, cin)).astype(np.float32)
    wt = (rng.standard_normal((cout, 9, cin)) / np.sqrt(9 * cin)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    xp = np.pad(bf(x), ((0, 1), (0, 1), (0, 0)))
    ref = np.zeros((H, W, cout)) + b
    for tap in range(9):
        ky, kx = tap // 3, tap % 3
        ref += xp[ky:ky + 2 * H:2, kx:kx + 2 * W:2, :] @ bf(wt)[:, tap, :].T
    dx, dw, db = tl.Dev.of(tl.to_bf16(x)), tl.Dev.of(tl.to_bf16(wt)), tl.Dev.of(b)
    ws_bytes = splits * H * W * cout * 4
    ws = tl.Dev(ws_bytes)
    o = tl.Dev(H * W * cout * 4)
    c = Conv(dx.ptr, dw.ptr, o.ptr, db.ptr, H, W, cin, cout, 2, cout, EPI_F32, splits, ws.ptr, ws_bytes)
    assert lib.iris_hip_conv3x3(ctypes.byref(c)) == 0, lib.iris_hip_last_error()
    assert lib.iris_hip_sync() == 0
    assert tl.rel_l2(o.get(np.float32, (H, W, cout)), ref) < 1e-5


@pytest.mark.parametrize("H,W,cin,cout,up,epi", [
    (20, 30, 64, 128, 0, EPI_BF16),    # 128-wide tile, ragged last row tile, sums before the bf16 rounding
    (16, 24, 128, 256, 1, EPI_F32),    # 256-wide tile through the upsample
    (13, 21, 64, 512, 0, EPI_ADD),     # two 256-wide column tiles, the updated stream's sums
    (9, 34, 128, 128, 2, EPI_F32),     # stride-2 convolution
])
def test_conv3x3_groupnorm_sums(lib, H, W, cin, cout, up, epi):
    """The GroupNorm sums a convolution forms in its epilogue: per row tile of
    256 output pixels and group of cout / 32 channels, the sum and sum of
    squares of exactly the f32 values it writes (the updated stream for the
    residual add, the values before rounding for bf16), in the layout
    iris_hip_gn_finalize reads, which then gives the statistics pass's scale
    and shift."""
    G = 32
    rng = np.random.default_rng(H * W * cout + up)
    hi = 2 * H if up == 2 else H >> up
    wi = 2 * W if up == 2 else W >> up
    x = rng.standard_normal((hi, wi, cin)).astype(np.float32)
    wt = (rng.standard_normal((cout, 9, cin)) / np.sqrt(9 * cin)).astype(np.float32)
    b = (0.3 * rng.standard_normal(cout)).astype(np.float32)
    dx, dw, db = tl.Dev.of(tl.to_bf16(x)), tl.Dev.of(tl.to_bf16(wt)), tl.Dev.of(b)
    P, tiles = H * W, (H * W + 255) // 256
    part = tl.Dev(tiles * G * 2 * 8)
    x0 = (2.0 + rng.standard_normal((P, cout))).astype(np.float32)
    out = tl.Dev.of(x0) if epi == EPI_ADD else tl.Dev(P * cout * (2 if epi == EPI_BF16 else 4))
    c = Conv(dx.ptr, dw.ptr, out.ptr, db.ptr, H, W, cin, cout, up, cout, epi, 1, None, 0, part.ptr, G)
    assert lib.iris_hip_conv3x3(ctypes.byref(c)) == 0, lib.iris_hip_last_error()
    assert lib.iris_hip_sync() == 0
    sums = part.get(np.float64, (tiles, G, 2))
    if epi == EPI_BF16:
        # the rounded output cannot give the pre-rounding values: the same conv with the f32 epilogue can
        o32 = tl.Dev(P * cout * 4)
        c32 = Conv(dx.ptr, dw.ptr, o32.ptr, db.ptr, H, W, cin, cout, up, cout, EPI_F32, 1, None, 0, None, 0)
        assert lib.iris_hip_conv3x3(ctypes.byref(c32)) == 0 and lib.iris_hip_sync() == 0
        y = o32.get(np.float32, (P, cout)).astype(np.float64)
    else:
        y = out.get(np.float32, (P, cout)).astype(np.float64)
    ypad = np.zeros((tiles * 256, cout))
    ypad[:P] = y
    yt = ypad.reshape(tiles, 256, G, cout // G)
    want = np.stack([yt.sum(axis=(1, 3)), (yt * yt).sum(axis=(1, 3))], axis=-1)
    np.testing.assert_allclose(sums, want, rtol=1e-5, atol=1e-3)
    # iris_hip_gn_finalize over these sums == over the statistics pass's
    gamma, beta = tl.Dev.of((1 + 0.1 * rng.standard_normal(cout)).astype(np.float32)), tl.Dev.of(
        (0.1 * rng.standard_normal(cout)).astype(np.float32))
    ab1, ab2 = tl.Dev(2 * cout * 4), tl.Dev(2 * cout * 4)
    assert lib.iris_hip_gn_finalize(part.ptr, tiles, P, cout, G, gamma.ptr, beta.ptr, ctypes.c_float(1e-6),
                                    ab1.ptr) == 0
    sp = tl.Dev(1024 * G * 2 * 8)
    src = o32 if epi == EPI_BF16 else out
    nblk = lib.iris_hip_gn_stats(src.ptr, 0, P, cout, G, sp.ptr, 1024)
    assert nblk > 0
    assert lib.iris_hip_gn_finalize(sp.ptr, nblk, P, cout, G, gamma.ptr, beta.ptr, ctypes.c_float(1e-6), ab2.ptr) == 0
    assert lib.iris_hip_sync() == 0
    np.testing.assert_allclose(ab1.get(np.float32, (2, cout)), ab2.get(np.float32, (2, cout)), rtol=2e-5, atol=2e-5)


def test_conv3x3_groupnorm_sums_rejects(lib):
    """Sums need groups of a multiple of 4 channels that divide the tile, no
    split-K and an aligned buffer."""
    d = tl.Dev(1 << 22)
    bad = [Conv(d.ptr, d.ptr, d.ptr, None, 16, 16, 64, 128, 0, 128, EPI_F32, 1, None, 0, d.ptr, 64),    # 2 per group
           Conv(d.ptr, d.ptr, d.ptr, None, 16, 16, 64, 96, 0, 96, EPI_F32, 1, None, 0, d.ptr, 32),     # 3 per group
           Conv(d.ptr, d.ptr, d.ptr, None, 16, 16, 64, 128, 0, 128, EPI_F32, 2, d.ptr, 1 << 20, d.ptr, 32),
           Conv(d.ptr, d.ptr, d.ptr, None, 16, 16, 64, 128, 0, 128, EPI_F32, 1, None, 0, d.ptr + 4, 32)]
    for c in bad:
        assert lib.iris_hip_conv3x3(ctypes.byref(c)) != 0


def test_conv3x3_rejects(lib):
    d = tl.Dev(1 << 20)
    bad = [Conv(d.ptr, d.ptr, d.ptr, None, 8, 8, 96, 64, 0, 64, EPI_F32, 1, None, 0),     # cin not 2^k
           Conv(d.ptr, d.ptr, d.ptr, None, 7, 8, 64, 64, 1, 64, EPI_F32, 1, None, 0),     # odd H with upsample
           Conv(d.ptr, d.ptr, d.ptr, None, 8, 8, 64, 64, 0, 64, 3, 1, None, 0),           # SwiGLU epilogue
           Conv(d.ptr, d.ptr, d.ptr, None, 64, 64, 64, 64, 0, 64, EPI_F32, 4, d.ptr, 16)]  # workspace too small
    for c in bad:
        assert lib.iris_hip_conv3x3(ctypes.byref(c)) != 0


@pytest.mark.parametrize("pixels,C,is_bf16,swish", [(1000, 128, 0, 1), (4096, 512, 1, 1), (777, 256, 0, 0)])
def test_group_norm(lib, pixels, C, is_bf16, swish):
    rng = np.random.default_rng(pixels + C)
    x = (rng.standard_normal((pixels, C)) * 3 + 1.5).astype(np.float32)
    xin = bf(x) if is_bf16 else x.astype(np.float64)
    g = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    b = (0.1 * rng.standard_normal(C)).astype(np.float32)
    cpg = C // 32
    xr = xin.reshape(pixels, 32, cpg)
    mean = xr.mean((0, 2), keepdims=True)
    var = ((xr - mean) ** 2).mean((0, 2), keepdims=True)
    y = ((xr - mean) / np.sqrt(var + 1e-4)).reshape(pixels, C) * g + b
    if swish:
        y = y / (1 + np.exp(-y))
    dx = tl.Dev.of(tl.to_bf16(x) if is_bf16 else x)
    dg, db = tl.Dev.of(g), tl.Dev.of(b)
    part, ab = tl.Dev(64 * C * 16), tl.Dev(2 * C * 4)
    dy, raw = tl.Dev(pixels * C * 2), tl.Dev(pixels * C * 2)
    nblk = lib.iris_hip_gn_stats(dx.ptr, is_bf16, pixels, C, 32, part.ptr, 64)
    assert 0 < nblk <= 64, lib.iris_hip_last_error()
    assert lib.iris_hip_gn_finalize(part.ptr, nblk, pixels, C, 32, dg.ptr, db.ptr, 1e-4, ab.ptr) == 0
    assert lib.iris_hip_gn_apply(dx.ptr, is_bf16, ab.ptr, pixels, C, swish, dy.ptr, raw.ptr) == 0
    assert lib.iris_hip_sync() == 0
    got = tl.bf16_to_f32(dy.get(np.uint16, (pixels, C)))
    assert tl.rel_l2(got, y) < 4e-3
    assert np.array_equal(raw.get(np.uint16, (pixels, C)), tl.to_bf16(xin.astype(np.float32)))


@pytest.mark.parametrize("rows,cols,pad", [(3, 1024, 1024), (70, 60, 64), (5, 16384, 16384), (4, 6000, 6016),
                                           (3, 4096, 4160), (2, 20000, 20032)])
def test_softmax_bf16(lib, rows, cols, pad):
    """Row softmax to bf16 against float64, up to the 1024x1024 bottleneck's
    16384 columns and beyond, with ragged and padded rows (padding columns
    written as zero)."""
    rng = np.random.default_rng(cols)
    s = (rng.standard_normal((rows, pad)) * 4).astype(np.float32)
    ds, dp = tl.Dev.of(s), tl.Dev(rows * pad * 2)
    assert lib.iris_hip_softmax_bf16(dp.ptr, pad, pad, ds.ptr, pad, rows, cols) == 0, lib.iris_hip_last_error()
    assert lib.iris_hip_sync() == 0
    got = tl.bf16_to_f32(dp.get(np.uint16, (rows, pad)))
    e = np.exp(s[:, :cols].astype(np.float64) - s[:, :cols].max(1, keepdims=True))
    ref = e / e.sum(1, keepdims=True)
    assert tl.rel_l2(got[:, :cols], ref) < 4e-3
    assert not got[:, cols:].any()


@pytest.mark.parametrize("M,N,d,scale", [(300, 1000, 512, 1.0), (512, 512, 128, 0.125), (1024, 16384, 512, 1.0),
                                         (77, 40, 64, 0.3)])
def test_softmax_scores(lib, M, N, d, scale):
    """Softmax over scaled products in two passes (tile row statistics, then
    probabilities): against float64 softmax(scale q k^T) within bf16
    rounding, rows summing to 1, zeros in the padding columns; ragged rows
    and columns (edge tiles), the 1024x1024 bottleneck's 16384 keys, and
    fewer keys than one tile. Repeats bit for bit."""
    rng = np.random.default_rng(M + N + d)
    ldq, ldk = 3 * d, 3 * d
    qkv = bf(rng.standard_normal((max(M, N), ldq), np.float32) * (2.0 / np.sqrt(d)) ** 0.5)
    q, k = qkv[:M, :d], qkv[:N, d:2 * d]
    pad = (N + 63) // 64 * 64
    tiles = (N + 255) // 256
    dqkv = tl.Dev.of(tl.to_bf16(qkv))
    dp, dst, drow = tl.Dev(M * pad * 2), tl.Dev(M * tiles * 8), tl.Dev(M * 8)
    outs = []
    for _ in range(2):
        assert lib.iris_hip_memset(dp.ptr, 0xff, M * pad * 2) == 0
        assert lib.iris_hip_softmax_scores(dqkv.ptr, ldq, dqkv.ptr + d * 2, ldk, M, N, d, scale, dp.ptr, pad, pad,
                                           dst.ptr, drow.ptr) == 0, lib.iris_hip_last_error()
        assert lib.iris_hip_sync() == 0
        outs.append(dp.get(np.uint16, (M, pad)))
    assert np.array_equal(outs[0], outs[1]), "not repeatable"
    got = tl.bf16_to_f32(outs[0])
    s = scale * (q.astype(np.float64) @ k.astype(np.float64).T)
    e = np.exp(s - s.max(1, keepdims=True))
    ref = e / e.sum(1, keepdims=True)
    assert tl.rel_l2(got[:, :N], ref) < 4e-3
    assert np.abs(got[:, :N].sum(1) - 1.0).max() < 2e-2
    assert not got[:, N:].any()
    print(f"softmax_scores {M}x{N}x{d}: rel_l2 {tl.rel_l2(got[:, :N], ref):.2e}")


def test_softmax_scores_rejects(lib):
    """Shapes the two passes do not take: padding past the last tile, d not
    a multiple of 64, misaligned statistics."""
    buf, st = tl.Dev(1 << 20), tl.Dev(4096)
    call = lib.iris_hip_softmax_scores
    assert call(buf.ptr, 192, buf.ptr, 192, 8, 100, 64, 1.0, buf.ptr, 512, 512, st.ptr, st.ptr) != 0
    assert call(buf.ptr, 192, buf.ptr, 192, 8, 100, 48, 1.0, buf.ptr, 128, 128, st.ptr, st.ptr) != 0
    assert call(buf.ptr, 192, buf.ptr, 192, 8, 100, 64, 1.0, buf.ptr, 128, 128, st.ptr + 4, st.ptr) != 0
    assert call(buf.ptr, 192, buf.ptr, 192, 8, 100, 64, 1.0, buf.ptr, 128, 90, st.ptr, st.ptr) != 0


def test_transpose_bf16(lib):
    rng = np.random.default_rng(0)
    rows, cols, ld, pad = 100, 512, 1536, 128
    src = rng.integers(0, 65535, (rows, ld), dtype=np.uint16)
    ds, dd = tl.Dev.of(src), tl.Dev(cols * pad * 2)
    assert lib.iris_hip_transpose_bf16(dd.ptr, pad, pad, ds.ptr + 1024 * 2, ld, rows, cols) == 0
    assert lib.iris_hip_sync() == 0
    got = dd.get(np.uint16, (cols, pad))
    assert np.array_equal(got[:, :rows], src[:, 1024:1024 + cols].T)
    assert not got[:, rows:].any()


@pytest.mark.parametrize("z,divide,pq", [(32, 0, 1), (16, 1, 0)])
def test_vae_front(lib, z, divide, pq):
    rng = np.random.default_rng(z)
    h, w = 5, 7
    lat = rng.standard_normal((4 * z, h, w)).astype(np.float32)
    sc = (1 + 0.2 * rng.random(4 * z)).astype(np.float32)
    sh = (0.1 * rng.standard_normal(4 * z)).astype(np.float32)
    pqw = (rng.standard_normal((z, z)) / np.sqrt(z)).astype(np.float32)
    pqb = (0.1 * rng.standard_normal(z)).astype(np.float32)
    x = lat / sc[:, None, None] + sh[:, None, None] if divide else lat * sc[:, None, None] + sh[:, None, None]
    u = np.zeros((2 * h, 2 * w, z))
    for c in range(z):
        for pi in range(2):
            for pj in range(2):
                u[pi::2, pj::2, c] = x[c * 4 + pi * 2 + pj]
    if pq:
        u = u @ pqw.T.astype(np.float64) + pqb
    d = [tl.Dev.of(a) for a in (lat, sc, sh, pqw, pqb)]
    out = tl.Dev(4 * h * w * 64 * 2)
    assert lib.iris_hip_vae_front(out.ptr, d[0].ptr, z, h, w, d[1].ptr, d[2].ptr, divide,
                                  d[3].ptr if pq else None, d[4].ptr if pq else None) == 0
    assert lib.iris_hip_sync() == 0
    got = tl.bf16_to_f32(out.get(np.uint16, (2 * h, 2 * w, 64)))
    assert tl.rel_l2(got[..., :z], u) < 4e-3
    assert not got[..., z:].any()


@pytest.mark.parametrize("H,W,cin", [
    (33, 47, 128),   # the decoder's 128 channels over ragged 16 x 16 output tiles (LDS-tiled kernel)
    (17, 16, 64),    # two 32-channel chunks, one ragged tile row
    (9, 21, 24),     # channels not a multiple of 32: the one-thread-per-pixel kernel
])
def test_conv_out(lib, H, W, cin):
    rng = np.random.default_rng(H * W + cin)
    g = rng.standard_normal((H, W, cin)).astype(np.float32)
    w = (0.5 * rng.standard_normal((3, cin, 3, 3)) / np.sqrt(9 * cin)).astype(np.float32)
    b = (0.1 * rng.standard_normal(3)).astype(np.float32)
    wt = np.zeros((9, cin, 4), np.float32)
    for o in range(3):
        wt[:, :, o] = w[o].reshape(cin, 9).T
    ref = np_conv3(bf(g), w.reshape(3, cin, 9).transpose(0, 2, 1).astype(np.float64), b, 0)   # [H][W][3]
    dg, dw, db = tl.Dev.of(tl.to_bf16(g)), tl.Dev.of(wt), tl.Dev.of(np.r_[b, 0].astype(np.float32))
    rgb, f = tl.Dev(H * W * 3), tl.Dev(3 * H * W * 4)
    assert lib.iris_hip_vae_conv_out(rgb.ptr, f.ptr, dg.ptr, H, W, cin, dw.ptr, db.ptr) == 0
    assert lib.iris_hip_sync() == 0
    got = f.get(np.float32, (3, H, W))
    assert tl.rel_l2(got, ref.transpose(2, 0, 1)) < 1e-5
    u8 = rgb.get(np.uint8, (H, W, 3))
    v = np.clip((got.transpose(1, 2, 0) + 1.0) * 0.5 * 255.0, 0, 255)
    assert np.array_equal(u8, (v + 0.5).astype(np.uint8))
