"""The reference's host-pointer math API (iris_kernels.h:42-312) served by the
HIP build, through its C ABI (needs an MI355X).

References are float64 numpy statements of each operation; where the
reference's loop order defines a layout (patchify, conv weight order) the
reference here is a reshape/transposition, a formulation independent of the
kernel's index arithmetic. f32 products must beat plain bf16 by two orders of
magnitude: rel-L2 <= 3e-5 (bf16 operands alone give ~3e-3), which pins the
three-term split.
"""
import ctypes

import numpy as np
import pytest

import iris_testlib as tl

pytestmark = pytest.mark.gpu
FP = tl.FP
c_int, c_float = ctypes.c_int, ctypes.c_float


@pytest.fixture(scope="module")
def lib():
    lib = tl.hip()
    vp = ctypes.c_void_p
    sig = {
        "iris_add": [vp, vp, vp, c_int],
        "iris_add_inplace": [vp, vp, c_int],
        "iris_mul_inplace": [vp, vp, c_int],
        "iris_axpy": [vp, c_float, vp, c_int],
        "iris_silu": [vp, c_int],
        "iris_silu_mul": [vp, vp, c_int],
        "iris_copy": [vp, vp, c_int],
        "iris_matmul": [vp, vp, vp, c_int, c_int, c_int],
        "iris_matmul_t": [vp, vp, vp, c_int, c_int, c_int],
        "iris_linear": [vp, vp, vp, vp, c_int, c_int, c_int],
        "iris_linear_nobias": [vp, vp, vp, c_int, c_int, c_int],
        "iris_linear_nobias_bf16": [vp, vp, vp, c_int, c_int, c_int],
        "iris_conv2d": [vp, vp, vp, vp] + [c_int] * 9,
        "iris_rms_norm": [vp, vp, vp, c_int, c_int, c_float],
        "iris_group_norm": [vp, vp, vp, vp] + [c_int] * 5 + [c_float],
        "iris_batch_norm": [vp] * 6 + [c_int] * 4 + [c_float],
        "iris_softmax": [vp, c_int, c_int],
        "iris_softmax_cpu": [vp, c_int, c_int],
        "iris_attention": [vp] * 4 + [c_int] * 5 + [c_float],
        "iris_flash_attention": [vp] * 4 + [c_int] * 4 + [c_float],
        "iris_upsample_nearest": [vp, vp] + [c_int] * 6,
        "iris_patchify": [vp, vp] + [c_int] * 5,
        "iris_unpatchify": [vp, vp] + [c_int] * 5,
        "iris_randn": [vp, c_int],
        "iris_rand": [vp, c_int],
        "iris_rng_seed": [ctypes.c_uint64],
    }
    for name, args in sig.items():
        getattr(lib, name).argtypes = args
        getattr(lib, name).restype = None
    lib.iris_random_uniform.restype = c_float
    lib.iris_random_normal.restype = c_float
    return lib


def p(a):
    return a.ctypes.data


def rel_l2(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(got, np.float64) - ref) / max(np.linalg.norm(ref), 1e-30))


def f32(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


# ---------------------------------------------------------------- elementwise

def test_elementwise(lib):
    rng = np.random.default_rng(0)
    n = 100003
    a, b = f32(rng, n), f32(rng, n)
    out = np.empty(n, np.float32)
    lib.iris_add(p(out), p(a), p(b), n)
    np.testing.assert_array_equal(out, a + b)
    x = a.copy()
    lib.iris_add_inplace(p(x), p(b), n)
    np.testing.assert_array_equal(x, a + b)
    x = a.copy()
    lib.iris_mul_inplace(p(x), p(b), n)
    np.testing.assert_array_equal(x, a * b)
    x = a.copy()
    lib.iris_axpy(p(x), 0.375, p(b), n)
    np.testing.assert_allclose(x, a + np.float32(0.375) * b, rtol=1e-6, atol=1e-7)
    x = a.copy()
    lib.iris_silu(p(x), n)
    ad = a.astype(np.float64)
    np.testing.assert_allclose(x, ad / (1 + np.exp(-ad)), rtol=2e-6, atol=1e-7)
    x = a.copy()
    lib.iris_silu_mul(p(x), p(b), n)
    np.testing.assert_allclose(x, ad / (1 + np.exp(-ad)) * b, rtol=4e-6, atol=1e-7)
    y = np.empty(n, np.float32)
    lib.iris_copy(p(y), p(a), n)
    np.testing.assert_array_equal(y, a)
    lib.iris_add(p(out), p(a), p(b), 0)   # empty: no-op


# ---------------------------------------------------------------- products

@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (37, 100, 53), (300, 3072, 260), (512, 64, 1024), (5, 7680, 17)])
def test_matmul_family(lib, M, K, N):
    rng = np.random.default_rng(M + K + N)
    A = f32(rng, M, K)
    Bt = f32(rng, N, K, scale=0.05)
    bias = f32(rng, N)
    ref_t = A.astype(np.float64) @ Bt.astype(np.float64).T
    C = np.empty((M, N), np.float32)
    lib.iris_matmul_t(p(C), p(A), p(Bt), M, K, N)
    assert rel_l2(C, ref_t) < 3e-5
    B = np.ascontiguousarray(Bt.T)
    C2 = np.empty((M, N), np.float32)
    lib.iris_matmul(p(C2), p(A), p(B), M, K, N)
    assert rel_l2(C2, ref_t) < 3e-5
    lib.iris_linear(p(C), p(A), p(Bt), p(bias), M, K, N)
    assert rel_l2(C, ref_t + bias) < 3e-5
    lib.iris_linear(p(C), p(A), p(Bt), None, M, K, N)
    assert rel_l2(C, ref_t) < 3e-5
    lib.iris_linear_nobias(p(C), p(A), p(Bt), M, K, N)
    assert rel_l2(C, ref_t) < 3e-5
    if M * K > 64:
        # the bound is far below what bf16 operands would give
        plain = tl.bf16_to_f32(tl.to_bf16(A)).astype(np.float64) @ tl.bf16_to_f32(tl.to_bf16(Bt)).astype(np.float64).T
        assert rel_l2(plain, ref_t) > 10 * 3e-5


@pytest.mark.parametrize("M,K,N", [(3, 64, 5), (77, 3072, 300), (256, 130, 256)])
def test_linear_nobias_bf16(lib, M, K, N):
    rng = np.random.default_rng(K)
    x = f32(rng, M, K)
    W16 = tl.to_bf16(f32(rng, N, K, scale=0.05))
    ref = x.astype(np.float64) @ tl.bf16_to_f32(W16).astype(np.float64).T
    y = np.empty((M, N), np.float32)
    lib.iris_linear_nobias_bf16(p(y), p(x), p(W16), M, K, N)
    assert rel_l2(y, ref) < 3e-5


def conv_ref(x, w, b, stride, pad):
    B, C, H, W = x.shape
    O, _, kh, kw = w.shape
    xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    oh, ow = (H + 2 * pad - kh) // stride + 1, (W + 2 * pad - kw) // stride + 1
    out = np.zeros((B, O, oh, ow))
    for i in range(kh):
        for j in range(kw):
            patch = xp[:, :, i:i + stride * oh:stride, j:j + stride * ow:stride]     # [B, C, oh, ow]
            out += np.einsum("bchw,oc->bohw", patch, w[:, :, i, j].astype(np.float64))
    if b is not None:
        out += b[None, :, None, None]
    return out


@pytest.mark.parametrize("B,C,O,H,W,k,s,pad,bias", [(2, 3, 5, 9, 11, 3, 1, 1, True), (1, 4, 8, 16, 16, 3, 2, 0, False),
                                                    (1, 16, 7, 6, 5, 1, 1, 0, True), (1, 128, 128, 40, 40, 3, 1, 1,
                                                                                        True)])
def test_conv2d(lib, B, C, O, H, W, k, s, pad, bias):
    rng = np.random.default_rng(C * 31 + O)
    x = f32(rng, B, C, H, W)
    w = f32(rng, O, C, k, k, scale=0.1)
    b = f32(rng, O) if bias else None
    ref = conv_ref(x, w, b, s, pad)
    out = np.empty(ref.shape, np.float32)
    lib.iris_conv2d(p(out), p(x), p(w), p(b) if bias else None, B, C, O, H, W, k, k, s, pad)
    assert rel_l2(out, ref) < 3e-5


# ---------------------------------------------------------------- normalisation, softmax

def test_rms_norm(lib):
    rng = np.random.default_rng(3)
    for rows, cols in [(5, 3072), (17, 7), (3, 5000)]:
        x, w = f32(rng, rows, cols), f32(rng, cols)
        xd = x.astype(np.float64)
        ref = xd / np.sqrt((xd * xd).mean(1, keepdims=True) + 1e-6) * w
        out = np.empty_like(x)
        lib.iris_rms_norm(p(out), p(x), p(w), rows, cols, 1e-6)
        np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)


def test_group_and_batch_norm(lib):
    rng = np.random.default_rng(4)
    B, C, H, W, G = 2, 64, 7, 9, 32
    x = f32(rng, B, C, H, W) * 3 + 1
    g, b = f32(rng, C), f32(rng, C)
    xd = x.astype(np.float64).reshape(B, G, -1)
    n = ((xd - xd.mean(-1, keepdims=True)) / np.sqrt(xd.var(-1, keepdims=True) + 1e-6)).reshape(B, C, H, W)
    ref = n * g[None, :, None, None] + b[None, :, None, None]
    out = np.empty_like(x)
    lib.iris_group_norm(p(out), p(x), p(g), p(b), B, C, H, W, G, 1e-6)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=2e-5)
    mean, var = f32(rng, C), np.abs(f32(rng, C)) + 0.5
    ref = ((x - mean[None, :, None, None]) / np.sqrt(var[None, :, None, None].astype(np.float64) + 1e-5)
           * g[None, :, None, None] + b[None, :, None, None])
    lib.iris_batch_norm(p(out), p(x), p(mean), p(var), p(g), p(b), B, C, H, W, 1e-5)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=2e-5)
    ref = (x - mean[None, :, None, None]) / np.sqrt(var[None, :, None, None].astype(np.float64) + 1e-5)
    lib.iris_batch_norm(p(out), p(x), p(mean), p(var), None, None, B, C, H, W, 1e-5)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=2e-5)


@pytest.mark.parametrize("fn", ["iris_softmax", "iris_softmax_cpu"])
def test_softmax(lib, fn):
    rng = np.random.default_rng(5)
    for rows, cols in [(7, 1), (33, 4608), (3, 100)]:
        x = f32(rng, rows, cols, scale=20.0)
        xd = x.astype(np.float64)
        e = np.exp(xd - xd.max(1, keepdims=True))
        ref = e / e.sum(1, keepdims=True)
        getattr(lib, fn)(p(x), rows, cols)
        np.testing.assert_allclose(x, ref, rtol=1e-5, atol=1e-7)


# ---------------------------------------------------------------- attention

def attn_ref(q, k, v, scale):
    s = np.einsum("...qd,...kd->...qk", q.astype(np.float64), k.astype(np.float64)) * scale
    e = np.exp(s - s.max(-1, keepdims=True))
    return np.einsum("...qk,...kd->...qd", e / e.sum(-1, keepdims=True), v.astype(np.float64))


def test_attention_bhsd(lib):
    rng = np.random.default_rng(6)
    B, H, Sq, Sk, D = 2, 3, 17, 29, 40
    q, k, v = f32(rng, B, H, Sq, D), f32(rng, B, H, Sk, D), f32(rng, B, H, Sk, D)
    out = np.empty_like(q)
    lib.iris_attention(p(out), p(q), p(k), p(v), B, H, Sq, Sk, D, D ** -0.5)
    np.testing.assert_allclose(out, attn_ref(q, k, v, D ** -0.5), rtol=1e-4, atol=2e-6)


@pytest.mark.parametrize("Sq,Sk,H,D", [(33, 70, 2, 64), (200, 600, 4, 128)])
def test_flash_attention_seq_major(lib, Sq, Sk, H, D):
    rng = np.random.default_rng(Sq)
    q, k, v = f32(rng, Sq, H * D), f32(rng, Sk, H * D), f32(rng, Sk, H * D)
    out = np.empty_like(q)
    lib.iris_flash_attention(p(out), p(q), p(k), p(v), Sq, Sk, H, D, D ** -0.5)
    hq = q.reshape(Sq, H, D).transpose(1, 0, 2)
    hk = k.reshape(Sk, H, D).transpose(1, 0, 2)
    hv = v.reshape(Sk, H, D).transpose(1, 0, 2)
    ref = attn_ref(hq, hk, hv, D ** -0.5).transpose(1, 0, 2).reshape(Sq, H * D)
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=2e-6)


# ---------------------------------------------------------------- reshapes (bit-exact)

def test_upsample_patchify_roundtrip(lib):
    rng = np.random.default_rng(7)
    B, C, H, W = 2, 3, 6, 10
    x = f32(rng, B, C, H, W)
    up = np.empty((B, C, H * 2, W * 3), np.float32)
    lib.iris_upsample_nearest(p(up), p(x), B, C, H, W, 2, 3)
    np.testing.assert_array_equal(up, x.repeat(2, axis=2).repeat(3, axis=3))
    pch = 2
    pt = np.empty((B, C * pch * pch, H // pch, W // pch), np.float32)
    lib.iris_patchify(p(pt), p(x), B, C, H, W, pch)
    ref = x.reshape(B, C, H // pch, pch, W // pch, pch).transpose(0, 1, 3, 5, 2, 4).reshape(pt.shape)
    np.testing.assert_array_equal(pt, ref)
    back = np.empty_like(x)
    lib.iris_unpatchify(p(back), p(pt), B, C, H // pch, W // pch, pch)
    np.testing.assert_array_equal(back, x)


# ---------------------------------------------------------------- RNG and batching

def test_rand_fills_follow_the_stream(lib):
    lib.iris_rng_seed(1234)
    a = np.empty(64, np.float32)
    lib.iris_randn(p(a), 64)
    lib.iris_rng_seed(1234)
    b = np.array([lib.iris_random_normal() for _ in range(64)], np.float32)
    np.testing.assert_array_equal(a, b)
    lib.iris_rng_seed(99)
    u = np.empty(1000, np.float32)
    lib.iris_rand(p(u), 1000)
    assert u.min() >= 0.0 and u.max() < 1.0 and abs(u.mean() - 0.5) < 0.05
    lib.iris_gpu_begin_batch()
    lib.iris_gpu_end_batch()


# ---------------------------------------------------------------- callbacks

SUBSTEP = ctypes.CFUNCTYPE(None, ctypes.c_int, ctypes.c_int, ctypes.c_int)
STEP = ctypes.CFUNCTYPE(None, ctypes.c_int, ctypes.c_int)


def test_progress_callbacks(lib):
    """Substeps fire per block in order (iris_transformer_flux.c:4085-4086,
    :4185-4186, :4315-4316) and the step callback fires at each step start
    (iris_sample.c:345-347)."""
    seen, steps = [], []
    sub_cb = SUBSTEP(lambda t, i, n: seen.append((t, i, n)))
    step_cb = STEP(lambda s, n: steps.append((s, n)))
    sub_ptr = ctypes.c_void_p.in_dll(lib, "iris_substep_callback")
    step_ptr = ctypes.c_void_p.in_dll(lib, "iris_step_callback")
    tf = ctypes.c_void_p(lib.iris_transformer_create_synthetic(256, 2, 2, 3, 64, 128, 3.0, 2000.0, 7))
    assert tf.value, lib.iris_hip_last_error()
    try:
        sub_ptr.value = ctypes.cast(sub_cb, ctypes.c_void_p).value
        step_ptr.value = ctypes.cast(step_cb, ctypes.c_void_p).value
        rng = np.random.default_rng(8)
        h = w = 4
        z = f32(rng, 128, h, w)
        txt = f32(rng, 5, 64)
        sched = np.array([1.0, 0.5, 0.0], np.float32)
        out = lib.iris_sample_euler(tf, None, tl.fptr(z), 1, 128, h, w, tl.fptr(txt), 5, tl.fptr(sched), 2, None)
        assert out, lib.iris_hip_last_error()
        ctypes.CDLL(None).free(ctypes.c_void_p(out))
    finally:
        sub_ptr.value = None
        step_ptr.value = None
        lib.iris_transformer_free(tf)
    assert steps == [(1, 2), (2, 2)]
    one = [(0, i, 2) for i in range(2)] + [(1, i, 3) for i in range(3)] + [(2, 0, 1)]
    assert seen == one * 2


# ---------------------------------------------------------------- the reference's own known answers

def test_reference_known_answers(lib):
    """The known-answer cases of debug/test_kernels.c:54-305 (inputs, expected
    values and tolerances as the reference states them), through the HIP build."""
    keep = []

    def a(*v):
        """a float32 array kept alive for the whole test (its address is passed to C)"""
        keep.append(np.array(v, np.float32))
        return keep[-1]

    x = a(1, 2, 3, 4)                                        # :54-64
    lib.iris_softmax_cpu(p(x), 1, 4)
    assert abs(x.sum() - 1) < 1e-5 and np.all(x > 0) and x[3] > x[2] > x[1] > x[0]
    x = a(5, 5, 5, 5)                                        # :66-74
    lib.iris_softmax_cpu(p(x), 1, 4)
    np.testing.assert_allclose(x, 0.25, atol=1e-5)
    x = a(1000, 1001, 1002)                                  # :76-83
    lib.iris_softmax_cpu(p(x), 1, 3)
    assert abs(x.sum() - 1) < 1e-5 and np.all(np.isfinite(x))
    x = a(1, 2, 3, 1)                                        # :85-94
    lib.iris_softmax_cpu(p(x), 2, 2)
    assert abs(x[0] + x[1] - 1) < 1e-5 and abs(x[2] + x[3] - 1) < 1e-5 and x[2] > x[3]
    x = a(0, 1)                                              # :96-103
    lib.iris_softmax_cpu(p(x), 1, 2)
    e = np.exp(np.float32(1))
    np.testing.assert_allclose(x, [1 / (1 + e), e / (1 + e)], atol=1e-5)

    out = np.empty(2, np.float32)                            # :109-120
    lib.iris_rms_norm(p(out), p(a(3, 4)), p(a(1, 1)), 1, 2, 1e-6)
    rms = np.sqrt(np.float32(12.5) + np.float32(1e-6))
    np.testing.assert_allclose(out, [3 / rms, 4 / rms], atol=1e-5)
    out = np.empty(4, np.float32)                            # :122-131
    lib.iris_rms_norm(p(out), p(a(1, 1, 1, 1)), p(a(2, 2, 2, 2)), 1, 4, 1e-6)
    np.testing.assert_allclose(out, 2.0, atol=1e-4)
    out = np.empty(2, np.float32)                            # :133-142
    lib.iris_rms_norm(p(out), p(a(0, 0)), p(a(1, 1)), 1, 2, 1e-5)
    assert np.all(np.isfinite(out))
    out = np.empty(4, np.float32)                            # :144-159
    lib.iris_rms_norm(p(out), p(a(3, 4, 1, 0)), p(a(1, 1)), 2, 2, 1e-6)
    r0, r1 = np.sqrt(12.5 + 1e-6), np.sqrt(0.5 + 1e-6)
    np.testing.assert_allclose(out, [3 / r0, 4 / r0, 1 / r1, 0], atol=1e-4)

    C = np.empty(4, np.float32)                              # :165-177
    lib.iris_matmul(p(C), p(a(1, 2, 3, 4)), p(a(1, 0, 0, 1)), 2, 2, 2)
    np.testing.assert_allclose(C, [1, 2, 3, 4], atol=1e-5)
    C1 = np.empty(1, np.float32)                             # :179-186
    lib.iris_matmul(p(C1), p(a(1, 2)), p(a(5, 6)), 1, 2, 1)
    assert abs(C1[0] - 17) < 1e-4
    lib.iris_matmul(p(C), p(a(1, 2, 3, 4, 5, 6)), p(a(7, 8, 9, 10, 11, 12)), 2, 3, 2)   # :188-202
    np.testing.assert_allclose(C, [58, 64, 139, 154], atol=1e-3)
    lib.iris_matmul_t(p(C), p(a(1, 0, 0, 0, 1, 0)), p(a(1, 0, 0, 0, 1, 0)), 2, 3, 2)   # :204-217
    np.testing.assert_allclose(C, [1, 0, 0, 1], atol=1e-5)

    x = a(0, 1, -1)                                          # :223-232
    lib.iris_silu(p(x), 3)
    np.testing.assert_allclose(x, [0, 0.7310586, -0.2689414], atol=1e-4)
    g = a(1, 0)                                              # :234-240
    lib.iris_silu_mul(p(g), p(a(2, 3)), 2)
    np.testing.assert_allclose(g, [0.7310586 * 2, 0], atol=1e-4)

    x = a(1, 2, 3)                                           # :246-254
    lib.iris_axpy(p(x), 2.0, p(a(4, 5, 6)), 3)
    np.testing.assert_allclose(x, [9, 12, 15], atol=1e-5)
    out = np.empty(2, np.float32)                            # :256-263
    lib.iris_add(p(out), p(a(1, 2)), p(a(3, 4)), 2)
    np.testing.assert_allclose(out, [4, 6], atol=1e-5)

    src = np.arange(32, dtype=np.float32)                    # :269-292
    pt, back = np.empty(32, np.float32), np.empty(32, np.float32)
    lib.iris_patchify(p(pt), p(src), 1, 2, 4, 4, 2)
    lib.iris_unpatchify(p(back), p(pt), 1, 2, 2, 2, 2)
    np.testing.assert_array_equal(back, src)
    src = np.arange(1, 13, dtype=np.float32)                 # :294-305
    out = np.empty(12, np.float32)
    lib.iris_patchify(p(out), p(src), 1, 3, 2, 2, 1)
    np.testing.assert_array_equal(out, src)


def test_reference_attention_parity_cases(lib):
    """debug/test_kernels.c:392-524: naive (iris_attention) and seq-major
    (iris_flash_attention) layouts agree (mean < 1e-3, max < 5e-3), on the
    reference's shapes and seeds, plus the identity-V case."""
    for heads, sq, sk, hd, seed in ((1, 8, 12, 16, 12345), (4, 16, 16, 8, 99999), (1, 96, 128, 8, 77777)):
        lib.iris_rng_seed(seed)
        q = np.empty(sq * heads * hd, np.float32)
        k = np.empty(sk * heads * hd, np.float32)
        v = np.empty(sk * heads * hd, np.float32)
        for arr in (q, k, v):
            lib.iris_randn(p(arr), arr.size)
        scale = 1.0 / np.sqrt(hd)
        to_naive = lambda t, s: np.ascontiguousarray(t.reshape(s, heads, hd).transpose(1, 0, 2))  # noqa: E731
        qn, kn, vn = to_naive(q, sq), to_naive(k, sk), to_naive(v, sk)
        out_n = np.empty(heads * sq * hd, np.float32)
        out_f = np.empty(sq * heads * hd, np.float32)
        lib.iris_attention(p(out_n), p(qn), p(kn), p(vn), 1, heads, sq, sk, hd, scale)
        lib.iris_flash_attention(p(out_f), p(q), p(k), p(v), sq, sk, heads, hd, scale)
        d = np.abs(out_n - to_naive(out_f, sq).ravel())
        assert d.mean() < 1e-3 and d.max() < 5e-3
        ref = attn_ref(qn, kn, vn, scale).ravel()
        np.testing.assert_allclose(out_n, ref, rtol=1e-4, atol=2e-6)
    eye = np.eye(4, dtype=np.float32).ravel()
    on, of = np.empty(16, np.float32), np.empty(16, np.float32)
    lib.iris_attention(p(on), p(eye), p(eye), p(eye), 1, 1, 4, 4, 4, 0.5)
    lib.iris_flash_attention(p(of), p(eye), p(eye), p(eye), 4, 4, 1, 4, 0.5)
    assert np.abs(on - of).mean() < 1e-5 and of[0] > of[1] and of[5] > of[4]
