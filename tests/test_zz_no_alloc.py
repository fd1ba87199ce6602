"""iris_hip_gemm_splitk_noalloc (the split-K GEMM without a workspace: its
f32 partials live in a device array the library holds) against
iris_hip_gemm_splitk with a caller workspace, through the C-ABI: bit for bit,
on two calls in a row, the second with a smaller problem, for each epilogue;
plus a float64 check and the rejection of problems larger than the array."""
import ctypes

import numpy as np
import pytest

import iris_testlib as tl

pytestmark = pytest.mark.gpu
SCRATCH = 32 << 20
EPI_F32, EPI_BF16, EPI_GATED_ADD, EPI_SWIGLU = 0, 1, 2, 3


@pytest.fixture(scope="module")
def lib():
    lib = tl.hip()
    lib.iris_hip_mem_in_use.restype = ctypes.c_size_t
    lib.iris_hip_gemm_splitk.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t]
    lib.iris_hip_gemm_splitk_noalloc.argtypes = [ctypes.c_void_p, ctypes.c_int]
    return lib


def run(lib, M, N, K, splits, epi, seed):
    rng = np.random.default_rng(seed)
    a = tl.to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    w = tl.to_bf16((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
    vec = rng.standard_normal(N).astype(np.float32)
    nout = N // 2 if epi == EPI_SWIGLU else N
    out_bytes = M * nout * (2 if epi in (EPI_BF16, EPI_SWIGLU) else 4)
    base = rng.standard_normal((M, nout)).astype(np.float32)
    da, dw, dv = tl.Dev.of(a), tl.Dev.of(w), tl.Dev.of(vec)
    outs = []
    for noalloc in (False, True):
        do = tl.Dev(out_bytes)
        if epi == EPI_GATED_ADD:
            do.put(base)
        p = tl.GemmProblem(da.ptr, dw.ptr, do.ptr, None if epi == EPI_SWIGLU else dv.ptr, M, N, K, K, K, nout, epi)
        if noalloc:
            # the library's device memory in use does not move across the call
            before = lib.iris_hip_mem_in_use()
            rc = lib.iris_hip_gemm_splitk_noalloc(ctypes.byref(p), splits)
            assert lib.iris_hip_mem_in_use() == before, "the no-allocation entry point allocated"
        else:
            ws = tl.Dev(SCRATCH)
            rc = lib.iris_hip_gemm_splitk(ctypes.byref(p), splits, ws.ptr, SCRATCH)
        assert rc == 0, lib.iris_hip_last_error()
        assert lib.iris_hip_sync() == 0
        if epi in (EPI_BF16, EPI_SWIGLU):
            outs.append(do.get(np.uint16, (M, nout)))
        else:
            outs.append(do.get(np.float32, (M, nout)))
    np.testing.assert_array_equal(outs[0], outs[1])
    # and the product itself, against float64
    acc = tl.bf16_to_f32(a).astype(np.float64) @ tl.bf16_to_f32(w).astype(np.float64).T
    if epi == EPI_SWIGLU:
        g = np.concatenate([acc[:, i * 64:i * 64 + 32] for i in range(N // 64)], 1)
        u = np.concatenate([acc[:, i * 64 + 32:i * 64 + 64] for i in range(N // 64)], 1)
        want, got = g / (1 + np.exp(-g)) * u, tl.bf16_to_f32(outs[1])
    elif epi == EPI_GATED_ADD:
        want, got = base + vec * acc, outs[1]
    elif epi == EPI_BF16:
        want, got = acc + vec, tl.bf16_to_f32(outs[1])
    else:
        want, got = acc + vec, outs[1]
    assert tl.rel_l2(got, want) < 1e-2


@pytest.mark.parametrize("epi", [EPI_F32, EPI_BF16, EPI_GATED_ADD, EPI_SWIGLU])
def test_noalloc_equals_workspace_path(lib, epi):
    """two calls in a row on the shared array: a large one, then a smaller one"""
    run(lib, 512, 2560, 9728, 4, epi, 1 + epi)
    run(lib, 300, 1024 if epi == EPI_SWIGLU else 1000, 3072, 3, epi, 11 + epi)


def test_noalloc_one_chunk_needs_no_scratch(lib):
    """K of one step leaves one chunk whatever the split count: the plain
    product, accepted even when M x N f32 partials would not fit the array
    (4096 x 4096 x 4 B = 64 MiB), equal to iris_hip_gemm bit for bit."""
    M = N = 4096
    K = 64
    rng = np.random.default_rng(5)
    a = tl.to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    w = tl.to_bf16((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
    da, dw = tl.Dev.of(a), tl.Dev.of(w)
    outs = []
    for noalloc in (True, False):
        do = tl.Dev(M * N * 4)
        p = tl.GemmProblem(da.ptr, dw.ptr, do.ptr, None, M, N, K, K, K, N, EPI_F32)
        if noalloc:
            before = lib.iris_hip_mem_in_use()
            assert lib.iris_hip_gemm_splitk_noalloc(ctypes.byref(p), 4) == 0, lib.iris_hip_last_error()
            assert lib.iris_hip_mem_in_use() == before
        else:
            assert lib.iris_hip_gemm(ctypes.byref(p), 1) == 0, lib.iris_hip_last_error()
        assert lib.iris_hip_sync() == 0
        outs.append(do.get(np.float32, (M, N)))
    np.testing.assert_array_equal(outs[0], outs[1])


def test_noalloc_rejects_oversized(lib):
    """chunks x M x N f32 partials beyond the array: an error, nothing launched"""
    p = tl.GemmProblem(None, None, None, None, 4096, 4096, 4096, 4096, 4096, 4096, EPI_F32)
    d = tl.Dev(256)
    p.A = p.W = p.out = d.ptr
    assert lib.iris_hip_gemm_splitk_noalloc(ctypes.byref(p), 4) == -1
    assert b"scratch" in lib.iris_hip_last_error()
