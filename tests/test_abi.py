"""The C-ABI boundary without a GPU: libiris_hip.so loads and exports every
function include/*.h declares (no compute calls)."""
import ctypes
import os
import re

import pytest

import iris_testlib as tl

INCLUDE = os.path.join(tl.ROOT, "include")


def declared_functions():
    names = {}
    for fn in sorted(os.listdir(INCLUDE)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, fn)).read()
        text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
        text = re.sub(r"//[^\n]*", " ", text)
        text = re.sub(r"^\s*#[^\n]*", " ", text, flags=re.M)
        # statements at file scope: the C++ linkage wrapper, then struct/enum bodies removed
        text = text.replace('extern "C" {', " ")
        while True:
            stripped = re.sub(r"\{[^{}]*\}", ";", text)     # a body ends a statement
            if stripped == text:
                break
            text = stripped
        text = text.replace("}", " ")
        for stmt in text.split(";"):
            s = " ".join(stmt.split())
            if not s or s.startswith(("typedef", "static", "extern \"C\"")):
                continue
            m = re.match(r"^(?:extern\s+)?[A-Za-z_][\w\s\*]*?[\s\*](\w+)\s*\((.*)\)$", s)
            if m:
                names.setdefault(fn, []).append(m.group(1))
                continue
            m = re.match(r"^extern\s+[A-Za-z_][\w\s\*]*?[\s\*](\w+)$", s)   # exported variables
            if m:
                names.setdefault(fn, []).append(m.group(1))
    return names


DECLS = declared_functions()


def test_headers_parsed():
    assert "iris_hip.h" in DECLS and "iris_transformer.h" in DECLS and "iris_sample.h" in DECLS
    assert "iris_hip_gemm" in DECLS["iris_hip.h"] and "iris_hip_conv3x3" in DECLS["iris_hip.h"]
    assert "iris_vae_gpu_decode" in DECLS["iris_vae.h"] and "iris_image_free" in DECLS["iris_vae.h"]
    assert "iris_transformer_forward" in DECLS["iris_transformer.h"]
    assert "zi_transformer_forward" in DECLS["iris_transformer.h"]
    assert "iris_conv2d" in DECLS["iris_kernels.h"] and "iris_substep_callback" in DECLS["iris_kernels.h"]
    assert "fast_expf" not in DECLS["iris_kernels.h"]          # static inline, not exported
    assert sum(len(v) for v in DECLS.values()) > 90


@pytest.mark.parametrize("header", sorted(DECLS))
def test_library_exports_declared(header):
    if not os.path.exists(tl.HIP_SO):
        pytest.fail(f"{tl.HIP_SO} is not built")
    lib = ctypes.CDLL(tl.HIP_SO)          # loads without a GPU; nothing is called
    missing = [n for n in DECLS[header] if not hasattr(lib, n)]
    assert not missing, f"{header}: not exported: {missing}"


def test_no_oracle_symbols_in_product():
    """The product library does not carry the oracle's functions."""
    lib = ctypes.CDLL(tl.HIP_SO)
    for n in ("orc_flux_forward", "orc_zi_forward", "orc_set_blas", "orc_linear"):
        assert not hasattr(lib, n), n


# ctypes mirrors of the header structs the tests and bench.py pass through the
# C-ABI, checked field by field against the compiler's own layout
MIRRORS = [("iris_gemm_problem_t", "iris_hip.h", tl.GemmProblem),
           ("iris_conv3x3_t", "iris_hip.h", tl.Conv3x3),
           ("iris_norm_args_t", "iris_hip.h", tl.NormArgs),
           ("iris_qkprep_args_t", "iris_hip.h", tl.QkPrepArgs),
           ("iris_attn_args_t", "iris_hip.h", tl.AttnArgs),
           ("iris_ref_t", "iris_transformer.h", tl.IrisRef),
           ("iris_kernel_time_t", "iris_hip.h", tl.KernelTime)]


C_NAME = {"inp": "in"}      # Python keywords renamed in the mirrors


def test_struct_mirrors_match_headers(tmp_path):
    import shutil
    import subprocess
    if not shutil.which("gcc"):
        pytest.skip("gcc not found")
    lines = ["#include <stddef.h>", "#include <stdint.h>", "#include <stdio.h>"]
    lines += sorted({f'#include "{h}"' for _, h, _ in MIRRORS})
    lines.append("int main(void) {")
    for cname, _, cls in MIRRORS:
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {C_NAME.get(f, f)}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", INCLUDE, str(src), "-o", str(exe)], check=True)
    got = dict(l.rsplit(" ", 1) for l in subprocess.run([str(exe)], check=True, capture_output=True,
                                                         text=True).stdout.splitlines())
    for cname, _, cls in MIRRORS:
        assert int(got[f"{cname} size"]) == ctypes.sizeof(cls), cname
        for f, _ in cls._fields_:
            assert int(got[f"{cname} {f}"]) == getattr(cls, f).offset, (cname, f)
