"""The C-ABI library loads on a CPU host and exports every entry point that
include/*.h declares, with the ctypes signatures the binding uses. No compute
calls are made here (no GPU)."""
import glob
import os
import re
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = []
    for h in glob.glob(os.path.join(REPO, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names += re.findall(r"^[A-Za-z_][\w \*]*?\b(sgl_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = _declared()
    for n in ("sgl_abi_version", "sgl_last_error", "sgl_tcsr_build", "sgl_recent_sample", "sgl_recent_compact"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from starry_unigraph.lib import _capi
    lib = _capi.load_library()
    so = _capi.LIB_PATH
    out = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (sgl_\w+)", out))
    declared = set(_declared())
    assert declared <= exported, f"declared but not exported: {sorted(declared - exported)}"
    assert declared == set(_capi.SIGNATURES), "ctypes signature table out of sync with the header"
    for name in declared:
        assert hasattr(lib, name)
    assert lib.sgl_abi_version() == _capi.ABI_VERSION


def test_host_side_queries_need_no_gpu():
    from starry_unigraph.lib import _capi
    lib = _capi.load_library()
    assert lib.sgl_tcsr_workspace_bytes(1000, 10 ** 6) >= 4 * 4 * 10 ** 6
    assert lib.sgl_compact_workspace_bytes(10 ** 6) >= 2 * 8 * (10 ** 6 // 256)


def test_argument_errors_are_reported_without_a_gpu():
    from starry_unigraph.lib import _capi
    lib = _capi.load_library()
    rc = lib.sgl_recent_sample(None, None, None, None, 10, None, 1, None, 5, None, None, 0, -3,
                               None, None, None, None, None, None, None)
    assert rc == 1
    assert b"fanout" in lib.sgl_last_error()
    rc = lib.sgl_tcsr_build(-1, 0, None, None, None, None, None, None, None, None, None, 0, None, None)
    assert rc == 1 and b"num_nodes" in lib.sgl_last_error()


def test_product_path_fails_loudly_without_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from starry_unigraph.native import is_bts_sampler_available
    from starry_unigraph.native.tcsr import build_tcsr
    assert is_bts_sampler_available() is False
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        build_tcsr(3, [0], [1], None, [1])


def test_grad_job_struct_layout_matches_header(tmp_path):
    """ctypes' GradJob has the size and field offsets of struct sgl_grad_job
    (host compiler on the header)."""
    import ctypes
    from starry_unigraph.lib import _capi
    fields = [f for f, _ in _capi.GradJob._fields_]
    src = tmp_path / "layout.cpp"
    src.write_text(
        '#include <cstdio>\n#include <cstddef>\n#include "starrygl_mi355x.h"\nint main() {\n'
        '  printf("%zu", sizeof(sgl_grad_job));\n'
        + "".join(f'  printf(" %zu", offsetof(sgl_grad_job, {f}));\n' for f in fields) + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-I" + os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [ctypes.sizeof(_capi.GradJob)] + [getattr(_capi.GradJob, f).offset for f in fields]
    assert got == want
