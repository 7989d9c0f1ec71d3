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


def test_conv_backward_tile_rows():
    """The ln_part / te_part tile of the attention backward is one workgroup
    of the instance sgl_conv_backward runs; callers size those arrays (and the
    fused update reduces them) by sgl_conv_backward_tile_rows, which asks the
    same instance picker: 1 root for the 16-wave bf16 instances, 8 for the
    8-wave bf16 ones, the fp32 / dropout instances' (sgl_conv_tile_rows) 4,
    or 8 where the 8-wave instances' 4-root layouts do not fit in LDS."""
    from starry_unigraph.lib import _capi
    lib = _capi.load_library()
    assert lib.sgl_conv_backward_tile_rows(100, 16, 100, 2, 1) == 1      # config 4, bf16 GEMMs
    assert lib.sgl_conv_backward_tile_rows(100, 16, 100, 2, 0) == 4      # config 4, fp32 / dropout
    assert lib.sgl_conv_backward_tile_rows(100, 172, 100, 2, 0) == 4     # config 1 (8 waves, 2 a root)
    assert lib.sgl_conv_backward_tile_rows(172, 16, 100, 4, 0) == 8      # config 5 fp32: 4 roots do not fit
    assert lib.sgl_conv_backward_tile_rows(172, 16, 100, 4, 1) == 8      # config 5 (split heads)
    assert lib.sgl_conv_backward_tile_rows(100, 16, 100, 3, 1) == 0      # D % H != 0
    for D in (8, 32, 100, 172, 200):
        for F in (0, 4, 16, 172):
            for T in (0, 8, 100):
                for H in (1, 2, 4):
                    if D % H:
                        continue
                    fp, bf = (lib.sgl_conv_backward_tile_rows(D, F, T, H, b) for b in (0, 1))
                    assert fp == lib.sgl_conv_tile_rows(D, F, T, H), (D, F, T, H)
                    if D + F + T > 512:
                        assert fp == bf == 0
                        continue
                    assert fp in (4, 8) and bf in (1, 8) and 16 % bf == 0, (D, F, T, H, fp, bf)


def test_bf16_gru_tile_rows_fit_lds():
    """The bf16 GRU's tile choice counts its static LDS (the root tables,
    60 bytes a row) with the dynamic tiles against the CU's 160 KiB: shapes
    whose 64-root tiles fit only without the static part take 16-root tiles."""
    from starry_unigraph.lib import _capi
    lib = _capi.load_library()

    def ld_bf16(n):
        return ((n + 7) & ~7) | 8

    def ld_f32(n):
        return ((n + 3) & ~3) | 4

    def need(D, F, rows):
        dyn = 4 * rows * ld_f32(D) + 2 * rows * (ld_bf16(2 * D + F) + 2 * ld_bf16(D))
        return dyn + 60 * rows

    big = 64 * 256
    assert lib.sgl_memory_update_bf16_tile_rows(172, 16, big) == 64      # config 5
    assert lib.sgl_memory_update_bf16_tile_rows(100, 16, 1200) == 16     # config 4's step
    assert lib.sgl_memory_update_bf16_tile_rows(102, 16, big) == 0       # rows not float4
    for D, F in ((192, 88), (192, 96)):
        assert need(D, F, 64) - 60 * 64 <= 160 * 1024 < need(D, F, 64), (D, F)
        assert lib.sgl_memory_update_bf16_tile_rows(D, F, big) == 16, (D, F)
    for D in range(4, 197, 4):
        for F in (0, 16, 96, 172):
            want = 0 if (D + 15) // 16 > 12 else (64 if need(D, F, 64) <= 160 * 1024 else
                                                   (16 if need(D, F, 16) <= 160 * 1024 else 0))
            assert lib.sgl_memory_update_bf16_tile_rows(D, F, big) == want, (D, F)


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


def test_bf16_weights_struct_layout_matches_header(tmp_path):
    """ctypes' Bf16Weights has the size and field offsets of struct
    sgl_bf16_weights."""
    import ctypes
    from starry_unigraph.lib import _capi
    fields = [f for f, _ in _capi.Bf16Weights._fields_]
    src = tmp_path / "layout.cpp"
    src.write_text(
        '#include <cstdio>\n#include <cstddef>\n#include "starrygl_mi355x.h"\nint main() {\n'
        '  printf("%zu", sizeof(sgl_bf16_weights));\n'
        + "".join(f'  printf(" %zu", offsetof(sgl_bf16_weights, {f}));\n' for f in fields) + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-I" + os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [ctypes.sizeof(_capi.Bf16Weights)] + [getattr(_capi.Bf16Weights, f).offset for f in fields]
    assert got == want


def test_plan_op_struct_layout_matches_header(tmp_path):
    """ctypes' Op has the size and field offsets of struct sgl_op."""
    import ctypes
    from starry_unigraph.lib import _capi
    fields = [f for f, _ in _capi.Op._fields_]
    src = tmp_path / "layout.cpp"
    src.write_text(
        '#include <cstdio>\n#include <cstddef>\n#include "starrygl_mi355x.h"\nint main() {\n'
        '  printf("%zu %d", sizeof(sgl_op), SGL_OP_MAX_ARGS);\n'
        + "".join(f'  printf(" %zu", offsetof(sgl_op, {f}));\n' for f in fields) + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-I" + os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [ctypes.sizeof(_capi.Op), _capi.SGL_OP_MAX_ARGS] + [getattr(_capi.Op, f).offset for f in fields]
    assert got == want


def test_header_constants_match_binding(tmp_path):
    """The binding's copies of the header's constants (ABI version, device
    error bits, fixed-point scale, completion-counter size and range-flag
    word) are the header's."""
    from starry_unigraph.lib import _capi
    names = ["SGL_ABI_VERSION", "SGL_DERR_NODE_RANGE", "SGL_DERR_EID_RANGE", "SGL_DERR_STALE_NODE_BITS",
             "SGL_FIXED_SHIFT", "SGL_DONE_WORDS",
             "SGL_DONE_RANGE_WORD", "SGL_OP_MAX_ARGS", "SGL_COMPACT_NOALLOC_MAX_QUERIES",
             "SGL_LINK_METRICS_MAX_SCORES"]
    src = tmp_path / "consts.cpp"
    src.write_text('#include <cstdio>\n#include "starrygl_mi355x.h"\nint main() {\n'
                   + "".join(f'  printf("%d ", int({n}));\n' for n in names) + "  return 0;\n}\n")
    exe = tmp_path / "consts"
    subprocess.run(["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-I" + os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [_capi.ABI_VERSION, _capi.SGL_DERR_NODE_RANGE, _capi.SGL_DERR_EID_RANGE, _capi.SGL_DERR_STALE_NODE_BITS,
            _capi.SGL_FIXED_SHIFT,
            _capi.SGL_DONE_WORDS, _capi.SGL_DONE_RANGE_WORD, _capi.SGL_OP_MAX_ARGS,
            _capi.SGL_COMPACT_NOALLOC_MAX_QUERIES, _capi.SGL_LINK_METRICS_MAX_SCORES]
    assert got == want


def test_plan_recording_and_packing():
    """Recorded calls pack into sgl_op slots as the library's op table expects
    (no launch: a recording intercepts the calls): every plannable entry point
    is known to the library with the binding's argument count, pointers and
    integers keep their value (negative integers in two's complement), floats
    their bit pattern, host pointer arrays their address; unknown names are
    rejected."""
    import ctypes
    import struct
    from starry_unigraph.lib import _capi
    L = _capi.lib()
    plannable = ["sgl_batch_prepare", "sgl_recent_sample", "sgl_memory_update", "sgl_memory_commit",
                 "sgl_conv_forward", "sgl_predictor", "sgl_conv_backward", "sgl_grad_adam", "sgl_adam_coef",
                 "sgl_edge_rows", "sgl_memory_update_bf16", "sgl_recent_sample_packed"]
    for name in plannable:
        n = ctypes.c_int32(-1)
        assert L.sgl_plan_op_kind(name.encode(), ctypes.byref(n)) >= 0, name
        assert n.value == len(_capi.SIGNATURES[name][1]) - 1 <= _capi.SGL_OP_MAX_ARGS, name
    assert L.sgl_plan_op_kind(b"sgl_tcsr_build", None) == -1
    host_arr = (ctypes.c_void_p * 2)(0x1000, 0x2000)
    types = _capi.SIGNATURES["sgl_grad_adam"][1]
    args = []
    for t in types[:-1]:
        if t is ctypes.c_float:
            args.append(0.125)
        elif t is ctypes.c_int32:
            args.append(-3)
        else:
            args.append(0xABC0)
    args[9] = host_arr          # gates: a host array of device pointers
    args[3] = None              # a NULL pointer
    with _capi.record() as calls:
        assert _capi.call("sgl_grad_adam", *args, 0xDEAD) == 0
    assert len(calls) == 1 and calls[0][0] == "sgl_grad_adam" and len(calls[0][1]) == len(types) - 1
    ops = _capi.pack_ops(calls)
    op = ops[0]
    assert op.kind == L.sgl_plan_op_kind(b"sgl_grad_adam", None) and op.nargs == len(types) - 1
    for j, t in enumerate(types[:-1]):
        if j == 9:
            assert op.a[j] == ctypes.addressof(host_arr)
        elif j == 3:
            assert op.a[j] == 0
        elif t is ctypes.c_float:
            assert op.a[j] == struct.unpack("<I", struct.pack("<f", 0.125))[0]
        elif t is ctypes.c_int32:
            assert op.a[j] == (-3) & 0xFFFFFFFFFFFFFFFF
        else:
            assert op.a[j] == 0xABC0
    with pytest.raises(RuntimeError):
        _capi.pack_ops([("sgl_tcsr_build", (1, 2))])
