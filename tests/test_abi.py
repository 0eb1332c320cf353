"""The C ABI: libe2v2.so loads (no GPU needed) and exports every function that
include/e2v2.h declares; the Python binding lists the same set."""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared():
    text = (ROOT / "include" / "e2v2.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|size_t|const char\*)\s+(e2v2_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_api():
    names = declared()
    assert "e2v2_attn_fwd" in names and "e2v2_nbr_fill" in names and len(names) >= 17


def test_library_exports_every_declared_symbol(pkg):
    from ubio_molfm_amd import _lib
    lib = _lib.load()
    for name in declared():
        assert hasattr(lib, name), name
    assert sorted(_lib.EXPORTS) == declared()
    assert lib.e2v2_version() >= 1


def test_error_path_reports_message(pkg):
    from ubio_molfm_amd import _lib
    import ctypes
    lib = _lib.load()
    # a negative length is rejected on the host before any launch
    rc = lib.e2v2_scan_i32(None, ctypes.c_int(-1), None, None, None)
    assert rc != 0 and b"negative" in lib.e2v2_last_error()


def test_noalloc_rejects_oversized_plan(pkg):
    """e2v2_nbr_count_noalloc checks the plan against its static scratch before any
    HIP call: more atoms than E2V2_NOALLOC_MAX_ATOMS is an error with a message."""
    from ubio_molfm_amd import _lib
    import ctypes
    lib = _lib.load()
    plan = _lib.NbrPlan()
    plan.n_atoms = (1 << 20) + 1
    plan.n_bins = 8
    dummy = ctypes.c_void_p(16)          # never dereferenced: the size check fails first
    rc = lib.e2v2_nbr_count_noalloc(ctypes.byref(plan), dummy, dummy, dummy, None)
    assert rc != 0 and b"exceed the static scratch" in lib.e2v2_last_error()


def test_header_so2_layout_macros_match_generated_tables(tmp_path):
    """E2V2_SO2_A / _LD / _COL of include/e2v2.h (compiled with gcc) equal the
    l3-grouped row placement the kernels are generated with (so3.so2_row_layout)."""
    import shutil
    import subprocess
    import sys
    if shutil.which("gcc") is None or not Path("/opt/rocm/include/hip/hip_runtime_api.h").exists():
        pytest.skip("gcc or the HIP headers are not available")
    src = tmp_path / "m.c"
    src.write_text('#include <stdio.h>\n#include "e2v2.h"\nint main(void) {\n'
                   '  for (int t = 0; t < 20; ++t) printf("%d %d %d\\n", E2V2_SO2_A(t), E2V2_SO2_LD(t), '
                   'E2V2_SO2_COL(t));\n  return 0;\n}\n')
    exe = tmp_path / "m"
    subprocess.run(["gcc", "-D__HIP_PLATFORM_AMD__", "-I", str(ROOT / "include"), "-I", "/opt/rocm/include",
                    str(src), "-o", str(exe)], check=True, capture_output=True)
    got = [tuple(int(x) for x in line.split()) for line in subprocess.run([str(exe)], check=True,
                                                                          capture_output=True, text=True).stdout.split("\n") if line]
    sys.path.insert(0, str(ROOT / "ubio-molfm_amd"))
    import so3
    a, ld, col, _ = so3.so2_row_layout()
    assert got == list(zip(a, ld, col))


def test_split_gemm_host_checks(pkg):
    """e2v2_gemm_s3 / e2v2_gemm_packed_bytes validate shapes and weight indices on
    the host, before any HIP call."""
    from ubio_molfm_amd import _lib
    lib = _lib.load()
    assert lib.e2v2_gemm_packed_bytes(3, 256, 64, 3) == 3 * 2 * 2 * 3 * 512 * 16
    assert lib.e2v2_gemm_packed_bytes(3, 256, 64, 1) == 3 * 2 * 2 * 1 * 512 * 16
    assert lib.e2v2_gemm_packed_bytes(1, 100, 64, 3) == -1 and lib.e2v2_gemm_packed_bytes(1, 128, 40, 3) == -1
    assert lib.e2v2_gemm_packed_bytes(1, 128, 64, 2) == -1
    g = _lib.GemmArgs()
    g.a = g.b = g.c = 16                 # never dereferenced: the checks fail first
    g.lda, g.ldc, g.m, g.n, g.k, g.batch, g.n_w, g.pieces = 64, 128, 10, 128, 64, 2, 1, 3
    g.widx[1] = 1                         # only weight 0 exists
    assert lib.e2v2_gemm_s3(_lib.C.byref(g), None) != 0 and b"widx[1]" in lib.e2v2_last_error()
    g.widx[1], g.n = 0, 100
    assert lib.e2v2_gemm_s3(_lib.C.byref(g), None) != 0 and b"multiple of 128" in lib.e2v2_last_error()
    g.n, g.a_bf16 = 128, 1               # a bf16 A needs the one-piece packing
    assert lib.e2v2_gemm_s3(_lib.C.byref(g), None) != 0 and b"one piece" in lib.e2v2_last_error()
    g.pieces, g.lda = 1, 68              # bf16 rows of 16 bytes: lda % 8 == 0
    assert lib.e2v2_gemm_s3(_lib.C.byref(g), None) != 0 and b"lda % 8" in lib.e2v2_last_error()


def test_grouped_gemm_host_checks(pkg):
    """e2v2_gemm_s3_grouped takes 1 .. 4 groups and checks each group as
    e2v2_gemm_s3 does, on the host, before any HIP call."""
    from ubio_molfm_amd import _lib
    lib = _lib.load()
    arr = (_lib.GemmArgs * 4)()
    for g in arr:
        g.a = g.b = g.c = 16                 # never dereferenced: the checks fail first
        g.lda, g.ldc, g.m, g.n, g.k, g.batch, g.n_w, g.pieces = 64, 128, 10, 128, 64, 1, 1, 3
    assert lib.e2v2_gemm_s3_grouped(arr, 0, None) != 0 and b"groups" in lib.e2v2_last_error()
    assert lib.e2v2_gemm_s3_grouped(arr, 5, None) != 0 and b"groups" in lib.e2v2_last_error()
    arr[1].pieces = 1                        # the groups of one launch share the operand pieces
    assert lib.e2v2_gemm_s3_grouped(arr, 3, None) != 0 and b"share the operand pieces" in lib.e2v2_last_error()
    arr[1].pieces = 3
    arr[2].k = 40
    assert lib.e2v2_gemm_s3_grouped(arr, 3, None) != 0 and b"multiple of 16" in lib.e2v2_last_error()


def test_gated_gemm_host_checks(pkg):
    """e2v2_gemm_s3_gated checks the gate logits' layout against the batches'
    weight indices on the host, before any HIP call."""
    from ubio_molfm_amd import _lib
    lib = _lib.load()
    g = _lib.GemmArgs()
    g.a = g.b = g.c = 16                 # never dereferenced: the checks fail first
    g.lda, g.ldc, g.m, g.n, g.k, g.batch, g.n_w, g.pieces = 64, 128, 10, 128, 64, 3, 3, 3
    g.widx[0], g.widx[1], g.widx[2] = 0, 1, 2
    f = _lib.C.c_float
    assert lib.e2v2_gemm_s3_gated(_lib.C.byref(g), _lib.C.c_void_p(16), _lib.C.c_int64(128), f(1.0), f(1.0),
                                  None) != 0 and b"past ld_s" in lib.e2v2_last_error()
    assert lib.e2v2_gemm_s3_gated(_lib.C.byref(g), _lib.C.c_void_p(0), _lib.C.c_int64(192), f(1.0), f(1.0),
                                  None) != 0 and b"alignment" in lib.e2v2_last_error()
