"""CPU checks of the C-ABI boundary: the library loads, exports every
function include/nnz.h declares, the ctypes table matches the header, and
argument validation answers without touching a GPU."""
import ctypes as C
import subprocess

import pytest

from nnzap_amd import _lib as L


def test_library_loads_and_reports_version():
    assert L.lib().nnz_version().decode().startswith("nnzap_amd")


def test_every_declared_function_is_exported():
    names = L.header_functions()
    assert len(names) > 50
    out = subprocess.run(["nm", "-D", "--defined-only", str(L.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [n for n in names if n not in exported]
    assert not missing, f"declared but not exported: {missing}"


def test_ctypes_table_covers_header():
    assert set(L.header_functions()) == set(L.PROTOS)


def test_null_context_is_rejected_without_gpu():
    lib = L.lib()
    d = L.QMVDims(64, 256, 128)
    assert lib.nnz_dispatch_qmv(None, None, None, None, d) == L.EINVAL
    assert lib.nnz_stream_sync(None, 10) == L.EINVAL
    assert lib.nnz_model_forward_decode(None, 0, 0) == L.EINVAL
    assert lib.nnz_last_error(None) == b"null context"


def test_gqa_scratch_size_is_pure_host_math():
    d = L.GQADims(16, 8, 128, 32768, 32768, 2)
    n = L.lib().nnz_gqa_scratch_bytes(d)
    # 16 heads x chunks x (128 + 2) floats + q buffer
    assert n > 16 * 128 * 4 and n < 16 * 1024 * 130 * 4


def test_dims_structs_match_reference_layout():
    """The dims structs are the reference's extern structs byte for byte
    (transformer.zig:389-479): u32/f32 fields, no padding."""
    assert C.sizeof(L.QMVDims) == 12
    assert C.sizeof(L.RMSNormDims) == 12
    assert C.sizeof(L.RoPEDims) == 16
    assert C.sizeof(L.GQADims) == 24
    assert C.sizeof(L.GQAFusedDims) == 36
    assert C.sizeof(L.EmbedDims) == 16
    assert C.sizeof(L.FusedKNormRoPEKVDims) == 24


def _c_check_lib():
    """tests/c/abi_check.c compiled against include/nnz.h (gcc, -Werror):
    its static_asserts pin every dims struct's size and field offsets to the
    reference's extern structs (transformer.zig:389-479)."""
    import importlib.util
    from pathlib import Path
    here = Path(__file__).resolve().parent / "c"
    spec = importlib.util.spec_from_file_location("nnz_c_tests_build", here / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return C.CDLL(str(mod.build()))


def test_c_translation_unit_compiles_and_checks_error_paths():
    lib = _c_check_lib()
    assert lib.nnz_abi_check_host() == 0


def test_ctypes_argument_counts_match_header():
    """Every ctypes prototype takes as many arguments as the header
    declaration (a drifted signature would pass the name check)."""
    import re
    text = re.sub(r"/\*.*?\*/", "", L.HEADER.read_text(), flags=re.S)
    decls = dict(re.findall(r"\b(nnz_[a-z0-9_]+)\s*\(([^()]*)\)\s*;", text))
    assert set(decls) == set(L.PROTOS)
    for name, params in decls.items():
        params = params.strip()
        n = 0 if params in ("", "void") else params.count(",") + 1
        assert n == len(L.PROTOS[name][1]), f"{name}: header {n} args, ctypes {len(L.PROTOS[name][1])}"
