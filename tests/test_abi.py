"""The C-ABI library loads and exports every entry point include/sihip.h
declares (no device work: this runs without a GPU)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sihip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sihip_[A-Za-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("sihip_abi_version", "sihip_init", "sihip_weight_upload", "sihip_gemv",
                     "sihip_gemm", "sihip_quantize_q8_K", "sihip_quantize_q8_0",
                     "sihip_vec_dot", "sihip_quantize_q8_K_rows"):
        assert required in names


def test_library_exports_every_declared_symbol():
    import siphon_amd
    lib = siphon_amd.load_library()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_abi_version_matches_header():
    import siphon_amd
    lib = siphon_amd.load_library()
    hv = int(re.search(r"#define SIHIP_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert lib.sihip_abi_version() == hv == siphon_amd.ABI_VERSION


def test_library_is_gfx950_code():
    """The shared object carries a gfx950 code object."""
    import siphon_amd
    from siphon_amd.build import HIP_SO
    siphon_amd.load_library()
    blob = open(HIP_SO, "rb").read()
    assert b"gfx950" in blob


def test_missing_library_fails_loudly(tmp_path):
    import siphon_amd
    with pytest.raises(FileNotFoundError):
        siphon_amd.load_library_at(str(tmp_path / "nope.so"))
