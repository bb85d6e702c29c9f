"""Build the native parts in-tree:

  siphon_amd/lib/libsiphon_hip.so      C-ABI HIP library (gfx950 kernels)
  siphon_amd/lib/backend_hip.o,        C17 host side (the si_backend "hip"
    si_prefill.o                       adapter, the batched prefill): build check
  oracle/libsiq_oracle.so              CPU oracle (test infrastructure)
  oracle/_ref/libsiphon_ref.so         compiled reference checker (only
                                       where /root/reference exists)
  oracle/_ref/libsiphon_engine_ref.so  the reference engine with this
                                       repository's prefill (same condition)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_DIR = os.path.join(PKG, "lib")
HIP_SO = os.path.join(LIB_DIR, "libsiphon_hip.so")

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    # quantizers must be bit-exact: one rounding per float operation
    "-ffp-contract=off",
    # no packed-fp32 instructions in any kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def hipcc() -> str:
    for c in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def build_hip(verbose: bool = False) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = HIP_SO + ".tmp"
    _run([hipcc(), *HIPCC_FLAGS, "-o", tmp, os.path.join(PKG, "csrc", "sihip.hip")], verbose)
    os.replace(tmp, HIP_SO)
    return HIP_SO


def build_backend(verbose: bool = False) -> str:
    """Compile the C17 host side (siphon_amd/host: the "hip" si_backend
    adapter and the batched prefill) as the reference host would: C17,
    -Werror, no HIP headers, no contraction of a*b+c. Inside Siphon they are
    more source files of the engine; here they are compiled against the
    mirror of Siphon's declarations (SI_HIP_STANDALONE) to check they build.
    tests/host and oracle/Makefile (target `engine`) link them into test
    harnesses."""
    os.makedirs(LIB_DIR, exist_ok=True)
    out = None
    for name in ("backend_hip", "si_prefill"):
        src = os.path.join(PKG, "host", name + ".c")
        out = os.path.join(LIB_DIR, name + ".o")
        _run(["gcc", "-std=c17", "-O2", "-fPIC", "-c", "-Wall", "-Wextra", "-Werror",
              "-ffp-contract=off", "-D_POSIX_C_SOURCE=200809L", "-DSI_HIP_STANDALONE",
              "-I", os.path.join(ROOT, "include"), "-I", os.path.join(PKG, "host"), "-o", out, src],
             verbose)
    return out


def build_oracle(verbose: bool = False) -> None:
    odir = os.path.join(ROOT, "oracle")
    _run(["make", "-s", "-C", odir, "libsiq_oracle.so"], verbose)
    if os.path.isdir("/root/reference/src"):
        _run(["make", "-s", "-C", odir, "ref", "engine"], verbose)


def build_test_checkers(verbose: bool = False) -> None:
    """The host emulation of the matvec kernel (tests/emu, test checker only)."""
    _run(["make", "-s", "-C", os.path.join(ROOT, "tests", "emu")], verbose)


def build_all(verbose: bool = False) -> None:
    build_oracle(verbose)
    build_test_checkers(verbose)
    build_backend(verbose)
    build_hip(verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print("built:", HIP_SO)
