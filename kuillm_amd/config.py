"""Paths, environment flags and toolchain flags of the kuiops build.

Flag names follow the reference's ``kuipy/config.py:11-50`` so existing
environments keep working: KUIPY_JIT_VERBOSITY, KUIPY_JIT_FLUSH_CACHE,
KUIPY_PRINT_PROFILING, KUIPY_JIT_STRICTNESS, KUIPY_JIT_NVCC_FAST (here: a fast
-O1 hipcc build), KUIPY_RE_TUNE, KUIPY_CACHE.  The F*/karamel flags of the
reference have no counterpart: kernels are hand-written HIP compiled by hipcc.
"""
import os
from pathlib import Path

_HERE = Path(__file__).resolve().parent
_REPO_ROOT = _HERE.parent

# --------------------------------------------------------------------------
# paths
# --------------------------------------------------------------------------
CSRC = _HERE / "csrc"
INCLUDE = _REPO_ROOT / "include"
LIB_PATH = _HERE / "libkuiops.so"
ROCM_PATH = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = ROCM_PATH / "bin" / "hipcc"

KUIPY_CACHE = Path(os.environ.get("KUIPY_CACHE", _REPO_ROOT / ".kuipy_cache")).resolve()
KUIPY_JIT_BUILD = KUIPY_CACHE / "build"          # lock files / object dirs
# Persistent autotune parameters (the reference's "LATER: load these from
# json", kuipy/registry.py:71,76).
TUNE_FILE = Path(os.environ.get("KUIPY_TUNE_FILE", KUIPY_CACHE / "tune.json"))

# --------------------------------------------------------------------------
# behaviour
# --------------------------------------------------------------------------
JIT_VERBOSITY = int(os.environ.get("KUIPY_JIT_VERBOSITY", "0"))   # 2 = print mismatched ops
JIT_FLUSH_CACHE = os.environ.get("KUIPY_JIT_FLUSH_CACHE", "0") == "1"
ENABLE_PRINT_PROFILING = os.environ.get("KUIPY_PRINT_PROFILING", "0") == "1"

# 0 = no errors from the kernels: warn once and fall back to stock PyTorch
# 1 = error when the native library cannot be built / loaded or a kernel fails
# 2 = also error when an operator is not offloaded
JIT_STRICTNESS = int(os.environ.get("KUIPY_JIT_STRICTNESS", "1"))

JIT_NVCC_FAST = os.environ.get("KUIPY_JIT_NVCC_FAST", "0") == "1"
RE_TUNE = os.environ.get("KUIPY_RE_TUNE", "0") == "1"

# --------------------------------------------------------------------------
# hipcc flags (the reference's nvcc flags, kuipy/config.py:99-123)
# --------------------------------------------------------------------------
ARCH = os.environ.get("KUIOPS_ARCH", "gfx950")
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-std=c++17", "-fPIC",
    # packed-fp32 VALU ops stay disabled in all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-O1" if JIT_NVCC_FAST else "-O3",
]


def hipcc_arch_flag():
    """``--offload-arch`` of the build (the reference derives an sm_XX gencode
    from the visible device, kuipy/config.py:125-132; this build targets gfx950
    only)."""
    return f"--offload-arch={ARCH}"


def ensure_dirs():
    KUIPY_JIT_BUILD.mkdir(parents=True, exist_ok=True)


def log(*a):
    if JIT_VERBOSITY > 0:
        print("[kuipy-jit]", *a, flush=True)
