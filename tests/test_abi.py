"""The C ABI library: loads, exports every symbol include/kuiops.h declares,
and validates arguments on the host (no kernel launches, no GPU needed)."""
import ctypes
import re

import pytest

from kuillm_amd import _lib, compile as _compile, config as C

HEADER = C.INCLUDE / "kuiops.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"KUIOPS_API\s+[\w\s\*]*?\b(kuiops_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not C.LIB_PATH.exists():
        _compile.build_library()
    return _lib.load()


def test_header_declares_the_expected_entry_points():
    syms = declared_symbols()
    for name in ("kuiops_mm", "kuiops_addmm", "kuiops_bmm", "kuiops_gemv_splitk", "kuiops_sdpa_fwd",
                 "kuiops_sdpa_decode", "kuiops_softmax_lastdim", "kuiops_topk_lastdim", "kuiops_gather",
                 "kuiops_index", "kuiops_query_workspace", "kuiops_status_string", "kuiops_abi_version"):
        assert name in syms
    # the ctypes table mirrors the header one to one
    assert sorted(_lib.SIGNATURES) == syms


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(str(C.LIB_PATH))
    for name in declared_symbols():
        assert hasattr(raw, name), f"{name} not exported by {C.LIB_PATH.name}"


def test_version_and_status_strings(lib):
    assert lib.kuiops_abi_version() == 1
    assert lib.kuiops_status_string(0) == b"ok"
    assert b"unsupported" in lib.kuiops_status_string(-1)
    assert b"invalid" in lib.kuiops_status_string(-2)
    assert b"workspace" in lib.kuiops_status_string(-4)


def test_workspace_queries(lib):
    # gemv split-K: a 16 KB counter head plus splits * M * N * 4 bytes of
    # partials, splits chosen from N and K
    head = 16384
    ws = lib.kuiops_query_workspace(_lib.OP_GEMV_SPLITK, 16, 11008, 4096)
    assert ws > head and (ws - head) % (16 * 11008 * 4) == 0
    assert lib.kuiops_query_workspace(_lib.OP_GEMV_SPLITK, 1, 11008, 4096) - head == (ws - head) // 16
    # a 4096^3 GEMM fills the GPU without split-K
    assert lib.kuiops_query_workspace(_lib.OP_ADDMM, 4096, 4096, 4096) == 0
    # a few output tiles with a deep K do split
    assert lib.kuiops_query_workspace(_lib.OP_ADDMM, 128, 128, 8192) > 0
    assert lib.kuiops_query_workspace(_lib.OP_SDPA_DECODE, 32, 4096, 128) >= 32 * 32 * 130 * 4
    assert lib.kuiops_query_workspace(99, 1, 1, 1) == 0
    assert lib.kuiops_query_workspace(_lib.OP_ADDMM, -1, 1, 1) == 0
    # batched decode rows: K >= 4096 splits K (staged: only with fewer output
    # groups than CUs)
    assert lib.kuiops_query_workspace(_lib.OP_DECODE_ROWS_BATCHED, 64, 2048, 5632) > 0
    assert lib.kuiops_query_workspace(_lib.OP_DECODE_ROWS_BATCHED, 8, 2048, 5632) > 0
    assert lib.kuiops_query_workspace(_lib.OP_DECODE_ROWS_BATCHED, 64, 2048, 2048) == 0
    assert lib.kuiops_query_workspace(_lib.OP_DECODE_ROWS_BATCHED, 8, 2048, 2048) == 0


def test_host_side_argument_validation(lib):
    # invalid sizes are rejected before anything is enqueued
    assert lib.kuiops_mm(-1, 4, 4, _lib.BF16, None, 4, None, 4, 0, _lib.BF16, None, 4, None) == _lib.E_INVALID
    assert lib.kuiops_mm(4, 4, 4, _lib.BF16, None, 4, None, 4, 7, _lib.BF16, None, 4, None) == _lib.E_INVALID
    assert lib.kuiops_mm(4, 4, 4, _lib.BF16, None, 4, None, 4, 0, _lib.BF16, None, 4, None) == _lib.E_INVALID
    # empty problems are a no-op success
    assert lib.kuiops_mm(0, 4, 4, _lib.BF16, None, 4, None, 4, 0, _lib.BF16, None, 4, None) == _lib.OK
    assert lib.kuiops_softmax_lastdim(0, 10, _lib.F32, None, None, None) == _lib.OK
    assert lib.kuiops_softmax_lastdim(-1, 10, _lib.F32, None, None, None) == _lib.E_INVALID
    # gemv: M above 64 is outside the kernel
    p = ctypes.c_void_p(16)
    assert lib.kuiops_gemv_splitk(65, 8, 8, _lib.BF16, p, 8, p, 8, 0, None, _lib.BF16, p, 8, 0, None, 0,
                                  None) == _lib.E_UNSUPPORTED
    # gemv with a workspace that is too small
    assert lib.kuiops_gemv_splitk(16, 11008, 4096, _lib.BF16, p, 4096, p, 11008, 0, None, _lib.BF16, p,
                                  11008, 8, p, 16, None) == _lib.E_WORKSPACE
    # topk: k > n is invalid, k > 1024 unsupported
    assert lib.kuiops_topk_lastdim(1, 10, 11, _lib.F32, p, p, None, 1, 1, None, 0, None) == _lib.E_INVALID
    assert lib.kuiops_topk_lastdim(1, 5000, 2000, _lib.F32, p, p, ctypes.cast(p, ctypes.POINTER(ctypes.c_int64)),
                                   1, 1, None, 0, None) == _lib.E_UNSUPPORTED
    # gather: rank out of range, dim out of range
    shp = _lib.i64_array([2, 2])
    assert lib.kuiops_gather(9, shp, shp, 0, 4, p, None, p, None, None) == _lib.E_INVALID
    assert lib.kuiops_gather(2, shp, shp, 2, 4, p, None, p, None, None) == _lib.E_INVALID
    # sdpa: head counts that do not divide, unsupported head dim
    s3 = _lib.strides3(0, 0, 0)
    assert lib.kuiops_sdpa_fwd(1, 3, 2, 4, 4, 64, 64, _lib.BF16, p, s3, p, s3, p, s3, p, s3, None, 1.0, 0,
                               None) == _lib.E_INVALID
    assert lib.kuiops_sdpa_fwd(1, 2, 2, 4, 4, 96, 96, _lib.BF16, p, s3, p, s3, p, s3, p, s3, None, 1.0, 0,
                               None) == _lib.E_UNSUPPORTED


@pytest.mark.parametrize("s, sk2, sv2", [
    (262145, 4096, 128),          # (B, S, H, D) keys, H*D = 4096: last key row ends past 2^31 bytes
    (262145, 128, 4096),          # the same through V
    (600000, 4096, 4096),         # far past: a 32-bit offset would wrap onto other keys
    (40, 1 << 27, 128),           # huge key stride: the padded last block passes 2^32
    (8, -64, 128),                # negative strides are never addressed by a descriptor
])
def test_sdpa_fwd_rejects_keys_beyond_32bit_offsets(lib, s, sk2, sv2):
    # fa_fwd_kernel reads K / V through buffer descriptors with 32-bit byte
    # offsets; the entry point must refuse shapes they cannot address rather
    # than read zeros or wrap (host-side gate, nothing is launched).
    p = ctypes.c_void_p(1 << 20)
    sq = _lib.strides3(0, 0, 128)
    so = _lib.strides3(0, 0, 128)
    sk = _lib.strides3(0, 0, sk2)
    sv = _lib.strides3(0, 0, sv2)
    for causal in (0, 1):
        assert lib.kuiops_sdpa_fwd(1, 1, 1, 1, s, 128, 128, _lib.BF16, p, sq, p, sk, p, sv, p, so, None,
                                   0.088, causal, None) == _lib.E_UNSUPPORTED


def test_error_mapping():
    with pytest.raises(_lib.Unsupported):
        _lib.check("x", _lib.E_UNSUPPORTED)
    with pytest.raises(_lib.KuiopsError):
        _lib.check("x", _lib.E_HIP)
    _lib.check("x", _lib.OK)


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load(tmp_path / "libkuiops.so")


def test_no_kernel_launch_stub_left_undefined(lib):
    # A kernel whose host-side launch stub is missing still links into the
    # .so (dlopen then fails with "undefined symbol ...__device_stub__...");
    # catch it at build time rather than on the GPU box.
    import subprocess
    out = subprocess.run(["nm", "-D", "--undefined-only", str(C.LIB_PATH)], capture_output=True, text=True).stdout
    assert "__device_stub__" not in out


def test_decode_step_host_checks(lib):
    """The persistent decode step's buffer sizes and argument checks (host
    only): the scratch grows with the steps per launch (one slot of new k / v
    rows per layer and step), and step counts outside 1..32, a cache longer
    than the one-pass attention covers (768 keys at head dim 64, 384 at 128)
    or a short scratch are refused before any launch."""
    L, d, ffn, hq, hkv, hd = 16, 2048, 5632, 32, 8, 64
    one = lib.kuiops_decode_step_scratch_bytes(L, 1, d, ffn, hq, hkv, hd)
    eight = lib.kuiops_decode_step_scratch_bytes(L, 8, d, ffn, hq, hkv, hd)
    slot = L * hkv * hd * 4                       # two 16-bit elements per 8-byte word
    assert eight - one == 2 * 7 * slot
    assert lib.kuiops_decode_step_scratch_bytes(L, 0, d, ffn, hq, hkv, hd) == 0
    assert lib.kuiops_decode_step_sync_bytes(L) == 11 * 128
    p = ctypes.c_void_p(1 << 20)                  # never dereferenced: the checks come first

    def call(n_steps, scratch_bytes, cap=640, hd_=hd, hq_=hq):
        return lib.kuiops_decode_step(L, d, ffn, hq_, hkv, hd_, 32000, cap, _lib.BF16, 1e-5, p, cap * hd_, hd_,
                                      cap * hd_, hd_, p, p, p, p, p, p, p, p, 1024, p, p, n_steps, p,
                                      scratch_bytes, p, 11 * 128, None)

    assert call(0, eight) == _lib.E_UNSUPPORTED
    assert call(33, 1 << 30) == _lib.E_UNSUPPORTED
    assert call(8, one) == _lib.E_WORKSPACE
    # the one-pass attention covers 8 waves x (512 / hd) lane groups x 12 keys
    assert call(8, 1 << 30, cap=769) == _lib.E_UNSUPPORTED
    assert call(8, 1 << 30, cap=385, hd_=128, hq_=16) == _lib.E_UNSUPPORTED
    sup = lib.kuiops_decode_step_supported
    assert sup(L, d, ffn, hq, hkv, hd, 32000, 769, _lib.BF16) == _lib.E_UNSUPPORTED
    assert sup(L, d, ffn, 16, hkv, 128, 32000, 385, _lib.BF16) == _lib.E_UNSUPPORTED
    assert sup(L, d, ffn, hq, hkv, hd, 32000, 640, _lib.F32) == _lib.E_UNSUPPORTED
    assert sup(L, d, ffn, hq, hkv, hd, 32000, 0, _lib.BF16) == _lib.E_INVALID
