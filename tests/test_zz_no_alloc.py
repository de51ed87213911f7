"""kuiops_gemv_splitk_noalloc (the allocation-free decode GEMM) against
kuiops_gemv_splitk on the same inputs, both called through the C ABI.

Both run the same kernels, so the results must be bit-identical.  Two calls
in a row, the second on a smaller input (so the second reads the shared
device array that the first left behind), for each kernel family (row
streaming M=1, strip M=16, K-contiguous split-K), plus the size limit."""
import ctypes

import pytest
import torch

from kuillm_amd import _lib

pytestmark = pytest.mark.gpu


def _call(lib, name, x, W, layout, out, bias=None, ws=None):
    M, K = x.shape
    N = out.shape[1]
    ldw = W.stride(0) if layout == _lib.B_ROW else W.stride(1)
    args = [M, N, K, _lib.BF16, x.data_ptr(), x.stride(0), W.data_ptr(), ldw, layout,
            None if bias is None else bias.data_ptr(), _lib.BF16, out.data_ptr(), out.stride(0), 0]
    if name == "kuiops_gemv_splitk":
        args += [ws.data_ptr(), ws.numel()]
    args.append(torch.cuda.current_stream().cuda_stream)
    return getattr(lib, name)(*args)


def _reference(lib, x, W, layout, bias):
    M, K = x.shape
    N = W.shape[1] if layout == _lib.B_ROW else W.shape[1]
    need = lib.kuiops_query_workspace(_lib.OP_GEMV_SPLITK, M, N, K)
    ws = torch.zeros(max(need, 16), dtype=torch.uint8, device=x.device)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
    assert _call(lib, "kuiops_gemv_splitk", x, W, layout, out, bias, ws) == _lib.OK
    return out


@pytest.mark.parametrize("layout", ["row", "col"])
@pytest.mark.parametrize("shapes", [((16, 11008, 4096), (4, 4096, 2048)),     # strip, then strip
                                    ((1, 11008, 4096), (1, 2048, 1024)),      # row streaming
                                    ((16, 4096, 4096), (1, 4096, 4096))])     # strip, then rows
def test_noalloc_matches_workspace_entry_point(cuda, layout, shapes):
    lib = _lib.load()
    g = torch.Generator(device=cuda).manual_seed(5)
    lay = _lib.B_ROW if layout == "row" else _lib.B_COL
    for (M, N, K) in shapes:                   # second call: smaller input, same shared array
        print(f"noalloc case layout={layout} M={M} N={N} K={K}", flush=True)
        x = torch.randn(M, K, device=cuda, generator=g).to(torch.bfloat16)
        Wkn = (torch.randn(K, N, device=cuda, generator=g) * 0.02).to(torch.bfloat16)
        W = Wkn if lay == _lib.B_ROW else Wkn.t().contiguous().t()
        bias = torch.randn(N, device=cuda, generator=g).to(torch.bfloat16)
        want = _reference(lib, x, W, lay, bias)
        got = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=cuda)
        assert _call(lib, "kuiops_gemv_splitk_noalloc", x, W, lay, got, bias) == _lib.OK
        again = torch.empty_like(got)
        assert _call(lib, "kuiops_gemv_splitk_noalloc", x, W, lay, again, bias) == _lib.OK
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        assert torch.equal(again, want)
        ref32 = x.float() @ Wkn.float() + bias.float()
        assert torch.allclose(got.float(), ref32, rtol=1e-2, atol=1e-2)


def test_noalloc_rejects_shapes_beyond_its_array(cuda):
    lib = _lib.load()
    cap = lib.kuiops_gemv_splitk_noalloc_max_bytes()
    assert cap == 8 << 20
    M, N, K = 64, 65536, 65536                  # split partials far above 8 MiB
    assert lib.kuiops_query_workspace(_lib.OP_GEMV_SPLITK, M, N, K) > cap
    p = ctypes.c_void_p(1 << 20)
    st = lib.kuiops_gemv_splitk_noalloc(M, N, K, _lib.BF16, p, K, p, N, _lib.B_ROW, None, _lib.BF16, p, N, 0,
                                        torch.cuda.current_stream().cuda_stream)
    assert st == _lib.E_WORKSPACE
