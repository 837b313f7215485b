"""The allocation-free split-K GEMM entry point (laya_ext_gemm_splitk_static) through the C ABI:
on two calls in a row, the second with fewer rows, its output equals, bit for bit, that of
laya_ext_gemm with the same split-K factor in a caller-provided workspace, for a bf16 store with
GELU and an fp32 residual update; a split whose partials cannot fit the static array is refused
before anything is launched."""
import ctypes

import numpy as np
import pytest

from layamd_amd import engine as le

pytestmark = pytest.mark.gpu


def _static(lib, epi, A, W, C, bias, act, ks):
    import torch
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return lib.laya_ext_gemm_splitk_static(epi, A.data_ptr(), W.data_ptr(), C.data_ptr(),
                                           bias.data_ptr() if bias is not None else None, act, A.shape[0], W.shape[0],
                                           A.shape[1], ks, st)


@pytest.mark.parametrize("ks", [4, 8])
def test_static_scratch_split_k_matches_workspace_split_k(ks):
    import torch
    lib = le.load_library()
    N, K = 1024, 2048
    g = torch.Generator(device="cpu").manual_seed(ks)
    for M in (1500, 130):                       # the first call runs several row chunks; the second one
        A = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
        W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).cuda()
        bias = (torch.randn(N, generator=g) * 0.1).float().cuda()
        X0 = torch.randn(M, N, generator=g).float().cuda()
        # reference: the existing entry point with the same split in a caller workspace
        ws = torch.empty(ks * 256 * N, dtype=torch.float32, device="cuda")
        prev = le.gemm_ksplit(lib, ks, ws)
        try:
            C_ref = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
            le.gemm(lib, A, W, C_ref, bias=bias, act=2)
            X_ref = X0.clone()
            le.gemm(lib, A, W, X_ref, bias=bias, residual=True)
        finally:
            le.gemm_ksplit(lib, prev)
        C = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        assert _static(lib, 0, A, W, C, bias, 2, ks) == 0
        X = X0.clone()
        assert _static(lib, 1, A, W, X, bias, 0, ks) == 0
        torch.cuda.synchronize()
        assert torch.equal(C.cpu(), C_ref.cpu()), M
        assert torch.equal(X.cpu(), X_ref.cpu()), M
        ref = A.cpu().double() @ W.cpu().double().T + bias.cpu().double()
        assert (X.cpu().double() - X0.cpu().double() - ref).abs().max().item() < 1e-4 * K ** 0.5


def test_static_scratch_rejects_what_does_not_fit():
    import torch
    lib = le.load_library()
    A = torch.zeros(64, 4096, dtype=torch.bfloat16, device="cuda")
    W = torch.zeros(65536, 4096, dtype=torch.bfloat16, device="cuda")   # 64 x 65536 x 4 B > 8 MiB per row
    X = torch.zeros(64, 65536, dtype=torch.float32, device="cuda")
    assert _static(lib, 1, A, W, X, None, 0, 64) == -2
    assert _static(lib, 1, A[:, :1000].contiguous(), W[:8, :1000].contiguous(), X[:, :8].contiguous(), None, 0, 4) == -1
    assert _static(lib, 1, A, W[:1024], X[:, :1024].contiguous(), None, 0, 1) == -1
    torch.cuda.synchronize()
    assert X.abs().max().item() == 0.0
