"""The allocation-free stream-K GEMM entry point (kr_op_gemm_streamk_noalloc)
against the workspace entry point it mirrors (kr_op_gemm_streamk), through
the C ABI: two calls in a row, the second with a smaller split, each equal
bit for bit to the workspace call (same plan, same piece order) and within
the bf16 bar of the oracle; a split larger than the library's scratch is
refused with an error and launches nothing."""

import pytest
import torch

from kernrelay_amd import ops
from oracle import ops as O
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _case(M, N, K, seed, bias):
    announce("gemm streamk noalloc %dx%dx%d" % (M, N, K))
    g = torch.Generator(device="cuda").manual_seed(seed)
    A = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    Bt = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(N, device="cuda", generator=g) * 0.5).to(torch.bfloat16) if bias else None
    nbytes, ncnt = ops.gemm_streamk_workspace(M, N, K)
    assert nbytes > 0, "the shape must split K"
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    cnt = torch.zeros(ncnt, dtype=torch.int32, device="cuda")
    ref = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops.gemm_streamk(A, Bt, ref, ws, cnt, bias=b)
    pad = torch.full((M + 4, N + 8), 5.0, dtype=torch.bfloat16, device="cuda")
    C = pad[:M, :N]
    ops.gemm_streamk_noalloc(A, Bt, C, bias=b)
    torch.cuda.synchronize()
    assert torch.equal(C, ref)
    assert torch.all(pad[M:] == 5.0) and torch.all(pad[:, N:] == 5.0)
    rows = torch.arange(0, M, max(1, M // 32))
    want = O.gemm(A[rows].float().cpu(), Bt.float().cpu().t(), bias=b.float().cpu() if bias else None)
    err = (C[rows].float().cpu() - want).abs()
    assert bool((err <= 2e-2 + 1e-2 * want.abs()).all()), float(err.max())


def test_noalloc_matches_workspace_entry_two_calls(gpu):
    # 2048x896x4864: 32 tiles in four pieces (32 MiB of partials), then a
    # smaller split on the same scratch: 1024x512x4096, 8 tiles (8 MiB)
    _case(2048, 896, 4864, 70, True)
    _case(1024, 512, 4096, 71, False)
    # and the larger one again after the smaller
    _case(2048, 896, 4864, 72, False)


def test_noalloc_refuses_a_split_beyond_the_scratch(gpu):
    M, N, K = 2048, 2048, 32768  # 64 MiB of partials
    assert ops.gemm_streamk_workspace(M, N, K)[0] > 48 << 20
    A = torch.zeros(M, K, dtype=torch.bfloat16, device="cuda")
    Bt = torch.zeros(N, K, dtype=torch.bfloat16, device="cuda")
    C = torch.full((M, N), 3.0, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="scratch holds"):
        ops.gemm_streamk_noalloc(A, Bt, C)
    torch.cuda.synchronize()
    assert torch.all(C == 3.0)
