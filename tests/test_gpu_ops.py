"""Op-level parity of the HIP kernels (through the C ABI) against the oracle.

Tolerance for bf16 outputs: |gpu - oracle| <= 2e-2 + 1e-2 * |oracle|
(the task's max-abs 2e-2 / relative 1e-2); integer, byte and copy work
bit-exact; the relay split bit-exact against the unsplit kernel.
"""

import os

import numpy as np
import pytest
import torch

from kernrelay_amd import ops
from oracle import ops as O
from tests.conftest import announce

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def close(gpu, ref, atol=ATOL, rtol=RTOL):
    g = gpu.float().cpu()
    r = ref.float().cpu()
    err = (g - r).abs()
    bound = atol + rtol * r.abs()
    bad = err > bound
    i = int((err - bound).flatten().argmax())
    assert not bool(bad.any()), "max err %.4g at flat index %d (ref %.4g gpu %.4g), %d bad" % (
        float(err.max()), i, float(r.flatten()[i]), float(g.flatten()[i]), int(bad.sum()))


def rand(shape, std=1.0, seed=0, dt=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dt)


@pytest.mark.parametrize("M,N,K", [(256, 512, 512), (100, 200, 72), (512, 640, 1024), (64, 1024, 4096),
                                   (2048, 4608, 3584)])
def test_gemm_matches_oracle(gpu, M, N, K):
    announce("gemm %dx%dx%d" % (M, N, K))
    A = rand((M, K), 1.0, 1)
    W = rand((K, N), 0.02, 2)                       # weight_t layout [K, N]
    ref = O.gemm(A.float(), W.float())
    Bt = W.t().contiguous().cuda()
    C = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops.gemm(A.cuda(), Bt, C)
    torch.cuda.synchronize()
    close(C, ref)


def test_gemm_fp16_and_bias(gpu):
    announce("gemm fp16 + bias")
    M, N, K = 256, 384, 256
    A = rand((M, K), 1.0, 3, torch.float16)
    W = rand((K, N), 0.05, 4, torch.float16)
    b = rand((N,), 0.5, 5, torch.float16)
    ref = O.gemm(A.float(), W.float(), b.float(), dt=torch.float16)
    C = torch.empty(M, N, dtype=torch.float16, device="cuda")
    ops.gemm(A.cuda(), W.t().contiguous().cuda(), C, bias=b.cuda())
    torch.cuda.synchronize()
    close(C, ref)
    # bias applied to the rounded product: exactly rnd(rnd(acc) + b) of the GPU's own acc
    C0 = torch.empty_like(C)
    ops.gemm(A.cuda(), W.t().contiguous().cuda(), C0)
    torch.cuda.synchronize()
    assert torch.equal(C.cpu(), (C0.cpu().float() + b.float()).to(torch.float16))


def test_gemm_tiles_bit_exact(gpu):
    """Every macro-tile shape runs the same MFMA and K order: identical bits."""
    announce("gemm tile variants")
    M, N, K = 512, 768, 1536
    A = rand((M, K), 1.0, 6).cuda()
    Bt = rand((N, K), 0.02, 7).cuda()
    outs = []
    for bm in (256, 192, 128, 64):  # 192: three row blocks of 192 (the last 128 rows in bounds)
        C = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        ops.gemm(A, Bt, C, bm=bm)
        outs.append(C)
    torch.cuda.synchronize()
    for c in outs[1:]:
        assert torch.equal(outs[0], c)
    # row slices computed alone equal the rows of the full product
    C2 = torch.empty(128, N, dtype=torch.bfloat16, device="cuda")
    ops.gemm(A[256:384], Bt, C2)
    torch.cuda.synchronize()
    assert torch.equal(C2, outs[0][256:384])


def test_gemm_192_rows_qkv_shape(gpu):
    """The q/k/v projection shape 2048x4608x3584 (+bias) runs 192x256 tiles
    (198 tiles fill 75% of the device against 144 256x256 tiles' 56%): the
    same bits as 256x256 tiles, the oracle's values, nothing written outside
    C; a ragged M (1000 rows: a partial last row block) too."""
    announce("gemm 192x256 q/k/v shape")
    for M in (2048, 1000):
        N, K = 4608, 3584
        A = rand((M, K), 1.0, 60).cuda()
        Bt = rand((N, K), 0.02, 61).cuda()
        b = rand((N,), 0.5, 62).cuda()
        pad = torch.full((M + 4, N + 8), 5.0, dtype=torch.bfloat16, device="cuda")
        C = pad[:M, :N]
        ops.gemm(A, Bt, C, bias=b)
        ref = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        ops.gemm(A, Bt, ref, bias=b, bm=256)
        torch.cuda.synchronize()
        assert torch.equal(C, ref)
        assert torch.all(pad[M:] == 5.0) and torch.all(pad[:, N:] == 5.0)
        rows = slice(0, M, 97)
        close(C[rows].cpu(), O.gemm(A[rows].cpu(), Bt.cpu().t(), bias=b.cpu()))


@pytest.mark.parametrize("op", ["gelu", "silu"])
def test_unary_ops(gpu, op):
    announce("elementwise " + op)
    x = rand((300, 1024), 2.0, 8)
    y = torch.empty(300, 1024, dtype=torch.bfloat16, device="cuda")
    ops.elementwise(op, x.cuda(), y)
    torch.cuda.synchronize()
    ref = O.gelu_tanh(x.float()) if op == "gelu" else O.silu(x.float())
    close(y, ref, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("op", ["mul", "add", "swiglu"])
def test_binary_ops(gpu, op):
    announce("elementwise " + op)
    a = rand((257, 896), 2.0, 9)
    b = rand((257, 896), 1.0, 10)
    y = torch.empty(257, 896, dtype=torch.bfloat16, device="cuda")
    ops.elementwise(op, a.cuda(), y, x1=b.cuda())
    torch.cuda.synchronize()
    ref = {"mul": O.mul, "add": O.add, "swiglu": O.swiglu}[op](a.float(), b.float())
    close(y, ref, atol=1e-2, rtol=1e-2)


def test_swiglu_interleaved_matches_plain(gpu):
    announce("swiglu_gu")
    rows, I = 128, 1024
    g = rand((rows, I), 2.0, 11)
    u = rand((rows, I), 1.0, 12)
    gu = torch.stack([g.reshape(rows, I // 8, 8), u.reshape(rows, I // 8, 8)], dim=2).reshape(rows, 2 * I)
    y1 = torch.empty(rows, I, dtype=torch.bfloat16, device="cuda")
    y2 = torch.empty_like(y1)
    ops.elementwise("swiglu_gu", gu.contiguous().cuda(), y1, rows=rows, cols=I)
    ops.elementwise("swiglu", g.cuda(), y2, x1=u.cuda())
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


def test_cast_bf16_to_f16_exhaustive(gpu):
    """All 65536 bf16 patterns; reference is numpy's fp32->fp16 (round to nearest even)."""
    announce("cast exhaustive")
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    x = bits.view(torch.bfloat16).reshape(512, 128)
    y = torch.empty(512, 128, dtype=torch.float16, device="cuda")
    ops.elementwise("cast", x.cuda(), y)
    torch.cuda.synchronize()
    ref = x.float().numpy().astype(np.float16)
    got = y.cpu().numpy()
    nan_r, nan_g = np.isnan(ref), np.isnan(got)
    assert np.array_equal(nan_r, nan_g)
    assert np.array_equal(ref[~nan_r].view(np.uint16), got[~nan_g].view(np.uint16))


def test_cast_f16_to_bf16_exhaustive(gpu):
    """All 65536 fp16 patterns rounded to bf16 (every 16-bit store of the
    kernels goes through the same f32 -> bf16 conversion): round to nearest
    even, ties included, against torch's conversion of the exact values."""
    announce("cast f16->bf16 exhaustive")
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    x = bits.view(torch.float16).reshape(512, 128)
    y = torch.empty(512, 128, dtype=torch.bfloat16, device="cuda")
    ops.elementwise("cast", x.cuda(), y)
    torch.cuda.synchronize()
    ref = x.float().to(torch.bfloat16)
    nan = torch.isnan(ref)
    assert torch.equal(torch.isnan(y.cpu()), nan)
    assert torch.equal(y.cpu()[~nan].view(torch.int16), ref[~nan].view(torch.int16))


def test_cast_f16_to_f32(gpu):
    announce("cast f16->f32")
    x = rand((64, 256), 3.0, 13, torch.float16)
    y = torch.empty(64, 256, dtype=torch.float32, device="cuda")
    ops.elementwise("cast", x.cuda(), y)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), x.float())


@pytest.mark.parametrize("cols", [4096, 2048, 512, 128, 104])
def test_softmax(gpu, cols):
    announce("softmax cols=%d" % cols)
    x = rand((333, cols), 3.0, 14)
    y = torch.empty(333, cols, dtype=torch.bfloat16, device="cuda")
    ops.rowop("softmax", x.cuda(), y)
    torch.cuda.synchronize()
    close(y, O.softmax(x.float()), atol=1e-3, rtol=1e-2)
    s = y.float().sum(-1).cpu()
    assert torch.all((s - 1).abs() < cols * 2 ** -8)


@pytest.mark.parametrize("cols", [3584, 896, 4096, 128, 64])
def test_rmsnorm_and_add_rmsnorm(gpu, cols):
    announce("rmsnorm cols=%d" % cols)
    a = rand((200, cols), 1.0, 15)
    b = rand((200, cols), 1.0, 16)
    g = (1 + rand((cols,), 0.02, 17).float()).to(torch.bfloat16)
    y = torch.empty(200, cols, dtype=torch.bfloat16, device="cuda")
    s = torch.empty_like(y)
    rstd = torch.empty(200, dtype=torch.float32, device="cuda")
    ops.rowop("add_rmsnorm", a.cuda(), y, x1=b.cuda(), gamma=g.cuda(), sum_out=s, rstd_out=rstd, eps=1e-6)
    torch.cuda.synchronize()
    ry, rs, rr = O.add_rmsnorm(a.float(), b.float(), g.float(), 1e-6)
    assert torch.equal(s.cpu().float(), rs)
    close(y, ry)
    assert torch.allclose(rstd.cpu(), rr, rtol=1e-5)
    y2 = torch.empty_like(y)
    ops.rowop("rmsnorm", s, y2, gamma=g.cuda(), eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(y2, y)  # fused and separate paths agree bit for bit


@pytest.mark.parametrize("cols,dt", [(2048, torch.float16), (3584, torch.bfloat16), (896, torch.bfloat16),
                                     (128, torch.float16), (8192, torch.bfloat16)])
def test_layernorm(gpu, cols, dt):
    """LayerNorm (aclnnLayerNorm, reference exec/runtime/op_impl.cpp:237-254:
    weight, bias, eps 1e-5) against the oracle, one-wave rows, 16-lane rows and
    whole-workgroup rows."""
    announce("layernorm cols=%d %s" % (cols, dt))
    rows = 333
    x = rand((rows, cols), 2.0, 81, dt) + 0.25
    w, b = rand((cols,), 1.0, 82, dt), rand((cols,), 1.0, 83, dt)
    y = torch.empty(rows, cols, dtype=dt, device="cuda")
    xc = x.to(dt).cuda()
    ops.rowop("layernorm", xc, y, x1=b.cuda(), gamma=w.cuda(), eps=1e-5)
    torch.cuda.synchronize()
    close(y, O.layernorm(x.float(), w.float(), b.float(), 1e-5, dt))


def test_rope(gpu):
    announce("rope")
    S, Hh, D = 160, 3, 128
    x = rand((S, Hh, D), 1.0, 18)
    cos, sin = O.rope_tables(4096, D, 1e6)
    xg = x.clone().cuda()
    ops.rope(xg, S, Hh, D, cos[:S].contiguous().cuda(), sin[:S].contiguous().cuda())
    torch.cuda.synchronize()
    close(xg, O.rope(x.float(), cos[:S], sin[:S]), atol=1e-2, rtol=1e-2)


def test_embedding(gpu):
    announce("embedding")
    table = rand((1000, 256), 0.02, 19)
    ids = torch.randint(0, 1000, (77,), generator=torch.Generator().manual_seed(1))
    out = torch.empty(77, 256, dtype=torch.bfloat16, device="cuda")
    ops.embedding(table.cuda(), ids.cuda(), out)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), table[ids])


@pytest.mark.parametrize("S,HQ,HKV,D", [(128, 2, 2, 64), (256, 4, 2, 128), (200, 14, 2, 64), (384, 4, 1, 128),
                                         (1000, 3, 1, 128), (2048, 28, 4, 128), (2048, 64, 8, 128)])
def test_attention(gpu, S, HQ, HKV, D):
    """Against the oracle. The grids up to 28 heads at 2048 run the 8-wave
    key-half kernel; 64 heads at 2048 (1024 workgroups, more than one
    resident round) the 4-wave kernel."""
    announce("attention S=%d HQ=%d HKV=%d D=%d" % (S, HQ, HKV, D))
    q = rand((S, HQ, D), 1.0, 20)
    k = rand((S, HKV, D), 1.0, 21)
    v = rand((S, HKV, D), 1.0, 22)
    out = torch.empty(S, HQ, D, dtype=torch.bfloat16, device="cuda")
    ops.attention(q.cuda(), k.cuda(), v.cuda(), out, S, HQ, HKV, D)
    torch.cuda.synchronize()
    close(out, O.attention(q.float(), k.float(), v.float()))


@pytest.mark.parametrize("S,HQ,HKV,D,dt", [(4096, 64, 8, 64, torch.bfloat16), (512, 6, 3, 128, torch.bfloat16),
                                            (300, 6, 3, 64, torch.bfloat16), (1024, 8, 2, 128, torch.float16),
                                            (4096, 64, 8, 64, torch.float16)])
def test_attention_kernel_variants(gpu, S, HQ, HKV, D, dt):
    """Kernel variants the model shapes leave out, against the oracle on the
    first and last query-head groups: the 4-wave kernel at head size 64 (4096
    x 64 heads: 4096 workgroups, more than one resident round), the plain
    workgroup order where HKV neither divides nor is divided by the 8 XCDs
    (HKV 3), and fp16 inputs and outputs (fp16 MFMA, P rounded to fp16)."""
    announce("attention variant S=%d HQ=%d HKV=%d D=%d %s" % (S, HQ, HKV, D, dt))
    q = rand((S, HQ, D), 1.0, 40, dt)
    k = rand((S, HKV, D), 1.0, 41, dt)
    v = rand((S, HKV, D), 1.0, 42, dt)
    out = torch.empty(S, HQ, D, dtype=dt, device="cuda")
    ops.attention(q.cuda(), k.cuda(), v.cuda(), out, S, HQ, HKV, D)
    torch.cuda.synchronize()
    rep = HQ // HKV
    for g in sorted({0, HKV - 1}):
        hs = slice(g * rep, (g + 1) * rep)
        ref = O.attention(q[:, hs].float(), k[:, g:g + 1].float(), v[:, g:g + 1].float(), dt=dt)
        close(out[:, hs], ref)


@pytest.mark.parametrize("S,HQ,HKV,D", [(2048, 7, 1, 64), (1500, 3, 1, 128), (4096, 4, 2, 64), (1100, 2, 2, 64)])
def test_attention_split(gpu, S, HQ, HKV, D):
    """Long causal rows split across workgroups (query blocks of more than 16
    key blocks: two to four pieces summed in piece order by the last piece):
    matches the oracle and the unsplit kernel within the bf16 bar, repeats bit
    for bit, leaves its counters zero."""
    announce("attention split S=%d HQ=%d HKV=%d D=%d" % (S, HQ, HKV, D))
    nbytes, ncnt = ops.attention_workspace(S, HQ, D)
    assert nbytes > 0 and ncnt > 0
    q = rand((S, HQ, D), 1.0, 30).cuda()
    k = rand((S, HKV, D), 1.0, 31).cuda()
    v = rand((S, HKV, D), 1.0, 32).cuda()
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    cnt = torch.zeros(ncnt, dtype=torch.int32, device="cuda")
    out = torch.empty(S, HQ, D, dtype=torch.bfloat16, device="cuda")
    ops.attention_split(q, k, v, out, S, HQ, HKV, D, ws, cnt)
    first = out.clone()
    for _ in range(2):
        out.zero_()
        ops.attention_split(q, k, v, out, S, HQ, HKV, D, ws, cnt)
        torch.cuda.synchronize()
        assert torch.equal(out, first)
    assert int(cnt.abs().sum()) == 0
    plain = torch.empty_like(out)
    ops.attention(q, k, v, plain, S, HQ, HKV, D)
    close(out, plain)
    close(out, O.attention(q.cpu().float(), k.cpu().float(), v.cpu().float()))


def test_attention_split_workspace():
    """Nothing to split at or below 16 key blocks per query row, nor when the
    unsplit grid has more workgroups than half the CUs (256 on MI355X, the
    count the library also falls back to without a device)."""
    assert ops.attention_workspace(1024, 14, 64) == (0, 0)
    assert ops.attention_workspace(2048, 28, 128) == (0, 0)
    assert ops.attention_workspace(2048, 14, 64) == (0, 0)
    b, c = ops.attention_workspace(2048, 7, 64)
    assert c == 8 * 7 and b == 8 * 7 * 2 * 9 * 256 * 16


def test_attention_strided_views(gpu):
    """q/k/v read in place from one fused [S, (HQ+2HKV)*D] buffer."""
    announce("attention strided")
    S, HQ, HKV, D = 256, 4, 2, 64
    qkv = rand((S, (HQ + 2 * HKV) * D), 1.0, 23)
    q = qkv[:, : HQ * D].reshape(S, HQ, D)
    k = qkv[:, HQ * D:(HQ + HKV) * D].reshape(S, HKV, D)
    v = qkv[:, (HQ + HKV) * D:].reshape(S, HKV, D)
    g = qkv.cuda()
    ld = (HQ + 2 * HKV) * D
    out = torch.empty(S, HQ, D, dtype=torch.bfloat16, device="cuda")
    ops.attention(g, g[:, HQ * D:], g[:, (HQ + HKV) * D:], out, S, HQ, HKV, D, ldq=ld, ldk=ld, ldv=ld)
    torch.cuda.synchronize()
    close(out, O.attention(q.float(), k.float(), v.float()))


def test_relay_gemm_to_consumer_bit_exact(gpu):
    """Producer GEMM releases k row tiles from its epilogue on one stream; a
    GELU consumer on a second stream spins per tile. Output equals the unsplit
    kernels bit for bit, every edge reports status 1, and the counters keep
    counting across repeated runs without a host reset."""
    announce("relay gemm->gelu k=4")
    M, N, K, k = 1024, 1024, 512, 4
    A = rand((M, K), 1.0, 24).cuda()
    Bt = rand((N, K), 0.02, 25).cuda()
    ref_c = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ref_y = torch.empty_like(ref_c)
    ops.gemm(A, Bt, ref_c)
    ops.elementwise("gelu", ref_c, ref_y)
    torch.cuda.synchronize()

    ctrl = torch.zeros(k * ops.CTRL_WORDS, dtype=torch.int32, device="cuda")
    C = torch.empty_like(ref_c)
    Y = torch.empty_like(ref_c)
    sp, sc = ops.QueueStream(), ops.QueueStream()
    runs = 3
    try:
        for _ in range(runs):
            C.zero_()
            Y.zero_()
            torch.cuda.synchronize()
            w = ops.make_wait(ctrl, 0, 0, M // k, adv=(0, k))
            # consumer launched first: it must wait for the producer's releases
            ops.elementwise("gelu", C, Y, tile_rows=M // k, grid=32, wait=w, stream=sc)
            ops.gemm(A, Bt, C, pub=ops.make_pub(ctrl, 0, M // k), stream=sp)
            torch.cuda.synchronize()
            assert torch.equal(C, ref_c)
            assert torch.equal(Y, ref_y)
    finally:
        sp.close()
        sc.close()
    blk = ctrl.cpu().reshape(k, ops.CTRL_WORDS)
    assert torch.all(blk[:, 0] == runs) and torch.all(blk[:, 1] == runs)   # published == consumed
    assert torch.all(blk[:, 2] == 1)                                        # status ok
    assert torch.all(blk[:, 3] == 0) and torch.all(blk[:, 4] == 0)          # tickets reset


def test_relay_gemm_waits_on_consumer_tiles(gpu):
    """The GEMM as a relay consumer: a GELU releases k row tiles on one
    stream; a GEMM launched first on another stream waits, per workgroup, for
    the tiles its rows of A come from. C equals GELU-then-GEMM run serially bit
    for bit, and each tile is consumed exactly once per run with status 1."""
    announce("relay gelu->gemm k=4 (fused gemm wait)")
    M, N, K, k = 1024, 768, 512, 4
    X = rand((M, K), 1.0, 26).cuda()
    Bt = rand((N, K), 0.02, 27).cuda()
    ref_a = torch.empty(M, K, dtype=torch.bfloat16, device="cuda")
    ref_c = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops.elementwise("gelu", X, ref_a)
    ops.gemm(ref_a, Bt, ref_c)
    torch.cuda.synchronize()

    ctrl = torch.zeros(k * ops.CTRL_WORDS, dtype=torch.int32, device="cuda")
    A = torch.empty_like(ref_a)
    C = torch.empty_like(ref_c)
    sp, sc = ops.QueueStream(), ops.QueueStream()
    runs = 3
    try:
        for _ in range(runs):
            A.zero_()
            C.zero_()
            torch.cuda.synchronize()
            w = ops.make_wait(ctrl, 0, 0, M // k, adv=(0, k))
            ops.gemm(A, Bt, C, wait=w, stream=sc)
            ops.elementwise("gelu", X, A, tile_rows=M // k, pub=ops.make_pub(ctrl, 0, M // k), stream=sp)
            torch.cuda.synchronize()
            assert torch.equal(A, ref_a)
            assert torch.equal(C, ref_c)
    finally:
        sp.close()
        sc.close()
    blk = ctrl.cpu().reshape(k, ops.CTRL_WORDS)
    assert torch.all(blk[:, 0] == runs) and torch.all(blk[:, 1] == runs)
    assert torch.all(blk[:, 2] == 1)
    assert torch.all(blk[:, 3] == 0) and torch.all(blk[:, 4] == 0)


@pytest.mark.parametrize("k", [1, 2, 4])
def test_gemm_swiglu_tail_bit_exact(gpu, k):
    """The SwiGLU consumer appended to the gate/up GEMM's launch (waiting on
    the GEMM's own relay tiles) equals the GEMM followed by the standalone
    swiglu_gu kernel bit for bit, on every one of several runs (the counters
    carry over), and consumes each tile once with status 1."""
    announce("gemm+swiglu tail k=%d" % k)
    M, I, K = 1024, 1536, 512
    A = rand((M, K), 1.0, 30).cuda()
    Bt = rand((2 * I, K), 0.05, 31).cuda()
    ref_c = torch.empty(M, 2 * I, dtype=torch.bfloat16, device="cuda")
    ref_a = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    ops.gemm(A, Bt, ref_c)
    ops.elementwise("swiglu_gu", ref_c, ref_a, rows=M, cols=I)
    torch.cuda.synchronize()
    ctrl = torch.zeros(k * ops.CTRL_WORDS, dtype=torch.int32, device="cuda")
    C = torch.empty_like(ref_c)
    act = torch.empty_like(ref_a)
    runs = 3
    for _ in range(runs):
        C.zero_()
        act.zero_()
        ops.gemm_swiglu(A, Bt, C, act, ops.make_pub(ctrl, 0, M // k))
        torch.cuda.synchronize()
        assert torch.equal(C, ref_c)
        assert torch.equal(act, ref_a)
    blk = ctrl.cpu().reshape(k, ops.CTRL_WORDS)
    assert torch.all(blk[:, 0] == runs) and torch.all(blk[:, 1] == runs)
    assert torch.all(blk[:, 2] == 1) and torch.all(blk[:, 3] == 0) and torch.all(blk[:, 4] == 0)


def test_relay_wait_bound_reports_timeout(gpu):
    """A wait on a tile nobody publishes ends at its spin bound with status 2."""
    announce("relay timeout status")
    ctrl = torch.zeros(2 * ops.CTRL_WORDS, dtype=torch.int32, device="cuda")
    w = ops.make_wait(ctrl, 0, 0, 64, adv=(0, 1), max_spins=1000)
    ops.wait(w, 0, 64)
    torch.cuda.synchronize()
    blk = ctrl.cpu().reshape(2, ops.CTRL_WORDS)
    assert int(blk[0, 2]) == 2 and int(blk[0, 1]) == 1 and int(blk[0, 5]) == 0
    # a later publish + wait succeeds and reports 1
    ops.publish(ops.make_pub(ctrl, 0, 64), 0)
    ops.publish(ops.make_pub(ctrl, 0, 64), 0)
    ops.wait(w, 0, 64)
    torch.cuda.synchronize()
    blk = ctrl.cpu().reshape(2, ops.CTRL_WORDS)
    assert int(blk[0, 2]) == 1 and int(blk[0, 1]) == 2 and int(blk[0, 0]) == 2


@pytest.mark.parametrize("M,N,K", [(2048, 37888, 3584), (2048, 152064, 3584), (1000, 37888, 512)])
def test_gemm_wave_tail_split_bit_exact(gpu, M, N, K):
    """A 256x256 grid that is not a whole number of rounds on the device runs
    the columns of its partial last round as a second launch of 192x256
    tiles (gate/up 2048x37888: 1184 tiles = 4 rounds + 160; lm_head
    2048x152064: 18 rounds + 144; a ragged M of 1000). The product equals
    the single-launch grid (a forced 256-row tile, never split) bit for bit,
    the SwiGLU epilogue's act equals the standalone kernel on that product,
    and nothing outside C or act is written."""
    announce("gemm wave-tail split %dx%dx%d" % (M, N, K))
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    A = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    Bt = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    ref = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops.gemm(A, Bt, ref, bm=256)
    pad = torch.full((M + 8, N + 16), 7.0, dtype=torch.bfloat16, device="cuda")
    C = pad[:M, :N]
    ops.gemm(A, Bt, C)
    torch.cuda.synchronize()
    assert torch.equal(C, ref)
    assert bool(torch.all(pad[M:] == 7.0)) and bool(torch.all(pad[:, N:] == 7.0))
    del pad, C
    if N > 40000:
        return
    I = N // 2
    ref_a = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    ops.elementwise("swiglu_gu", ref, ref_a, rows=M, cols=I)
    apad = torch.full((M + 8, I + 16), 7.0, dtype=torch.bfloat16, device="cuda")
    act = apad[:M, :I]
    ops.gemm_swiglu_epilogue(A, Bt, act)
    torch.cuda.synchronize()
    assert torch.equal(act, ref_a)
    assert bool(torch.all(apad[M:] == 7.0)) and bool(torch.all(apad[:, I:] == 7.0))


@pytest.mark.parametrize("M,I,K", [(1024, 1536, 512), (300, 512, 256), (2048, 4864, 896)])
def test_gemm_swiglu_epilogue_bit_exact(gpu, M, I, K):
    """SwiGLU applied in the gate/up GEMM's epilogue (the in-register relay)
    equals the GEMM followed by the standalone swiglu_gu kernel bit for bit
    (ragged M included) and writes nothing outside act; the product and its
    SwiGLU each match the oracle."""
    announce("gemm swiglu epilogue %dx%dx%d" % (M, I, K))
    A = rand((M, K), 1.0, 40).cuda()
    Bt = rand((2 * I, K), 0.05, 41).cuda()
    ref_c = torch.empty(M, 2 * I, dtype=torch.bfloat16, device="cuda")
    ref_a = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    ops.gemm(A, Bt, ref_c)
    ops.elementwise("swiglu_gu", ref_c, ref_a, rows=M, cols=I)
    pad = torch.full((M + 8, I + 16), 7.0, dtype=torch.bfloat16, device="cuda")
    act = pad[:M, :I]
    for _ in range(2):
        act.zero_()
        ops.gemm_swiglu_epilogue(A, Bt, act)
        torch.cuda.synchronize()
        assert torch.equal(act, ref_a)
    assert torch.all(pad[M:] == 7.0) and torch.all(pad[:, I:] == 7.0)
    # each stage against the oracle at its own tolerance: the product, then
    # SwiGLU of that product (four bf16 roundings in a row turn a one-ulp
    # difference of the fp32 sum order into several ulps of act)
    close(ref_c, O.gemm(A.cpu(), Bt.cpu().t()))
    g = ref_c.cpu().view(M, I // 8, 2, 8)
    close(act, O.swiglu(g[:, :, 0, :].reshape(M, I), g[:, :, 1, :].reshape(M, I)))


@pytest.mark.parametrize("M,N,K,bias,wgs", [(2048, 3584, 18944, False, None), (1920, 3584, 16384, True, None),
                                            (1000, 2560, 16384, True, None),
                                            (2048, 896, 4864, True, None), (2048, 4608, 3584, True, 256),
                                            (2048, 3584, 3584, False, 256)])
def test_gemm_streamk(gpu, M, N, K, bias, wgs):
    """Stream-K: the default exact split of K (the down shape: two pieces per
    tile; 1920 rows: two pieces on 256x256 tiles whose last row of tiles is
    half outside M; a ragged one: four) and, forced over 256 workgroups, the uneven
    spread (the q/k/v and o shapes: pieces of unequal length, up to three per
    tile): matches the oracle and the data-parallel kernel within the bf16
    bar, repeats bit for bit (fixed piece order), leaves its counters zero
    and writes nothing outside C."""
    announce("gemm stream-K %dx%dx%d bias=%s wgs=%s" % (M, N, K, bias, wgs))
    if wgs is not None:
        os.environ["KR_GEMM_SK_WGS"] = str(wgs)
    try:
        _streamk_case(M, N, K, bias)
    finally:
        os.environ.pop("KR_GEMM_SK_WGS", None)


def test_gemm_streamk_policy(gpu):
    """The default plan splits K where the data-parallel tiling fills under
    60% of the device and whole pieces of >= 16 K stages fill idle CUs
    (2048x896x4864: 32 tiles of 76 stages, four pieces), or under 90% with K
    of >= 256 stages (the 7B down shape: 256x128 tiles fill 87.5%; two pieces
    of 148 stages on 112 tiles of 256x256). The other 7B shapes (o: 56
    stages; q/k/v: 144 tiles leave no room for a second piece), short K (14
    stages) and a full-device shape do not split."""
    assert ops.gemm_streamk_workspace(2048, 896, 4864) == (32 * 4 * 256 * 256 * 4, 32)
    assert ops.gemm_streamk_workspace(2048, 896, 896) == (0, 0)
    assert ops.gemm_streamk_workspace(2048, 3584, 18944) == (112 * 2 * 256 * 256 * 4, 112)
    assert ops.gemm_streamk_workspace(1920, 3584, 16384) == (112 * 2 * 256 * 256 * 4, 112)
    assert ops.gemm_streamk_workspace(2048, 3584, 16320) == (0, 0)  # 255 stages: below the long-K bar
    assert ops.gemm_streamk_workspace(2048, 3584, 3584) == (0, 0)
    assert ops.gemm_streamk_workspace(2048, 4608, 3584) == (0, 0)
    assert ops.gemm_streamk_workspace(4096, 4096, 18944) == (0, 0)


def _streamk_case(M, N, K, bias):
    nbytes, ncnt = ops.gemm_streamk_workspace(M, N, K)
    assert nbytes > 0 and ncnt > 0
    A = rand((M, K), 1.0, 50).cuda()
    Bt = rand((N, K), 0.02, 51).cuda()
    b = rand((N,), 0.5, 52).cuda() if bias else None
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    cnt = torch.zeros(ncnt, dtype=torch.int32, device="cuda")
    pad = torch.full((M + 4, N + 8), 3.0, dtype=torch.bfloat16, device="cuda")
    C = pad[:M, :N]
    ops.gemm_streamk(A, Bt, C, ws, cnt, bias=b)
    first = C.clone()
    for _ in range(2):
        C.zero_()
        ops.gemm_streamk(A, Bt, C, ws, cnt, bias=b)
        torch.cuda.synchronize()
        assert torch.equal(C, first)
    assert int(cnt.abs().sum()) == 0
    assert torch.all(pad[M:] == 3.0) and torch.all(pad[:, N:] == 3.0)
    dp = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops.gemm(A, Bt, dp, bias=b)
    close(C, dp)
    close(C, O.gemm(A.cpu(), Bt.cpu().t(), bias=b.cpu() if bias else None))


@pytest.mark.parametrize("M,N,K,k,streamk", [(2048, 3584, 3584, 1, False), (2048, 3584, 3584, 4, False),
                                             (2048, 3584, 18944, 8, False), (2048, 3584, 18944, 4, True),
                                             (2048, 896, 4864, 4, True),
                                             (2048, 896, 4864, 2, False), (256, 256, 512, 4, False),
                                             (512, 4096, 1024, 2, False), (8192, 4096, 512, 4, False)])
def test_gemm_add_rmsnorm_relay_bit_exact(gpu, M, N, K, k, streamk):
    """The row-tiled relay of a projection to its Add+RMSNorm consumer: the
    GEMM releases k row tiles and its own workgroups normalise each released
    tile. y, the residual sum and rstd equal the GEMM followed by the
    standalone Add+RMSNorm kernel bit for bit (the 7B o and down shapes, the
    latter also with its two-piece K split, the Qwen2.5-0.5B down shape with
    its four-piece K split, 64-row tiles); every
    relay tile's block ends with published == consumed == runs and status 1
    over repeated runs without a host reset; y matches the oracle's
    Add+RMSNorm of the stored product. 8192x4096 with k=4 is a grid of two
    rounds (512 workgroups of 256x256, 128 per relay tile) that runs in
    relay-tile order: the later tiles' workgroups start only as the earlier
    tiles' finish their Add+RMSNorm."""
    announce("gemm+add_rmsnorm relay %dx%dx%d k=%d streamk=%s" % (M, N, K, k, streamk))
    g = torch.Generator(device="cuda").manual_seed(60)
    A = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    Bt = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    res = torch.randn(M, N, device="cuda", generator=g).to(torch.bfloat16)
    gamma = (1.0 + 0.1 * torch.randn(N, device="cuda", generator=g)).to(torch.bfloat16)
    ws = cnt = None
    if streamk:
        nb, nc = ops.gemm_streamk_workspace(M, N, K)
        assert nb > 0
        ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
        cnt = torch.zeros(nc, dtype=torch.int32, device="cuda")
    ref_c = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    if streamk:
        ops.gemm_streamk(A, Bt, ref_c, ws, cnt)
    else:
        ops.gemm(A, Bt, ref_c)
    ref_y, ref_s = torch.empty_like(ref_c), torch.empty_like(ref_c)
    ref_r = torch.empty(M, dtype=torch.float32, device="cuda")
    ops.rowop("add_rmsnorm", res, ref_y, x1=ref_c, gamma=gamma, sum_out=ref_s, rstd_out=ref_r)
    torch.cuda.synchronize()
    ctrl = torch.zeros(k * ops.CTRL_WORDS, dtype=torch.int32, device="cuda")
    C, y, s = torch.empty_like(ref_c), torch.empty_like(ref_c), torch.empty_like(ref_c)
    rstd = torch.empty_like(ref_r)
    runs = 3
    for _ in range(runs):
        for t in (C, y, s, rstd):
            t.zero_()
        ops.gemm_add_rmsnorm(A, Bt, C, res, gamma, y, ops.make_pub(ctrl, 0, M // k), sum_out=s, rstd=rstd,
                             ws=ws, counters=cnt)
        torch.cuda.synchronize()
        assert torch.equal(C, ref_c)
        assert torch.equal(y, ref_y) and torch.equal(s, ref_s) and torch.equal(rstd, ref_r)
    blk = ctrl.cpu().reshape(k, ops.CTRL_WORDS)
    assert torch.all(blk[:, 0] == runs) and torch.all(blk[:, 1] == runs)   # published == consumed
    assert torch.all(blk[:, 2] == 1)                                        # status ok
    assert torch.all(blk[:, 3] == 0) and torch.all(blk[:, 4] == 0)          # tickets reset
    if cnt is not None:
        assert int(cnt.abs().sum()) == 0
    rows = torch.arange(0, M, max(1, M // 64))
    oy, osum, _ = O.add_rmsnorm(res[rows].float().cpu(), ref_c[rows].float().cpu(), gamma.float().cpu(), 1e-6)
    close(y[rows], oy)
    assert torch.equal(s[rows].float().cpu(), osum)


def test_gemm_add_rmsnorm_relay_refuses_unresident_tiles(gpu):
    """A relay tile whose producer workgroups cannot all be resident at once
    (8192 rows x 4096 columns in one tile: 512 workgroups of 256x256 against
    256 CUs) is refused before anything is launched: its consumer would wait
    on workgroups not yet placed."""
    M, N, K = 8192, 4096, 512
    A = torch.zeros(M, K, dtype=torch.bfloat16, device="cuda")
    Bt = torch.zeros(N, K, dtype=torch.bfloat16, device="cuda")
    C = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    res, y = torch.empty_like(C), torch.empty_like(C)
    gamma = torch.ones(N, dtype=torch.bfloat16, device="cuda")
    ctrl = torch.zeros(ops.CTRL_WORDS, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="do not fit the device at once"):
        ops.gemm_add_rmsnorm(A, Bt, C, res, gamma, y, ops.make_pub(ctrl, 0, M))
    torch.cuda.synchronize()
    assert int(ctrl.abs().sum()) == 0
