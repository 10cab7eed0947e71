"""Op-level bindings of libkernrelay.so (include/kr_ops.h) for torch tensors.

torch only supplies device memory and the current stream; every op runs a
hand-written HIP kernel from the library. Calling an op with a CPU tensor or
without the built library raises: there is no CPU fallback.
"""

import ctypes

from . import libapi

KR_BF16, KR_F16, KR_F32 = 0, 1, 2
EW = {"gelu": 0, "silu": 1, "cast": 2, "mul": 3, "add": 4, "swiglu": 5, "swiglu_gu": 6}
ROW = {"softmax": 0, "rmsnorm": 1, "add_rmsnorm": 2, "layernorm": 3}
CTRL_WORDS = 8


class KrWait(ctypes.Structure):
    _fields_ = [("ctrl", ctypes.c_void_p), ("flag0", ctypes.c_int32),
                ("state0", ctypes.c_int32), ("prod_rows", ctypes.c_int32),
                ("row_off", ctypes.c_int32), ("adv_lo", ctypes.c_int32),
                ("adv_hi", ctypes.c_int32), ("max_spins", ctypes.c_uint32)]


class KrPub(ctypes.Structure):
    _fields_ = [("ctrl", ctypes.c_void_p), ("flag0", ctypes.c_int32),
                ("rows_per_tile", ctypes.c_int32), ("arrivals", ctypes.c_int32)]


_BOUND = False


def _lib():
    global _BOUND
    L = libapi.lib()
    if not _BOUND:
        vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        L.kr_ops_last_error.restype = ctypes.c_char_p
        L.kr_ops_last_error.argtypes = []
        L.kr_op_gemm.argtypes = [i32, vp, i64, vp, i64, vp, i64, vp, i32, i32, i32, i32,
                                 ctypes.POINTER(KrWait), ctypes.POINTER(KrPub), vp]
        L.kr_op_elementwise.argtypes = [i32, i32, i32, vp, vp, vp, i32, i32, i32, i32,
                                        ctypes.POINTER(KrWait), ctypes.POINTER(KrPub), vp]
        L.kr_op_rowop.argtypes = [i32, i32, vp, vp, vp, vp, vp, vp, i32, i32, f32, i32, i32,
                                  ctypes.POINTER(KrWait), ctypes.POINTER(KrPub), vp]
        L.kr_op_wait.argtypes = [ctypes.POINTER(KrWait), i32, i32, vp]
        L.kr_op_publish.argtypes = [ctypes.POINTER(KrPub), i32, vp]
        L.kr_op_embedding.argtypes = [vp, vp, vp, i32, i32, i64, vp]
        L.kr_op_rope.argtypes = [i32, vp, i64, i32, i32, i32, vp, vp, vp]
        L.kr_op_attention.argtypes = [i32, vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, f32, vp]
        L.kr_op_attention_workspace.argtypes = [i32, i32, i32, ctypes.POINTER(ctypes.c_size_t),
                                                ctypes.POINTER(ctypes.c_int)]
        L.kr_op_attention_split.argtypes = [i32, vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, f32, vp,
                                            ctypes.c_size_t, vp, i32, vp]
        L.kr_op_transpose.argtypes = [vp, vp, i32, i32, vp]
        L.kr_op_gemm_swiglu.argtypes = [i32, vp, i64, vp, i64, vp, vp, i32, i32, i32, ctypes.POINTER(KrPub),
                                        i32, i32, vp]
        L.kr_op_gemm_swiglu_epilogue.argtypes = [i32, vp, i64, vp, i64, vp, i64, i32, i32, i32, vp]
        L.kr_op_gemm_streamk_workspace.argtypes = [i32, i32, i32, ctypes.POINTER(ctypes.c_size_t),
                                                    ctypes.POINTER(ctypes.c_int)]
        L.kr_op_gemm_streamk.argtypes = [i32, vp, i64, vp, i64, vp, i64, vp, i32, i32, i32, vp, ctypes.c_size_t, vp,
                                         i32, vp]
        L.kr_op_gemm_add_rmsnorm.argtypes = [i32, vp, i64, vp, i64, vp, i32, i32, i32, vp, vp, vp, vp, vp, f32,
                                             ctypes.POINTER(KrPub), ctypes.c_uint32, vp, ctypes.c_size_t, vp, i32, vp]
        L.kr_op_gemm_streamk_noalloc.argtypes = [i32, vp, i64, vp, i64, vp, i64, vp, i32, i32, i32, vp]
        L.kr_op_stream_create.argtypes = []
        L.kr_op_stream_create.restype = vp
        L.kr_op_stream_destroy.argtypes = [vp]
        L.kr_op_stream_destroy.restype = ctypes.c_int
        for name in ("kr_op_gemm", "kr_op_gemm_swiglu", "kr_op_gemm_swiglu_epilogue", "kr_op_gemm_streamk",
                     "kr_op_gemm_add_rmsnorm", "kr_op_gemm_streamk_noalloc",
                     "kr_op_gemm_streamk_workspace", "kr_op_elementwise", "kr_op_rowop", "kr_op_wait", "kr_op_publish",
                     "kr_op_embedding", "kr_op_rope", "kr_op_attention", "kr_op_attention_workspace",
                     "kr_op_attention_split", "kr_op_transpose"):
            getattr(L, name).restype = ctypes.c_int
        _BOUND = True
    return L


def _dt(t):
    import torch
    if t.dtype == torch.bfloat16:
        return KR_BF16
    if t.dtype == torch.float16:
        return KR_F16
    if t.dtype == torch.float32:
        return KR_F32
    raise TypeError("unsupported dtype %s" % t.dtype)


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise RuntimeError("kernrelay ops need device tensors (got a CPU tensor)")
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


class QueueStream:
    """A stream on a hardware queue of its own (kr_op_stream_create): relay
    parties that wait on each other on the device need two of these. Usable
    wherever the op wrappers take a stream."""

    def __init__(self):
        h = _lib().kr_op_stream_create()
        if not h:
            raise RuntimeError("kr_op_stream_create failed: %s" % _lib().kr_ops_last_error().decode())
        self.cuda_stream = h

    def close(self):
        if self.cuda_stream:
            _check(_lib().kr_op_stream_destroy(ctypes.c_void_p(self.cuda_stream)))
            self.cuda_stream = None


def _check(rc):
    if rc != 0:
        raise RuntimeError("kernrelay op failed: %s" % _lib().kr_ops_last_error().decode())


def make_wait(ctrl, flag0, state0, prod_rows, row_off=0, adv=(0, 0), max_spins=0):
    return KrWait(ctypes.c_void_p(ctrl.data_ptr()), flag0, state0, prod_rows, row_off,
                  adv[0], adv[1], max_spins)


def make_pub(ctrl, flag0, rows_per_tile):
    return KrPub(ctypes.c_void_p(ctrl.data_ptr()), flag0, rows_per_tile, 0)


def gemm(A, Bt, C, bias=None, pub=None, bm=0, wait=None, stream=None):
    """C[M,N] = A[M,K] @ Bt[N,K]^T (+bias), bf16/f16 in and out. `wait`: each
    workgroup first waits for the relay tiles of A it reads."""
    M, K = A.shape
    N = Bt.shape[0]
    assert Bt.shape[1] == K and C.shape[0] == M and C.shape[1] == N
    _check(_lib().kr_op_gemm(_dt(A), _ptr(A), A.stride(0), _ptr(Bt), Bt.stride(0), _ptr(C), C.stride(0),
                             _ptr(bias), M, N, K, bm, ctypes.byref(wait) if wait else None,
                             ctypes.byref(pub) if pub else None, _stream(stream)))


def gemm_swiglu(A, Bt, C, act, pub, tail_tiles=0, order_rows=0, stream=None):
    """C[M, 2I] = A @ Bt^T released in relay tiles (pub); act[M, I] =
    SwiGLU of C over the first tail_tiles relay tiles (0 = all) by workgroups
    appended to the same launch."""
    M, K = A.shape
    cols = act.shape[1]
    assert Bt.shape == (2 * cols, K) and C.shape == (M, 2 * cols) and act.shape[0] == M
    _check(_lib().kr_op_gemm_swiglu(_dt(A), _ptr(A), A.stride(0), _ptr(Bt), Bt.stride(0), _ptr(C), _ptr(act),
                                    M, cols, K, ctypes.byref(pub), tail_tiles, order_rows, _stream(stream)))


def gemm_add_rmsnorm(A, Bt, C, res, gamma, y, pub, sum_out=None, rstd=None, eps=1e-6, ws=None, counters=None,
                     max_spins=0, stream=None):
    """C = A @ Bt^T released in relay tiles (pub); the launch's own
    workgroups compute Add+RMSNorm(res + C) of each released tile (y, sum_out,
    rstd), the bits of rowop("add_rmsnorm"). ws/counters: stream-K workspace
    (None: data-parallel)."""
    M, K = A.shape
    N = Bt.shape[0]
    assert Bt.shape[1] == K and C.shape == (M, N) and res.shape == (M, N) and y.shape == (M, N)
    # the C entry takes C, res, y and sum_out as packed [M, N] rows and rstd
    # as [M]: a strided view would be read or written with row stride N
    for name, t in (("C", C), ("res", res), ("y", y), ("sum_out", sum_out), ("rstd", rstd), ("gamma", gamma)):
        if t is not None and not t.is_contiguous():
            raise ValueError("gemm_add_rmsnorm: %s must be contiguous" % name)
    if sum_out is not None and sum_out.shape != (M, N):
        raise ValueError("gemm_add_rmsnorm: sum_out must be [M, N]")
    if rstd is not None and rstd.numel() != M:
        raise ValueError("gemm_add_rmsnorm: rstd must hold M values")
    _check(_lib().kr_op_gemm_add_rmsnorm(_dt(A), _ptr(A), A.stride(0), _ptr(Bt), Bt.stride(0), _ptr(C), M, N, K,
                                         _ptr(res), _ptr(gamma), _ptr(y), _ptr(sum_out), _ptr(rstd), ctypes.c_float(eps),
                                         ctypes.byref(pub), ctypes.c_uint32(max_spins), _ptr(ws),
                                         0 if ws is None else ws.numel() * ws.element_size(), _ptr(counters),
                                         0 if counters is None else counters.numel(), _stream(stream)))


def gemm_streamk_workspace(M, N, K):
    """(workspace bytes, counters) a stream-K GEMM of this shape needs; (0, 0)
    when it runs data-parallel."""
    b, c = ctypes.c_size_t(0), ctypes.c_int(0)
    _check(_lib().kr_op_gemm_streamk_workspace(M, N, K, ctypes.byref(b), ctypes.byref(c)))
    return b.value, c.value


def gemm_streamk(A, Bt, C, ws, counters, bias=None, stream=None):
    """C = A @ Bt^T (+bias) split stream-K over the CUs (ws: uint8 device
    tensor, counters: int32 device tensor, zero before the first call)."""
    M, K = A.shape
    N = Bt.shape[0]
    _check(_lib().kr_op_gemm_streamk(_dt(A), _ptr(A), A.stride(0), _ptr(Bt), Bt.stride(0), _ptr(C), C.stride(0),
                                     _ptr(bias), M, N, K, _ptr(ws), ws.numel() * ws.element_size(),
                                     _ptr(counters), counters.numel(), _stream(stream)))


def gemm_streamk_noalloc(A, Bt, C, bias=None, stream=None):
    """gemm_streamk with the library's own scratch (no workspace argument,
    nothing allocated); raises for a split larger than the scratch."""
    M, K = A.shape
    N = Bt.shape[0]
    _check(_lib().kr_op_gemm_streamk_noalloc(_dt(A), _ptr(A), A.stride(0), _ptr(Bt), Bt.stride(0), _ptr(C),
                                             C.stride(0), _ptr(bias), M, N, K, _stream(stream)))


def gemm_swiglu_epilogue(A, Bt, act, stream=None):
    """act[M, I] = SwiGLU of A @ Bt^T (Bt = [2I, K], gate/up interleaved in
    groups of 8 rows), applied in the GEMM's epilogue; the product itself is
    never written."""
    M, K = A.shape
    cols = act.shape[1]
    assert Bt.shape == (2 * cols, K) and act.shape[0] == M
    _check(_lib().kr_op_gemm_swiglu_epilogue(_dt(A), _ptr(A), A.stride(0), _ptr(Bt), Bt.stride(0), _ptr(act),
                                             act.stride(0), M, cols, K, _stream(stream)))


def elementwise(op, x0, y, x1=None, rows=None, cols=None, tile_rows=0, grid=0, wait=None, pub=None,
                stream=None):
    rows = rows if rows is not None else y.shape[0]
    cols = cols if cols is not None else y.shape[-1]
    _check(_lib().kr_op_elementwise(EW[op], _dt(x0), _dt(y), _ptr(x0), _ptr(x1), _ptr(y), rows, cols,
                                    tile_rows, grid, ctypes.byref(wait) if wait else None,
                                    ctypes.byref(pub) if pub else None, _stream(stream)))


def rowop(op, x0, y, x1=None, gamma=None, sum_out=None, rstd_out=None, eps=1e-6, tile_rows=0, grid=0,
          wait=None, pub=None, stream=None):
    rows, cols = y.shape
    _check(_lib().kr_op_rowop(ROW[op], _dt(x0), _ptr(x0), _ptr(x1), _ptr(gamma), _ptr(y), _ptr(sum_out),
                              _ptr(rstd_out), rows, cols, float(eps), tile_rows, grid,
                              ctypes.byref(wait) if wait else None, ctypes.byref(pub) if pub else None,
                              _stream(stream)))


def wait(w, lo, hi, stream=None):
    _check(_lib().kr_op_wait(ctypes.byref(w), lo, hi, _stream(stream)))


def publish(p, tile, stream=None):
    _check(_lib().kr_op_publish(ctypes.byref(p), tile, _stream(stream)))


def embedding(table, ids, out, stream=None):
    rows, cols = out.shape
    _check(_lib().kr_op_embedding(_ptr(table), _ptr(ids), _ptr(out), rows, cols, table.shape[0],
                                  _stream(stream)))


def rope(x, S, heads, D, cos_t, sin_t, ld=None, stream=None):
    _check(_lib().kr_op_rope(_dt(x), _ptr(x), ld if ld is not None else heads * D, S, heads, D,
                             _ptr(cos_t), _ptr(sin_t), _stream(stream)))


def attention(q, k, v, out, S, HQ, HKV, D, scale=None, ldq=0, ldk=0, ldv=0, ldo=0, stream=None):
    scale = scale if scale is not None else D ** -0.5
    _check(_lib().kr_op_attention(_dt(q), _ptr(q), ldq, _ptr(k), ldk, _ptr(v), ldv, _ptr(out), ldo,
                                  S, HQ, HKV, D, float(scale), _stream(stream)))


def attention_workspace(S, HQ, D):
    """(workspace bytes, counters) attention_split needs; (0, 0) when no query
    row is long enough to split."""
    b, c = ctypes.c_size_t(0), ctypes.c_int(0)
    _check(_lib().kr_op_attention_workspace(S, HQ, D, ctypes.byref(b), ctypes.byref(c)))
    return b.value, c.value


def attention_split(q, k, v, out, S, HQ, HKV, D, ws, counters, scale=None, ldq=0, ldk=0, ldv=0, ldo=0,
                    stream=None):
    scale = scale if scale is not None else D ** -0.5
    _check(_lib().kr_op_attention_split(_dt(q), _ptr(q), ldq, _ptr(k), ldk, _ptr(v), ldv, _ptr(out), ldo,
                                        S, HQ, HKV, D, float(scale), _ptr(ws), ws.numel() * ws.element_size(),
                                        _ptr(counters), counters.numel(), _stream(stream)))


def transpose(src, dst, stream=None):
    R, C = src.shape
    assert dst.shape[0] == C and dst.shape[1] == R
    _check(_lib().kr_op_transpose(_ptr(src), _ptr(dst), R, C, _stream(stream)))
