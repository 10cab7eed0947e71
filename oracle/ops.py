"""fp32 torch-CPU restatement of the relay-path ops — test infrastructure only.

Convention: every tensor the reference keeps in HBM is a 16-bit type, so each
op computes in fp32 from 16-bit-exact inputs and rounds its stored outputs to
the storage type (bf16 or fp16). `dt` below is that storage dtype.

Reference semantics followed (the op math itself lives in closed CANN aclnn
libraries, so the restatement follows the call sites and HF's definitions):
  gemm        aclnnMatmul C = A.B, B = weight_t [K,N] (exec/qwen_main.cpp:499-512,
              scripts/export_model.py:159-161); QKV bias is a separate Add on
              the rounded product (EmitQkv :1336-1344)
  gelu_tanh   aclnnGelu (exec/runtime/op_impl.cpp:214-228); tanh form as
              the task pins it
  softmax     aclnnSoftmax dim=1 (op_impl.cpp:229-233)
  cast        aclnnCast (op_impl.cpp:219-223)
  silu, mul   aclnnSilu then aclnnMul with the silu result stored in between
              (qwen_main.cpp:616-644, used at :888-889)
  rmsnorm     aclnnRmsNorm (:531-546), HF Qwen2RMSNorm: fp32 variance,
              x*rsqrt(var+eps) rounded, then times gamma
  add_rmsnorm aclnnAddRmsNorm (:548-565): sum rounded, then rmsnorm of it
  layernorm   aclnnLayerNorm (exec/runtime/op_impl.cpp:237-254): biased
              variance, eps 1e-5, weight and bias, one rounding
  rope        aclnnApplyRotaryPosEmb layout 1 (:567-582), rotate-half with
              tables from export_model.py:70-77; fp32, one rounding
  attention   aclnnFlashAttentionScore (:591-614): causal (MakeMask :487-497),
              scale 1/sqrt(D), GQA head h -> h // (HQ/HKV)
  embedding   aclnnEmbedding (:646-659)

Pins (tests/test_oracle_ops.py): brute-force loops at small shapes (gemm,
attention), independent formulations (rope as complex rotation, softmax via
scipy), library routines (torch gelu/silu, transformers Qwen2RMSNorm),
exhaustive enumeration (cast over all 65536 bf16 patterns), invariants
(softmax rows sum to 1, split == unsplit).
"""

import math

import torch

F32 = torch.float32


def rnd(x, dt=torch.bfloat16):
    """Round an fp32 tensor to the storage type and back (what a reader sees)."""
    return x.to(dt).to(F32)


def gemm(a, w_t, bias=None, dt=torch.bfloat16):
    """C = a @ w_t (fp32 accumulate), stored in dt; bias added to the stored product."""
    c = rnd(torch.matmul(a.to(F32), w_t.to(F32)), dt)
    if bias is not None:
        c = rnd(c + bias.to(F32), dt)
    return c


def gelu_tanh(x, dt=torch.bfloat16):
    k0 = math.sqrt(2.0 / math.pi)
    x = x.to(F32)
    return rnd(0.5 * x * (1.0 + torch.tanh(k0 * (x + 0.044715 * x * x * x))), dt)


def softmax(x, dt=torch.bfloat16):
    x = x.to(F32)
    m = x.max(dim=-1, keepdim=True).values
    e = torch.exp(x - m)
    return rnd(e / e.sum(dim=-1, keepdim=True), dt)


def cast(x, dt_out):
    return x.to(F32).to(dt_out)


def silu(x, dt=torch.bfloat16):
    x = x.to(F32)
    return rnd(x / (1.0 + torch.exp(-x)), dt)


def mul(a, b, dt=torch.bfloat16):
    return rnd(a.to(F32) * b.to(F32), dt)


def add(a, b, dt=torch.bfloat16):
    return rnd(a.to(F32) + b.to(F32), dt)


def swiglu(gate, up, dt=torch.bfloat16):
    """silu(gate) stored, then multiplied by up and stored (two reference ops)."""
    return mul(silu(gate, dt), up, dt)


def rmsnorm(x, gamma, eps, dt=torch.bfloat16):
    """Returns (y, rstd): y = gamma * rnd(x * rstd), rstd = 1/sqrt(mean(x^2)+eps)."""
    x = x.to(F32)
    rstd = torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps)
    return rnd(gamma.to(F32) * rnd(x * rstd, dt), dt), rstd.squeeze(-1)


def add_rmsnorm(a, b, gamma, eps, dt=torch.bfloat16):
    """Returns (y, sum, rstd) with sum = rnd(a + b) and y = rmsnorm(sum)."""
    s = add(a, b, dt)
    y, rstd = rmsnorm(s, gamma, eps, dt)
    return y, s, rstd


def layernorm(x, weight, bias, eps=1e-5, dt=torch.bfloat16):
    """aclnnLayerNorm over the last dim (exec/runtime/op_impl.cpp:237-254,
    eps 1e-5 there): (x - mean) / sqrt(var + eps) * weight + bias, biased
    variance, fp32, one rounding to the storage type."""
    x = x.to(F32)
    mean = x.mean(dim=-1, keepdim=True)
    var = (x - mean).pow(2).mean(dim=-1, keepdim=True)
    return rnd((x - mean) * torch.rsqrt(var + eps) * weight.to(F32) + bias.to(F32), dt)


def rope_tables(max_pos, D, theta):
    """cos/sin [max_pos, D] in bf16, as scripts/export_model.py:70-77 builds them."""
    inv = 1.0 / (torch.tensor(theta, dtype=torch.float64) ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    pos = torch.arange(max_pos, dtype=torch.float64)
    freqs = torch.outer(pos, inv)
    cos = torch.cat([freqs.cos(), freqs.cos()], dim=-1).to(torch.bfloat16)
    sin = torch.cat([freqs.sin(), freqs.sin()], dim=-1).to(torch.bfloat16)
    return cos, sin


def rope(x, cos, sin, dt=torch.bfloat16):
    """x [S, heads, D]; cos/sin [S, D]: x*cos + rotate_half(x)*sin, one rounding."""
    x = x.to(F32)
    D = x.shape[-1]
    x1, x2 = x[..., : D // 2], x[..., D // 2:]
    c = cos.to(F32)[:, None, :]
    s = sin.to(F32)[:, None, :]
    o1 = x1 * c[..., : D // 2] - x2 * s[..., : D // 2]
    o2 = x2 * c[..., D // 2:] + x1 * s[..., D // 2:]
    return rnd(torch.cat([o1, o2], dim=-1), dt)


def attention(q, k, v, scale=None, dt=torch.bfloat16, p_dt=None):
    """Causal GQA attention. q [S, HQ, D], k/v [S, HKV, D] -> [S, HQ, D] (fp32 softmax).

    p_dt (e.g. torch.bfloat16): the products P.V take P rounded to p_dt, as
    a 16-bit matrix unit does: P = exp(s - rowmax) in fp32, rounded to p_dt
    before the P.V product (fp32 accumulation), then divided by the fp32 sum
    of the unrounded P. None: P stays fp32 (the reference's softmax)."""
    S, HQ, D = q.shape
    HKV = k.shape[1]
    scale = scale if scale is not None else 1.0 / math.sqrt(D)
    rep = HQ // HKV
    qh = q.to(F32).permute(1, 0, 2)                                   # [HQ, S, D]
    kh = k.to(F32).permute(1, 0, 2).repeat_interleave(rep, dim=0)     # [HQ, S, D]
    vh = v.to(F32).permute(1, 0, 2).repeat_interleave(rep, dim=0)
    scores = torch.matmul(qh, kh.transpose(1, 2).contiguous()) * scale
    mask = torch.ones(S, S, dtype=torch.bool).triu(1)
    scores = scores.masked_fill(mask, float("-inf"))
    if p_dt is None:
        p = torch.softmax(scores, dim=-1)
        return rnd(torch.matmul(p, vh).permute(1, 0, 2), dt)
    e = torch.exp(scores - scores.amax(dim=-1, keepdim=True))
    num = torch.matmul(rnd(e, p_dt), vh)
    return rnd((num / e.sum(dim=-1, keepdim=True)).permute(1, 0, 2), dt)


def embedding(table, ids):
    return table[ids.long()].to(F32)
