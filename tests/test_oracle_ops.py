"""Pin each oracle op with something other than its own formula: brute-force
loops, an independent formulation, a library routine or an invariant, chosen
so a dropped term, a wrong sign/index or a transposed operand fails."""

import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops as O

torch.manual_seed(0)


def bf(x):
    return x.to(torch.bfloat16).float()


def test_gemm_brute_force():
    a, w = bf(torch.randn(5, 9)), bf(torch.randn(9, 7) * 0.1)
    ref = torch.zeros(5, 7, dtype=torch.float64)
    for i, j, k in itertools.product(range(5), range(7), range(9)):
        ref[i, j] += float(a[i, k]) * float(w[k, j])
    assert torch.equal(O.gemm(a, w), bf(ref.float()))
    b = bf(torch.randn(7))
    assert torch.equal(O.gemm(a, w, b), bf(bf(ref.float()) + b))
    # transposed operand gives a different answer (the layout is pinned)
    assert not torch.equal(O.gemm(a[:, :7], w[:7, :7]), O.gemm(a[:, :7], w[:7, :7].t()))


def test_gelu_tanh_matches_library_and_not_erf():
    x = bf(torch.linspace(-6, 6, 4001))
    assert torch.allclose(O.gelu_tanh(x, torch.float32), F.gelu(x, approximate="tanh"), rtol=1e-6, atol=1e-6)
    # the tanh and erf forms differ at these points by more than one bf16 ulp
    xs = bf(torch.tensor([-2.5, 2.0, 3.0]))
    assert not torch.equal(O.gelu_tanh(xs, torch.float32), F.gelu(xs))


def test_softmax_independent():
    from scipy.special import softmax
    x = bf(torch.randn(17, 333) * 3)
    ref = torch.from_numpy(softmax(x.double().numpy(), axis=-1)).float()
    assert torch.allclose(O.softmax(x, torch.float32), ref, atol=1e-6)
    s = O.softmax(x).double().sum(-1)
    assert torch.all((s - 1).abs() < 333 * 2 ** -8)
    # shift invariance
    assert torch.allclose(O.softmax(x + 7.0, torch.float32), O.softmax(x, torch.float32), atol=1e-6)


def test_silu_swiglu():
    x, u = bf(torch.randn(1000) * 4), bf(torch.randn(1000))
    assert torch.equal(O.silu(x), bf(F.silu(x)))
    # swiglu stores silu before the multiply (two reference ops)
    assert torch.equal(O.swiglu(x, u), bf(bf(F.silu(x)) * u))


def test_cast_exhaustive_bf16_to_f16():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f32 = (bits.astype(np.uint32) << 16).view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = f32.astype(np.float16)
    got = O.cast(torch.from_numpy(f32), torch.float16).numpy()
    nan = np.isnan(ref)
    assert np.array_equal(nan, np.isnan(got))
    assert np.array_equal(ref[~nan].view(np.uint16), got[~nan].view(np.uint16))
    # a few hand-checked round-to-nearest-even cases
    assert O.cast(torch.tensor([65520.0]), torch.float16).isinf().all()
    assert float(O.cast(torch.tensor([65504.0]), torch.float16)) == 65504.0


def test_rmsnorm_matches_hf_qwen2_rmsnorm():
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm
    H = 896
    x = torch.randn(33, H).to(torch.bfloat16)
    g = (1 + 0.02 * torch.randn(H)).to(torch.bfloat16)
    norm = Qwen2RMSNorm(H, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(g)
        hf = norm(x)  # weight * hs.to(bf16); the fp32 weight promotes the product
    y, rstd = O.rmsnorm(x.float(), g.float(), 1e-6)
    assert torch.equal(y, bf(hf.float()))
    assert torch.allclose(rstd, 1 / torch.sqrt(x.float().pow(2).mean(-1) + 1e-6))


def test_add_rmsnorm_rounds_sum_first():
    a, b = bf(torch.randn(4, 64)), bf(torch.randn(4, 64))
    g = bf(torch.ones(64))
    y, s, _ = O.add_rmsnorm(a, b, g, 1e-6)
    assert torch.equal(s, bf(a + b))
    assert torch.equal(y, O.rmsnorm(bf(a + b), g, 1e-6)[0])


def test_rope_as_complex_rotation():
    """Rotate-half RoPE = multiplying (x_i, x_{i+D/2}) as a complex number by
    cos + i sin (independent formulation, fp64)."""
    S, Hh, D = 40, 3, 64
    x = bf(torch.randn(S, Hh, D))
    cos, sin = O.rope_tables(64, D, 1e6)
    c, s = cos[:S].double(), sin[:S].double()
    z = torch.complex(x[..., : D // 2].double(), x[..., D // 2:].double())
    rot = z * torch.complex(c[:, None, : D // 2], s[:, None, : D // 2])
    ref = bf(torch.cat([rot.real, rot.imag], -1).float())
    assert torch.equal(O.rope(x, cos[:S], sin[:S]), ref) or \
        (O.rope(x, cos[:S], sin[:S]) - ref).abs().max() <= 2 ** -7 * ref.abs().max()


def test_rope_tables_closed_form():
    cos, sin = O.rope_tables(100, 128, 1e6)
    i, p = 5, 37
    ang = p * (1e6 ** (-2 * i / 128))
    assert float(cos[p, i]) == float(torch.tensor(math.cos(ang)).to(torch.bfloat16))
    assert float(sin[p, i + 64]) == float(torch.tensor(math.sin(ang)).to(torch.bfloat16))
    assert torch.equal(cos[:, :64], cos[:, 64:])


def test_attention_brute_force_gqa_causal():
    S, HQ, HKV, D = 7, 4, 2, 8
    q, k, v = bf(torch.randn(S, HQ, D)), bf(torch.randn(S, HKV, D)), bf(torch.randn(S, HKV, D))
    ref = torch.zeros(S, HQ, D, dtype=torch.float64)
    for h in range(HQ):
        kv = h // (HQ // HKV)
        for i in range(S):
            sc = [float(q[i, h] @ k[j, kv]) / math.sqrt(D) for j in range(i + 1)]
            m = max(sc)
            e = [math.exp(t - m) for t in sc]
            z = sum(e)
            for j in range(i + 1):
                ref[i, h] += (e[j] / z) * v[j, kv].double()
    assert torch.allclose(O.attention(q, k, v, dt=torch.float32).double(), ref, atol=1e-5)
    # future keys are masked: changing the last key/value leaves earlier rows alone
    k2, v2 = k.clone(), v.clone()
    k2[-1] += 1.0
    v2[-1] -= 1.0
    assert torch.equal(O.attention(q, k2, v2)[:-1], O.attention(q, k, v)[:-1])


def test_attention_rounded_p_brute_force():
    """attention(p_dt=bf16) against a loop that rounds each unnormalised
    weight exp(s_j - max) to bf16 before weighting v_j and divides by the sum
    of the unrounded weights. Planted variants that round the normalised
    softmax instead, or divide by the sum of the rounded weights, or skip the
    rounding, each miss it by far more than the loop's own float error."""
    torch.manual_seed(5)
    S, HQ, HKV, D = 9, 4, 2, 16
    q, k, v = bf(3 * torch.randn(S, HQ, D)), bf(3 * torch.randn(S, HKV, D)), bf(torch.randn(S, HKV, D))

    def loop(variant):
        out = torch.zeros(S, HQ, D, dtype=torch.float64)
        for h in range(HQ):
            kv = h // (HQ // HKV)
            for i in range(S):
                sc = [float(q[i, h].double() @ k[j, kv].double()) / math.sqrt(D) for j in range(i + 1)]
                m = max(sc)
                e = [math.exp(t - m) for t in sc]
                z = sum(e)
                er = [float(torch.tensor(t, dtype=torch.float32).to(torch.bfloat16)) for t in e]
                if variant == "round_normalised":
                    w = [float(torch.tensor(t / z).to(torch.bfloat16)) for t in e]
                    z = 1.0
                elif variant == "sum_rounded":
                    w, z = er, sum(er)
                elif variant == "unrounded":
                    w = e
                else:
                    w = er
                for j in range(i + 1):
                    out[i, h] += w[j] * v[j, kv].double()
                out[i, h] /= z
        return out

    got = O.attention(q, k, v, dt=torch.float32, p_dt=torch.bfloat16).double()
    good = (got - loop("ok")).abs().max().item()
    assert good < 2e-5, good
    for bad in ("round_normalised", "sum_rounded", "unrounded"):
        assert (got - loop(bad)).abs().max().item() > 20 * max(good, 1e-6), bad
    # p_dt=None is the fp32 softmax
    assert torch.equal(O.attention(q, k, v, p_dt=None), O.attention(q, k, v))


def test_embedding():
    t = bf(torch.randn(50, 16))
    ids = torch.tensor([3, 0, 49, 3])
    assert torch.equal(O.embedding(t, ids), t[ids])


def test_layernorm_matches_library_and_rejects_variants():
    x = bf(torch.randn(9, 2048) * 2 + 0.5)
    w, b = bf(torch.randn(2048)), bf(torch.randn(2048))
    ref = F.layer_norm(x, (2048,), w, b, eps=1e-5)
    assert torch.allclose(O.layernorm(x, w, b, 1e-5, torch.float32), ref, atol=2e-5, rtol=1e-5)
    # unbiased variance or a dropped bias are visible
    unbiased = (x - x.mean(-1, keepdim=True)) / torch.sqrt(x.var(-1, unbiased=True, keepdim=True) + 1e-5) * w + b
    assert not torch.allclose(O.layernorm(x, w, b, 1e-5, torch.float32), unbiased, atol=1e-5)
    assert not torch.allclose(O.layernorm(x, w, torch.zeros_like(b), 1e-5, torch.float32), ref, atol=1e-2)
