"""Pins the oracle's RMSNorm, attention and SwiGLU MLP pieces.

Each check compares against something the mathematics fixes independently of
the oracle's code: closed forms, brute force in float64 with Python loops on
tiny shapes, and special cases (pos = 0, identical keys, a dominant score,
GQA as MHA with repeated heads). The bf16 rounding points of the "mk" mode are
checked on a hand-computed case (attention.py:354-392: exp cast to bf16 before
PV, fp32 denominator).
"""

import math

import pytest
import torch

from oracle.llama_ref import Dims, OracleLlama


def bare(mode="exact", d=None):
    o = OracleLlama.__new__(OracleLlama)
    o.mode = mode
    o.dt = torch.float64 if mode == "exact" else torch.float32
    o.d = d or Dims(hidden=8, n_q=4, n_kv=1, head_dim=4)
    o.scale = 1.0 / math.sqrt(o.d.head_dim)
    return o


def test_rmsnorm_closed_forms():
    o = bare(d=Dims(hidden=2048))
    for c in (0.5, -3.0, 1e-3):
        x = torch.full((2048,), c, dtype=torch.float64)
        y = o.norm_scale(x)
        expect = math.copysign(1.0, c) / math.sqrt(1 + 1e-5 / (c * c))
        assert torch.allclose(y, torch.full_like(y, expect), rtol=1e-12)
    z = o.norm_scale(torch.zeros(2048, dtype=torch.float64))
    assert torch.all(z == 0)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2048, dtype=torch.float64, generator=g)
    ms = sum(float(v) ** 2 for v in x) / 2048
    ref = x / math.sqrt(ms + 1e-5)
    assert torch.allclose(o.norm_scale(x), ref, rtol=1e-12, atol=1e-14)


def brute_attention(q, K, V, n_valid, scale):
    """float64 loops: q [T, n_q, D], K/V [n_kv, S, D]; head h reads kv h // (n_q/n_kv)."""
    T, n_q, D = q.shape
    n_kv = K.shape[0]
    g = n_q // n_kv
    out = torch.zeros(T, n_q, D, dtype=torch.float64)
    for t in range(T):
        for h in range(n_q):
            kv = h // g
            s = [scale * sum(float(q[t, h, e]) * float(K[kv, j, e]) for e in range(D))
                 for j in range(n_valid[t])]
            m = max(s)
            p = [math.exp(x - m) for x in s]
            den = sum(p)
            for e in range(D):
                out[t, h, e] = sum(p[j] * float(V[kv, j, e]) for j in range(n_valid[t])) / den
    return out


def test_attention_matches_bruteforce():
    d = Dims(hidden=16, n_q=4, n_kv=2, head_dim=4)
    o = bare(d=d)
    g = torch.Generator().manual_seed(3)
    q = torch.randn(3, 4, 4, dtype=torch.float64, generator=g)
    K = torch.randn(2, 7, 4, dtype=torch.float64, generator=g)
    V = torch.randn(2, 7, 4, dtype=torch.float64, generator=g)
    n_valid = [3, 5, 7]
    got = o.attention(q, K, V, torch.tensor(n_valid))
    ref = brute_attention(q, K, V, n_valid, 0.5)
    assert torch.allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_attention_special_cases():
    d = Dims(hidden=16, n_q=4, n_kv=1, head_dim=4)
    o = bare(d=d)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 4, 4, dtype=torch.float64, generator=g)
    K = torch.randn(1, 6, 4, dtype=torch.float64, generator=g)
    V = torch.randn(1, 6, 4, dtype=torch.float64, generator=g)
    # pos = 0: only the fresh row -> output is that V row exactly
    out = o.attention(q, K, V, torch.tensor([1]))
    assert torch.equal(out[0], V[0, 0].expand(4, 4))
    # identical keys -> uniform average of V
    K2 = K[:, :1].expand(1, 6, 4).clone()
    out = o.attention(q, K2, V, torch.tensor([6]))
    assert torch.allclose(out[0], V[0].mean(0).expand(4, 4), rtol=1e-12)
    # one dominant score -> one-hot
    K3 = K.clone()
    K3[0, 4] = q[0, 0] * 1e4
    out = o.attention(q[:, :1].expand(1, 4, 4), K3, V, torch.tensor([6]))
    assert torch.allclose(out[0, 0], V[0, 4], atol=1e-9)
    # masked rows never contribute, even if they hold inf / nan
    K4, V4 = K.clone(), V.clone()
    K4[0, 3:] = float("inf")
    V4[0, 3:] = float("nan")
    a = o.attention(q, K4, V4, torch.tensor([3]))
    b = o.attention(q, K[:, :3], V[:, :3], torch.tensor([3]))
    assert torch.equal(a, b)


def test_gqa_equals_mha_with_repeated_heads():
    d_gqa = Dims(hidden=16, n_q=4, n_kv=2, head_dim=4)
    d_mha = Dims(hidden=16, n_q=4, n_kv=4, head_dim=4)
    g = torch.Generator().manual_seed(7)
    q = torch.randn(2, 4, 4, dtype=torch.float64, generator=g)
    K = torch.randn(2, 5, 4, dtype=torch.float64, generator=g)
    V = torch.randn(2, 5, 4, dtype=torch.float64, generator=g)
    a = bare(d=d_gqa).attention(q, K, V, torch.tensor([4, 5]))
    b = bare(d=d_mha).attention(q, K.repeat_interleave(2, 0), V.repeat_interleave(2, 0),
                                 torch.tensor([4, 5]))
    assert torch.equal(a, b)
    # and the grouping is h -> h // 2 (not h % 2): swapping kv heads changes head 0
    c = bare(d=d_gqa).attention(q, K.flip(0), V.flip(0), torch.tensor([4, 5]))
    assert not torch.allclose(a[:, 0], c[:, 0])


def test_mk_attention_rounding_points():
    """exp cast to bf16 in the numerator only; denominator from fp32 exp."""
    d = Dims(hidden=4, n_q=1, n_kv=1, head_dim=4)
    o = bare("mk", d)
    q = torch.tensor([[[1.0, 0.5, -0.25, 0.125]]])
    K = torch.tensor([[[0.3, -0.7, 0.2, 0.9], [1.1, 0.4, -0.6, 0.05], [-0.2, 0.8, 0.33, -0.41]]])
    V = torch.tensor([[[1.0, 2.0, 3.0, 4.0], [-1.5, 0.25, 2.5, -3.0], [0.7, -0.9, 1.3, 0.1]]])
    s = [0.5 * sum(q[0, 0, e].item() * K[0, j, e].item() for e in range(4)) for j in range(3)]
    s32 = torch.tensor(s, dtype=torch.float32)
    p = torch.exp(s32 - s32.max())
    pb = p.to(torch.bfloat16).float()
    num = (pb[:, None] * V[0]).sum(0)
    expect = (num * (1.0 / p.sum())).to(torch.bfloat16).float()
    got = o.attention(q, K, V, torch.tensor([3]))[0, 0]
    assert torch.allclose(got, expect, atol=0, rtol=0) or (got - expect).abs().max() <= 2 ** -8 * expect.abs().max()
    # the bf16 rounding of p is visible: differs from the unrounded result
    exact = ((p[:, None] * V[0]).sum(0) / p.sum())
    assert not torch.equal(num, (p[:, None] * V[0]).sum(0))
    assert (got - exact).abs().max() < 1e-2


def test_unrounded_p_variant():
    """round_p = False (the noise-floor variant of a split-K kernel): the
    numerator uses fp32 p, i.e. the hand-computed case without bf16(p)."""
    d = Dims(hidden=4, n_q=1, n_kv=1, head_dim=4)
    o = bare("mk", d)
    o.round_p = False
    q = torch.tensor([[[1.0, 0.5, -0.25, 0.125]]])
    K = torch.tensor([[[0.3, -0.7, 0.2, 0.9], [1.1, 0.4, -0.6, 0.05], [-0.2, 0.8, 0.33, -0.41]]])
    V = torch.tensor([[[1.0, 2.0, 3.0, 4.0], [-1.5, 0.25, 2.5, -3.0], [0.7, -0.9, 1.3, 0.1]]])
    V = V.to(torch.bfloat16).float()          # cache rows are bf16
    s = [0.5 * sum(q[0, 0, e].item() * K[0, j, e].item() for e in range(4)) for j in range(3)]
    e = [math.exp(x - max(s)) for x in s]
    expect = [sum(e[j] * V[0, j, c].item() for j in range(3)) / sum(e) for c in range(4)]
    got = o.attention(q, K, V, torch.tensor([3]))[0, 0]
    want = torch.tensor(expect, dtype=torch.float32).to(torch.bfloat16).float()
    assert torch.all((got - want).abs() <= 2 ** -8 * want.abs())
    o.round_p = True
    assert not torch.equal(o.attention(q, K, V, torch.tensor([3]))[0, 0], got)


def test_oracle_mlp_is_swiglu_of_gate_and_up():
    """The oracle's decoder layer, MLP half (mlp.py:98-192): with the attention's
    output projection zero, layer(h) = h + W_d (silu(W_g n) * (W_u n)), n the
    RMS-normalised h times the post-attention gamma. Checked in float64 against
    Python loops with silu(x) = x / (1 + e^-x) written out, on random weights
    where gate and up differ, so a swapped pair, silu on the wrong projection or
    a transposed down projection fails."""
    d = Dims(n_layers=1, hidden=8, n_q=2, n_kv=1, head_dim=4, inter=6, vocab=16)
    g = torch.Generator().manual_seed(3)
    r = lambda *shape: torch.randn(*shape, dtype=torch.float64, generator=g)
    p = "layers.0."
    sd = {
        p + "input_layernorm.weight": 1.0 + 0.1 * r(8), p + "post_attention_layernorm.weight": 1.0 + 0.1 * r(8),
        p + "self_attn.q_proj.weight": r(8, 8), p + "self_attn.k_proj.weight": r(4, 8),
        p + "self_attn.v_proj.weight": r(4, 8), p + "self_attn.o_proj.weight": torch.zeros(8, 8, dtype=torch.float64),
        p + "mlp.gate_proj.weight": r(6, 8), p + "mlp.up_proj.weight": r(6, 8), p + "mlp.down_proj.weight": r(8, 6),
        "embed_tokens.weight": r(16, 8), "norm.weight": torch.ones(8, dtype=torch.float64),
    }
    o = OracleLlama(sd, d=d, mode="exact")
    h = r(1, 8)
    K, V = torch.zeros(1, 4, 4, dtype=torch.float64), torch.zeros(1, 4, 4, dtype=torch.float64)
    got = o.layer(0, h, torch.tensor([0]), (K, V))[0]
    x = [float(v) for v in h[0]]
    ms = sum(v * v for v in x) / 8
    gp = [float(v) for v in sd[p + "post_attention_layernorm.weight"]]
    n = [x[i] / math.sqrt(ms + 1e-5) * gp[i] for i in range(8)]
    Wg, Wu, Wd = (sd[p + f"mlp.{k}_proj.weight"].tolist() for k in ("gate", "up", "down"))
    gate = [sum(Wg[j][i] * n[i] for i in range(8)) for j in range(6)]
    up = [sum(Wu[j][i] * n[i] for i in range(8)) for j in range(6)]
    act = [gate[j] / (1.0 + math.exp(-gate[j])) * up[j] for j in range(6)]
    expect = torch.tensor([x[i] + sum(Wd[i][j] * act[j] for j in range(6)) for i in range(8)], dtype=torch.float64)
    assert torch.allclose(got, expect, rtol=1e-12, atol=1e-12)
    # the plausible miswirings give something else
    swapped = [up[j] / (1.0 + math.exp(-up[j])) * gate[j] for j in range(6)]
    bad = torch.tensor([x[i] + sum(Wd[i][j] * swapped[j] for j in range(6)) for i in range(8)], dtype=torch.float64)
    assert (got - bad).abs().max() > 1e-3
