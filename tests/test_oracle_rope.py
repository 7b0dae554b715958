"""Pins the oracle's RoPE (llama.py:888-953) and the product's RoPE table.

Checks: fp64 closed form of the llama3 frequency smoothing, the independent
HF implementation (``_compute_llama3_parameters``), rotation invariants, and
bit-equality of the product's precomputed bf16 table with the oracle.
"""

import math

import pytest
import torch

from oracle.llama_ref import LLAMA_1B, Dims, OracleLlama, cos_sin, inv_freq, rotate_half


def closed_form_inv_freq_f64(d: Dims):
    """llama3 smoothing evaluated in float64 from its defining formulas."""
    out = []
    for i in range(d.head_dim // 2):
        f = d.rope_theta ** (-2.0 * i / d.head_dim)
        wl = 2 * math.pi / f
        if wl < d.rope_orig / d.rope_high:
            out.append(f)
        elif wl > d.rope_orig / d.rope_low:
            out.append(f / d.rope_factor)
        else:
            s = (d.rope_orig / wl - d.rope_low) / (d.rope_high - d.rope_low)
            out.append((1 - s) * f / d.rope_factor + s * f)
    return torch.tensor(out, dtype=torch.float64)


def test_inv_freq_matches_fp64_closed_form():
    got = inv_freq(LLAMA_1B).double()
    ref = closed_form_inv_freq_f64(LLAMA_1B)
    assert got.shape == (32,)
    rel = ((got - ref).abs() / ref).max().item()
    assert rel < 2e-6, rel
    # all three regimes occur for Llama-3.2-1B: unscaled, divided by 8, smoothed
    raw = torch.tensor([LLAMA_1B.rope_theta ** (-2.0 * i / 64) for i in range(32)], dtype=torch.float64)
    ratio = ref / raw
    assert (ratio == 1).any() and ((ratio - 1 / 8).abs() < 1e-12).any()
    assert ((ratio > 1 / 8 + 1e-9) & (ratio < 1 - 1e-9)).any()


def test_inv_freq_matches_hf_llama3():
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    cfg = LlamaConfig(hidden_size=2048, num_attention_heads=32, num_key_value_heads=8, head_dim=64,
                      rope_theta=500000.0, max_position_embeddings=131072,
                      rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                    "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})
    hf, scale = ROPE_INIT_FUNCTIONS["llama3"](cfg, torch.device("cpu"))
    assert scale == 1.0
    ours = inv_freq(LLAMA_1B)
    assert hf.dtype == torch.float32
    # independent implementation of the same fp32 formula: equal to the last ulp
    ulps = (ours.view(torch.int32) - hf.view(torch.int32)).abs().max().item()
    assert ulps <= 1, ulps


def test_product_inv_freq_and_table_match_oracle():
    from mk_weights import llama3_inv_freq, rope_table
    assert torch.equal(llama3_inv_freq().view(torch.int32), inv_freq(LLAMA_1B).view(torch.int32))
    tab = rope_table(1024)
    c, s = cos_sin(LLAMA_1B, torch.arange(1024))
    assert tab.dtype == torch.bfloat16 and tab.shape == (1024, 128)
    assert torch.equal(tab[:, :64], c.to(torch.bfloat16))
    assert torch.equal(tab[:, 64:], s.to(torch.bfloat16))


def test_position_zero_is_identity():
    c, s = cos_sin(LLAMA_1B, torch.tensor([0]))
    assert torch.all(c == 1) and torch.all(s == 0)
    x = torch.randn(3, 64, dtype=torch.float64)
    sd = {}
    o = OracleLlama.__new__(OracleLlama)
    o.mode, o.dt = "exact", torch.float64
    y = o.rope(x, c.double(), s.double())
    assert torch.equal(y, x)


def test_rotation_preserves_pair_norms_and_relative_position():
    o = OracleLlama.__new__(OracleLlama)
    o.mode, o.dt = "exact", torch.float64
    g = torch.Generator().manual_seed(1)
    q = torch.randn(64, dtype=torch.float64, generator=g)
    k = torch.randn(64, dtype=torch.float64, generator=g)

    def rot(x, p):
        c, s = cos_sin(LLAMA_1B, torch.tensor([p]))
        return o.rope(x[None], c.double(), s.double())[0]

    for p in (1, 17, 1023, 8191):
        y = rot(q, p)
        n_in = q[:32] ** 2 + q[32:] ** 2
        n_out = y[:32] ** 2 + y[32:] ** 2
        assert torch.allclose(n_in, n_out, rtol=5e-7, atol=1e-12)   # cos, sin are fp32 values
    # q.k after rotation depends only on the position difference
    a = rot(q, 100) @ rot(k, 90)
    b = rot(q, 1010) @ rot(k, 1000)
    assert abs(a - b) < 5e-4 * (q.norm() * k.norm())   # fp32 angles -> small drift
    # rotate_half convention: cat(-x[half:], x[:half])
    x = torch.arange(64, dtype=torch.float64)
    assert torch.equal(rotate_half(x), torch.cat([-x[32:], x[:32]]))
