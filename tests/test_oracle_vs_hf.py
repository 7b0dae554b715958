"""Pins the oracle's whole decoder against HF transformers' LlamaForCausalLM.

HF's Llama (transformers, not vendored by the reference, used by it as the CPU
fallback at llama.py:50, 170-178) is an independent implementation of the same
model. It is built offline from a local LlamaConfig on a reduced shape (same
head_dim, GQA group of 4 and llama3 RoPE) with random weights, in float64 and
eager attention. The oracle's "exact" mode must reproduce its logits to the
precision HF itself computes at (its RMSNorm and softmax run in fp32), with
unit and with random RMSNorm gammas (which exercises the gamma fold of
llama_with_megakernel.py:312-316 and the final-norm gamma).

Also pinned here: prefill (T tokens at once) equals T incremental decode steps
(same logits, same cache), and the "mk" rounding mode stays close to "exact".
"""

import pytest
import torch

from oracle.llama_ref import OracleLlama


def make_sd(d, seed, random_gamma):
    from mk_weights import param_specs, synthetic_state_dict
    sd = synthetic_state_dict(seed=seed, d=d, workers=2)
    if random_gamma:
        g = torch.Generator().manual_seed(seed + 99)
        for name, shape, kind in param_specs(d):
            if kind == "ones":
                sd[name] = (1.0 + 0.25 * torch.randn(shape, generator=g)).to(torch.bfloat16)
    return sd


def hf_model(d_prod, sd):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(
        vocab_size=d_prod.vocab, hidden_size=d_prod.hidden, intermediate_size=d_prod.intermediate,
        num_hidden_layers=d_prod.n_layers, num_attention_heads=d_prod.n_q_heads,
        num_key_value_heads=d_prod.n_kv_heads, head_dim=d_prod.head_dim, rms_norm_eps=d_prod.rms_eps,
        rope_theta=d_prod.rope_theta, max_position_embeddings=131072, tie_word_embeddings=True,
        rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                      "high_freq_factor": 4.0, "original_max_position_embeddings": 8192},
        attn_implementation="eager")
    m = LlamaForCausalLM(cfg).to(torch.float64).eval()
    sd_hf = {("model." + k): v.to(torch.float64) for k, v in sd.items()}
    sd_hf["lm_head.weight"] = sd["embed_tokens.weight"].to(torch.float64)
    missing, unexpected = m.load_state_dict(sd_hf, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    return m


@pytest.mark.parametrize("random_gamma", [False, True])
def test_exact_mode_matches_hf_llama(small, random_gamma):
    d_prod, d_or = small
    sd = make_sd(d_prod, seed=11, random_gamma=random_gamma)
    toks = torch.randint(0, d_or.vocab, (40,), generator=torch.Generator().manual_seed(2))
    # start positions beyond the llama3 smoothing knee so all RoPE regimes matter
    with torch.no_grad():
        ref = hf_model(d_prod, sd)(toks[None]).logits[0]
    o = OracleLlama(sd, d_or, mode="exact")
    cache = o.new_cache(64)
    logits, _ = o.forward(toks, 0, cache)
    scale = ref.abs().max().item()
    err = (logits - ref).abs().max().item()
    assert err <= 2e-5 * max(1.0, scale), (err, scale)
    # the comparison is sharp: a sign slip in rotate_half is far outside it
    assert torch.equal(logits.argmax(-1), ref.argmax(-1))


def test_hf_comparison_catches_a_planted_mistake(small):
    """A wrong GQA grouping in the oracle (h % n_kv instead of h // g) must fail
    the HF comparison by far more than its tolerance."""
    d_prod, d_or = small
    from oracle.llama_ref import Dims
    d2 = Dims(n_layers=1, hidden=256, n_q=4, n_kv=2, head_dim=64, inter=512, vocab=1000)
    from mk_config import LlamaDims
    p2 = LlamaDims(n_layers=1, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=64, intermediate=512,
                   vocab=1000)
    sd = make_sd(p2, seed=5, random_gamma=False)
    toks = torch.randint(0, 1000, (24,), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        ref = hf_model(p2, sd)(toks[None]).logits[0]

    class Planted(OracleLlama):
        def attention(self, q, K, V, n_valid):
            # wrong mapping: q head h -> kv head h % n_kv (instead of h // group)
            idx = torch.arange(self.d.n_q) % self.d.n_kv
            s = torch.einsum("thd,hsd->hts", q, K[idx]) * self.scale
            mask = torch.arange(K.shape[1])[None, :] >= torch.as_tensor(n_valid)[:, None]
            p = torch.softmax(s.masked_fill(mask[None], float("-inf")), -1)
            return torch.einsum("hts,hsd->htd", p, V[idx]).permute(1, 0, 2)

    good = OracleLlama(sd, d2, mode="exact").forward(toks, 0, OracleLlama(sd, d2, "exact").new_cache(32))[0]
    bad_o = Planted(sd, d2, mode="exact")
    bad = bad_o.forward(toks, 0, bad_o.new_cache(32))[0]
    tol = 2e-5 * max(1.0, ref.abs().max().item())
    assert (good - ref).abs().max().item() <= tol
    assert (bad - ref).abs().max().item() > 100 * tol


def test_prefill_equals_incremental_decode(small):
    d_prod, d_or = small
    sd = make_sd(d_prod, seed=3, random_gamma=True)
    toks = torch.randint(0, d_or.vocab, (20,), generator=torch.Generator().manual_seed(8))
    o = OracleLlama(sd, d_or, mode="mk")
    c1 = o.new_cache(32)
    l1, h1 = o.forward(toks, 0, c1)
    c2 = o.new_cache(32)
    l2 = []
    for t in range(20):
        lt, _ = o.forward(toks[t:t + 1], t, c2)
        l2.append(lt)
    l2 = torch.cat(l2)
    assert (l1 - l2).abs().max().item() < 2e-2
    assert (l1.argmax(-1) == l2.argmax(-1)).float().mean().item() >= 0.95
    for (k1, v1), (k2, v2) in zip(c1, c2):
        # identical up to rare bf16 rounding flips from fp32 summation order
        assert (k1 - k2).abs().max().item() <= 0.05 * k1.abs().max().item()
        assert (k1 != k2).float().mean().item() < 0.02
        assert (v1 != v2).float().mean().item() < 0.02


def test_mk_mode_tracks_exact_mode(small):
    d_prod, d_or = small
    sd = make_sd(d_prod, seed=4, random_gamma=False)
    toks = torch.randint(0, d_or.vocab, (16,), generator=torch.Generator().manual_seed(9))
    a = OracleLlama(sd, d_or, "mk")
    b = OracleLlama(sd, d_or, "exact")
    la, _ = a.forward(toks, 0, a.new_cache(16))
    lb, _ = b.forward(toks, 0, b.new_cache(16))
    assert (la.double() - lb).abs().max().item() < 5e-2
