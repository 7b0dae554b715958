"""GPU parity of the on-device sampler (mk_sample in libmk.so) with the CPU
oracle (oracle/sampling_ref.py, pinned against transformers' warpers and the
Philox4x32-10 known-answer vectors in tests/test_oracle_sampling.py).

* 32 rows of full-vocabulary logits (128256, N(0, s^2) with s from 0.5 to 4)
  with per-row (top_k, top_p, temperature) covering greedy, small and large
  top_k, the global cap (top_k 0 and > 1024) and nucleus cuts: every row's u
  equals the oracle's bit for bit (integer Philox), every drawn token lies in
  the oracle's inverse-CDF bracket of u widened by 1e-5 (fp32 softmax sums
  against the oracle's float64), and at least 31 of 32 tokens equal the
  oracle's exactly (a boundary case is the only allowed difference);
* greedy ties resolve to the lowest index; ties at the top-k threshold are
  all kept;
* 4096 draws from one distribution (top_k 12, top_p 0.9, temperature 0.8)
  pass a chi-square test against the oracle's kept probabilities;
* generate() with sampling: reproducible for a seed, and every sampled token
  is the oracle's draw from the GPU's own logits of that step.
"""

import numpy as np
import pytest
import torch

from gpu_common import need_gpu, say

pytestmark = pytest.mark.gpu

V = 128256
ROW_PARAMS = [
    (1, 1.0, 1.0), (5, 1.0, 1.0), (50, 1.0, 1.0), (50, 0.9, 0.7), (0, 1.0, 1.0), (0, 0.95, 1.0),
    (1024, 0.5, 1.3), (2000, 1.0, 0.5), (3, 1.0, 2.0), (50, 0.3, 1.0), (10, 0.99, 0.2), (1, 0.9, 0.7),
    (50, 1.0, 0.0), (100, 0.8, 1.0), (7, 0.6, 3.0), (0, 0.5, 0.8),
]


def run(logits, params, seed, counter):
    import mk_lib
    B = logits.shape[0]
    tok = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    u = torch.full((B,), -9.0, dtype=torch.float32, device="cuda")
    mk_lib.sample(logits, params, tok, seed=seed, counter=counter, uniforms_out=u)
    torch.cuda.synchronize()
    return tok.cpu().numpy(), u.cpu().numpy()


def test_sample_matches_oracle_full_vocab():
    need_gpu()
    from oracle.sampling_ref import cdf_bracket, sample
    rows = ROW_PARAMS * 2
    B = len(rows)
    g = torch.Generator().manual_seed(11)
    scale = torch.linspace(0.5, 4.0, B)[:, None]
    logits = (torch.randn(B, V, generator=g) * scale).float()
    params = torch.tensor(rows, dtype=torch.float32)
    counter = torch.arange(100, 100 + B, dtype=torch.int32)
    seed = 0x1234ABCD5678
    tok, u = run(logits.cuda(), params.cuda(), seed, counter.cuda())
    exact = 0
    for b in range(B):
        k, p, t = rows[b]
        x = logits[b].numpy()
        ref_tok, ref_u = sample(x, int(k), float(p), float(t), seed, int(counter[b]), b)
        assert u[b] == np.float32(ref_u), (b, u[b], ref_u)
        lo, hi = cdf_bracket(x, int(k), float(p), float(t), int(tok[b]))
        assert lo - 1e-5 <= (ref_u if ref_u >= 0 else 0.0) < hi + 1e-5, (b, rows[b], int(tok[b]), ref_tok, lo, hi)
        exact += int(tok[b]) == ref_tok
    say(f"[sample] {exact}/{B} tokens equal the oracle's")
    assert exact >= B - 1


def test_sample_ties():
    need_gpu()
    x = torch.full((2, V), -5.0)
    x[0, [900, 17, 5000]] = 4.0          # greedy: three-way tie at the max
    x[1, [10, 20]] = 6.0                 # top_k = 3: ties at the 3rd value all kept
    x[1, [30, 40, 50]] = 5.0
    params = torch.tensor([[1, 1.0, 1.0], [3, 1.0, 1.0]], dtype=torch.float32).cuda()
    seen = set()
    for c in range(200):
        tok, _ = run(x.cuda(), params, 3, torch.tensor([c, c], dtype=torch.int32).cuda())
        assert tok[0] == 17
        seen.add(int(tok[1]))
    assert seen == {10, 20, 30, 40, 50}, seen


def test_sample_distribution_chi_square():
    need_gpu()
    from oracle.sampling_ref import kept_distribution
    g = torch.Generator().manual_seed(5)
    row = (torch.randn(V, generator=g) * 3).float()
    B = 32
    logits = row[None].repeat(B, 1).cuda()
    params = torch.tensor([[12, 0.9, 0.8]] * B, dtype=torch.float32).cuda()
    keep, prob = kept_distribution(row.numpy(), 12, 0.9, 0.8)
    counts = {}
    for it in range(128):
        tok, _ = run(logits, params, 99, torch.arange(it * B, (it + 1) * B, dtype=torch.int32).cuda())
        for t_ in tok.tolist():
            counts[t_] = counts.get(t_, 0) + 1
    n = 128 * B
    assert set(counts) <= set(keep.tolist())
    obs = np.array([counts.get(int(t_), 0) for t_ in keep], dtype=np.float64)
    exp = prob * n
    chi2 = float(((obs - exp) ** 2 / exp).sum())
    dof = keep.size - 1
    say(f"[sample] chi-square {chi2:.1f} over {dof} degrees of freedom ({n} draws, {keep.size} kept tokens)")
    assert chi2 < dof + 6 * np.sqrt(2 * dof)


def test_generate_with_sampling():
    need_gpu()
    import mk_lib
    from llama_with_megakernel import LlamaInferenceConfig, NeuronConfigLlamaMK, NeuronLlamaForCausalLM
    from mk_weights import random_token_ids
    from oracle.sampling_ref import sample
    cfg = LlamaInferenceConfig(NeuronConfigLlamaMK(seq_len=256, max_context_length=256))
    m = NeuronLlamaForCausalLM("random:0", cfg)
    m.compile()
    m.load()
    ids = random_token_ids(40, seed=2)
    sp = mk_lib.prepare_sampling_params(1, 40, 0.9, 0.8)
    out1, lg = m.generate(ids, 24, return_logits=True, sampling_params=sp, seed=7)
    out2 = m.generate(ids, 24, sampling_params=sp, seed=7)
    assert torch.equal(out1, out2)
    for t in range(24):
        pos = 40 + t          # the step that produced token t left pos at 40 + t
        ref, _ = sample(lg[t].numpy(), 40, 0.9, 0.8, 7, pos, 0)
        assert int(out1[t]) == ref, (t, int(out1[t]), ref)
    greedy = m.generate(ids, 8)
    say(f"[sample] generate: sampled {out1[:8].tolist()} greedy {greedy.tolist()}")
