"""Pins of the sampling oracle (oracle/sampling_ref.py) on the CPU.

* Philox4x32-10 against the Random123 known-answer vectors (counter, key ->
  output) for the all-zero, all-ones and pi-digits inputs;
* the kept set and renormalised probabilities against transformers'
  TemperatureLogitsWarper -> TopKLogitsWarper -> TopPLogitsWarper followed by a
  softmax (HF generation semantics, which NxDI's sampler follows), for several
  (top_k, top_p, temperature); top_k <= 0 is the global cap of 1024 candidates;
* greedy rows (top_k == 1 or temperature <= 0) are the argmax, lowest index on
  ties;
* draws follow the kept distribution (chi-square over 20000 counters);
* the inverse-CDF bracket of the drawn token contains its u.
A planted mistake — top-p keeping the token that crosses the mass instead of
stopping before the next, or a key word swapped in Philox — fails these.
"""

import numpy as np
import pytest
import torch

from oracle.sampling_ref import (cdf_bracket, kept_distribution, philox4x32_10, prepare_sampling_params, sample,
                                 uniform)

KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,out", KAT)
def test_philox_known_answers(ctr, key, out):
    assert philox4x32_10(ctr, key) == out


def test_uniform_is_top_24_bits():
    w = philox4x32_10((5, 3, 0, 0), (0x1234, 0x5678))[0]
    assert uniform(0x0000567800001234, 5, 3) == (w >> 8) / 2 ** 24


def hf_probs(logits: np.ndarray, top_k: int, top_p: float, temperature: float) -> np.ndarray:
    from transformers.generation.logits_process import (TemperatureLogitsWarper, TopKLogitsWarper,
                                                        TopPLogitsWarper)
    s = torch.from_numpy(logits.astype(np.float32))[None]
    s = TemperatureLogitsWarper(temperature)(None, s)
    s = TopKLogitsWarper(top_k=1024 if top_k <= 0 else top_k)(None, s)
    if 0 < top_p < 1:
        s = TopPLogitsWarper(top_p=top_p)(None, s)
    return torch.softmax(s.double(), -1)[0].numpy()


@pytest.mark.parametrize("top_k,top_p,temperature", [
    (50, 1.0, 1.0), (50, 0.9, 0.7), (0, 0.95, 1.0), (0, 1.0, 1.3), (5, 0.5, 2.0), (1024, 0.3, 0.5),
])
def test_kept_distribution_matches_transformers(top_k, top_p, temperature):
    rng = np.random.default_rng(top_k + int(100 * top_p))
    logits = (rng.standard_normal(5000) * 2).astype(np.float32)
    keep, prob = kept_distribution(logits, top_k, top_p, temperature)
    ref = hf_probs(logits, top_k, top_p, temperature)
    nz = np.nonzero(ref > 0)[0]
    assert sorted(keep.tolist()) == nz.tolist()
    np.testing.assert_allclose(prob, ref[keep], rtol=1e-6, atol=1e-12)
    # draw order: descending logit
    assert np.all(np.diff(logits[keep]) <= 0)


def test_greedy_rows_take_lowest_index_of_the_max():
    x = np.zeros(100, dtype=np.float32)
    x[[7, 40]] = 3.0
    assert sample(x, 1, 1.0, 1.0, 0, 0, 0) == (7, -1.0)
    assert sample(x, 50, 0.9, 0.0, 0, 0, 0) == (7, -1.0)


def test_draws_follow_the_kept_distribution():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(300) * 1.5).astype(np.float32)
    keep, prob = kept_distribution(x, 20, 0.9, 0.8)
    n = 20000
    counts = {}
    for c in range(n):
        tok, u = sample(x, 20, 0.9, 0.8, 1234, c, 0)
        counts[tok] = counts.get(tok, 0) + 1
    assert set(counts) <= set(keep.tolist())
    obs = np.array([counts.get(int(t), 0) for t in keep], dtype=np.float64)
    exp = prob * n
    chi2 = float(((obs - exp) ** 2 / exp).sum())
    dof = keep.size - 1
    assert chi2 < dof + 6 * np.sqrt(2 * dof), (chi2, dof)


def test_cdf_bracket_contains_u():
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(1000)).astype(np.float32)
    for c in range(50):
        tok, u = sample(x, 100, 0.8, 1.0, 77, c, 3)
        lo, hi = cdf_bracket(x, 100, 0.8, 1.0, tok)
        assert lo <= u < hi


def test_prepare_sampling_params_broadcasts():
    p = prepare_sampling_params(3, [50], [0.9], [0.7])
    assert p.shape == (3, 3) and p.dtype == np.float32
    assert np.allclose(p[:, 0], 50) and np.allclose(p[:, 1], 0.9) and np.allclose(p[:, 2], 0.7)
    p = prepare_sampling_params(2, [1, 5], [1.0, 0.5], [1.0, 2.0])
    assert p[1].tolist() == [5.0, 0.5, 2.0]
