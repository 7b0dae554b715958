"""CPU oracle for on-device sampling — TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, and only as the checker of the HIP
sampling kernel (``mk_sample`` in libmk.so). The product never calls it.

It restates the sampling the reference configures through NxDI's on-device
sampler: ``--top-k`` / ``--top-p`` / ``--temperature`` / ``--global-topk``
(main.py:57-61, 85, 129-130), per-sequence parameters from
``prepare_sampling_params`` (main.py:195-206), with HF generation semantics
(transformers' TemperatureLogitsWarper, TopKLogitsWarper, TopPLogitsWarper,
applied in that order; NxDI itself is not importable anywhere here):

* greedy when top_k == 1 or temperature <= 0: ``argmax`` (lowest index on ties);
* ``x = logits / temperature``; keep ``x >= `` the top_k-th largest x (ties at
  the threshold kept); top_k <= 0 or > ``MAX_TOPK`` uses the global cap;
* nucleus: over the kept tokens' softmax in descending order, keep a token
  while the mass before it is < top_p (the top token always stays) — the
  same set TopPLogitsWarper keeps (it removes ascending-cumulative mass
  <= 1 - top_p);
* draw: inverse CDF over the kept tokens in descending order of x (ties by
  ascending index) of the renormalised numerators, with
  ``u = Philox4x32-10(key = seed, counter = (counter, row, 0, 0))[0] >> 8``
  times 2**-24.

Philox4x32-10 follows Salmon, Moraes, Dror and Shaw, "Parallel random numbers:
as easy as 1, 2, 3" (SC'11); the tests pin it with the Random123 known-answer
vectors. The filtered distribution is pinned against transformers' warpers.
"""

from __future__ import annotations

from typing import List, Tuple

import numpy as np

MAX_TOPK = 1024
M0, M1, W0, W1 = 0xD2511F53, 0xCD9E8D57, 0x9E3779B9, 0xBB67AE85
MASK = 0xFFFFFFFF


def philox4x32_10(ctr: Tuple[int, int, int, int], key: Tuple[int, int]) -> Tuple[int, int, int, int]:
    """One Philox4x32 block with 10 rounds (pure Python integers)."""
    c0, c1, c2, c3 = ctr
    k0, k1 = key
    for _ in range(10):
        p0 = M0 * c0
        p1 = M1 * c2
        hi0, lo0 = p0 >> 32, p0 & MASK
        hi1, lo1 = p1 >> 32, p1 & MASK
        c0, c1, c2, c3 = (hi1 ^ c1 ^ k0) & MASK, lo1, (hi0 ^ c3 ^ k1) & MASK, lo0
        k0 = (k0 + W0) & MASK
        k1 = (k1 + W1) & MASK
    return c0, c1, c2, c3


def uniform(seed: int, counter: int, row: int) -> float:
    """The kernel's u for one row: the first Philox word's top 24 bits / 2**24."""
    w = philox4x32_10((counter & MASK, row & MASK, 0, 0), (seed & MASK, (seed >> 32) & MASK))[0]
    return (w >> 8) / 16777216.0


def kept_distribution(logits: np.ndarray, top_k: int, top_p: float, temperature: float):
    """Kept token ids in draw order (descending x, ascending index on ties)
    and their renormalised probabilities (float64). Greedy rows return the
    argmax alone with probability 1."""
    x = np.asarray(logits, dtype=np.float32)
    if top_k == 1 or not temperature > 0:
        return np.array([int(np.argmax(x))]), np.array([1.0])
    V = x.size
    k = MAX_TOPK if (top_k <= 0 or top_k > MAX_TOPK) else top_k
    k = min(k, V)
    xs = x / np.float32(temperature)   # fp32 division, as the kernel
    order = np.lexsort((np.arange(V), -xs.astype(np.float64)))   # descending x, ascending index
    thr = xs[order[k - 1]]
    keep = order[xs[order] >= thr]
    z = xs[keep].astype(np.float64)
    e = np.exp(z - z[0])
    if 0.0 < top_p < 1.0:
        before = np.concatenate([[0.0], np.cumsum(e)[:-1]])
        n = int(np.count_nonzero(before < top_p * e.sum()))
        keep, e = keep[:n], e[:n]
    return keep, e / e.sum()


def sample(logits: np.ndarray, top_k: int, top_p: float, temperature: float, seed: int, counter: int,
           row: int) -> Tuple[int, float]:
    """(token, u) the kernel must produce for one row (float64 arithmetic)."""
    keep, prob = kept_distribution(logits, top_k, top_p, temperature)
    if keep.size == 1 and (top_k == 1 or not temperature > 0):
        return int(keep[0]), -1.0
    u = uniform(seed, counter, row)
    c = np.cumsum(prob)
    j = int(np.searchsorted(c, u, side="right"))
    return int(keep[min(j, keep.size - 1)]), u


def cdf_bracket(logits: np.ndarray, top_k: int, top_p: float, temperature: float, token: int) -> Tuple[float, float]:
    """[lo, hi) of u that selects `token` in the oracle's inverse CDF (for
    tolerance checks of fp32 kernels near a boundary); (nan, nan) if the
    token is not kept."""
    keep, prob = kept_distribution(logits, top_k, top_p, temperature)
    hits = np.nonzero(keep == token)[0]
    if hits.size == 0:
        return float("nan"), float("nan")
    j = int(hits[0])
    c = np.concatenate([[0.0], np.cumsum(prob)])
    return float(c[j]), float(c[j + 1])


def prepare_sampling_params(batch_size: int, top_k: List[int], top_p: List[float],
                            temperature: List[float]) -> np.ndarray:
    """[batch][3] (top_k, top_p, temperature) rows; single values broadcast
    (the shape NxDI's prepare_sampling_params builds, main.py:195-206)."""
    def col(v):
        v = list(v)
        return v * batch_size if len(v) == 1 else v
    return np.stack([np.array(col(top_k), dtype=np.float32), np.array(col(top_p), dtype=np.float32),
                     np.array(col(temperature), dtype=np.float32)], axis=1)
