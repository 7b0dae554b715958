"""Logit validation rules of the reference's ``validate`` mode, restated.

The reference validates the megakernel model against the baseline model with
NxDI's ``logit_validation`` (main.py:347-353), fed with

* ``tol_map = {None: (1e-5, 0.05), 1000: (1e-5, 0.03), 50: (1e-5, 0.03), 5: (1e-5, 0.03)}``
  (main.py:544, a string the reference assigns over whatever ``--tol-map``
  held): for each top-k of the expected logits (``None`` = all of them) an
  (atol, rtol) pair;
* ``divergence_difference_tol = 0.001`` (main.py:51): how close the
  expected logits of two tokens must be for a greedy divergence between them
  to count as a tie.

``logit_validation`` itself lives in torch_neuronx, which is not vendored and
not importable here, so its exact pass/fail algorithm is parity-unpinned. This
module restates the checks those numbers parameterise:

* ``topk_tolerance``: at each step, over the indices of the expected logits'
  top-k, every ``|actual - expected| <= atol + rtol * |expected|``;
* ``divergences``: a step whose greedy tokens differ is a tie when the
  expected logits of the two tokens differ by at most the divergence
  tolerance.
"""

from __future__ import annotations

import ast
from typing import Dict, Optional, Tuple

import torch

REFERENCE_TOL_MAP: Dict[Optional[int], Tuple[float, float]] = {
    None: (1e-5, 0.05), 1000: (1e-5, 0.03), 50: (1e-5, 0.03), 5: (1e-5, 0.03)}
REFERENCE_DIVERGENCE_TOL = 0.001
REFERENCE_TOL_MAP_TEXT = "{None: (1e-5, 0.05), 1000: (1e-5, 0.03), 50: (1e-5, 0.03), 5: (1e-5, 0.03)}"


def parse_tol_map(text: Optional[str]) -> Dict[Optional[int], Tuple[float, float]]:
    """``--tol-map`` as the reference writes it (main.py:544): a Python dict
    literal from top-k (an int, or None for all logits) to (atol, rtol).
    ``None`` or an empty string gives the reference's map. The literal is read
    with ``ast.literal_eval`` (no code runs). The reference overwrites the
    parsed flag with its own map, so on its command line ``--tol-map`` has no
    effect; this build uses the map it is given."""
    if text is None or not str(text).strip():
        return dict(REFERENCE_TOL_MAP)
    try:
        m = ast.literal_eval(str(text))
    except (ValueError, SyntaxError) as e:
        raise ValueError(f"not a Python literal: {text!r} ({e})") from None
    if not isinstance(m, dict) or not m:
        raise ValueError(f"expected a non-empty dict {{top_k: (atol, rtol)}}, got {text!r}")
    out: Dict[Optional[int], Tuple[float, float]] = {}
    for k, v in m.items():
        if not (k is None or (isinstance(k, int) and not isinstance(k, bool) and k >= 1)):
            raise ValueError(f"top-k key {k!r} is neither None nor a positive int")
        if not (isinstance(v, (tuple, list)) and len(v) == 2
                and all(isinstance(x, (int, float)) and not isinstance(x, bool) and x >= 0 for x in v)):
            raise ValueError(f"value for {k!r} must be (atol, rtol) with non-negative numbers, got {v!r}")
        out[k] = (float(v[0]), float(v[1]))
    return out


def topk_tolerance(actual: torch.Tensor, expected: torch.Tensor,
                   tol_map: Dict[Optional[int], Tuple[float, float]] = REFERENCE_TOL_MAP) -> Dict[str, dict]:
    """Per top-k entry of ``tol_map``: the fraction of steps (rows of the
    [T, V] logits) that pass, and the worst ratio ``|a - e| / (atol + rtol |e|)``
    (a step passes when its worst ratio is <= 1)."""
    a, e = actual.double(), expected.double()
    if a.shape != e.shape or a.dim() != 2:
        raise ValueError("actual and expected must be [steps, vocab] of the same shape")
    out = {}
    for k, (atol, rtol) in tol_map.items():
        if k is None:
            ae, ee = a, e
        else:
            idx = e.topk(min(k, e.shape[1]), dim=1).indices
            ae, ee = a.gather(1, idx), e.gather(1, idx)
        ratio = ((ae - ee).abs() / (atol + rtol * ee.abs())).max(dim=1).values   # [T]
        out["all" if k is None else f"top{k}"] = {
            "atol": atol, "rtol": rtol, "steps_passing": float((ratio <= 1.0).double().mean()),
            "worst_ratio": float(ratio.max())}
    return out


def divergences(actual: torch.Tensor, expected: torch.Tensor,
                tol: float = REFERENCE_DIVERGENCE_TOL) -> Dict[str, object]:
    """Steps whose greedy tokens differ, and how many of them are ties of the
    expected logits within ``tol``."""
    ta, te = actual.argmax(1), expected.argmax(1)
    steps = (ta != te).nonzero().flatten()
    gaps = (expected[steps, te[steps]] - expected[steps, ta[steps]]).double()
    return {"steps": int(steps.numel()), "within_tol": int((gaps <= tol).sum()),
            "first": int(steps[0]) if steps.numel() else None,
            "largest_expected_gap": float(gaps.max()) if steps.numel() else 0.0}
