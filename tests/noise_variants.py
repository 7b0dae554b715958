"""Variants of the CPU oracle used to measure the floating-point noise floor
that the GPU parity bounds are set against (test infrastructure).

* ``FP64Accumulate``: the oracle's "mk" rounding points (bf16 at the
  reference kernel's points) with fp64 accumulation instead of fp32;
* ``FP64AccumulateFP32P``: the same, with the softmax numerator's p kept
  unrounded, as a split-K decode kernel keeps it (the reference casts p to
  bf16 against the global maximum, attention.py:376-387, which per-split
  maxima cannot reproduce).

Both are correct restatements of the reference's algorithm up to rounding,
so how far the oracle moves against them, from one state, is the spread any
correct bf16 implementation of that algorithm shows.
"""

import torch

from oracle.llama_ref import OracleLlama


class FP64Accumulate(OracleLlama):
    """The oracle with fp64 accumulation and its bf16 rounding points kept."""

    def __init__(self, sd, d=None):
        if d is None:
            super().__init__(sd, mode="exact")
        else:
            super().__init__(sd, d, mode="exact")
        self.mode = "mk"

    def rnd(self, x):
        return x.to(torch.bfloat16).to(self.dt)


class FP64AccumulateFP32P(FP64Accumulate):
    round_p = False


def rms(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.double() - b.double()).pow(2).mean().sqrt().item()
