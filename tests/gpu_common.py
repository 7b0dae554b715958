"""Helpers shared by the ``-m gpu`` tests (imported by them only)."""

from __future__ import annotations

import sys

import pytest
import torch


def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mk_lib
    if not mk_lib.LIB_PATH.exists():
        raise RuntimeError("libmk.so is not built: run __graft_entry__.build() first")


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 values at |x| (1 ulp), floored at the normal minimum."""
    ax = x.float().abs().clamp_min(1e-30)
    e = torch.floor(torch.log2(ax))
    return torch.pow(2.0, e - 7)


def packed_on_device(sd, dims, rope_rows, device="cuda"):
    from mk_weights import pack_for_megakernel
    return pack_for_megakernel(sd, dims, device=device, rope_rows=rope_rows)


def new_caches(n_layers, s_max, device="cuda", fill=None, seed=0):
    """Per-layer K and V caches bf16 [1, 8, s_max, 64] (optionally N(0,1))."""
    ks, vs = [], []
    g = torch.Generator().manual_seed(seed)
    for _ in range(n_layers):
        if fill == "randn":
            k = torch.randn(1, 8, s_max, 64, generator=g).to(torch.bfloat16)
            v = torch.randn(1, 8, s_max, 64, generator=g).to(torch.bfloat16)
        else:
            k = torch.zeros(1, 8, s_max, 64, dtype=torch.bfloat16)
            v = torch.zeros(1, 8, s_max, 64, dtype=torch.bfloat16)
        ks.append(k.to(device))
        vs.append(v.to(device))
    return ks, vs


def record_parity(name: str, data: dict) -> None:
    """Write a test's measured parity numbers as <name>.json into the directory
    MK_PARITY_DIR, else the repository's run-output folder (`parity/` under
    it); the committed parity summary under profiles/ cites these files."""
    import json
    import os
    from pathlib import Path
    out = Path(os.environ.get("MK_PARITY_DIR", Path(__file__).resolve().parents[1] / "gpurun_out" / "parity"))
    out.mkdir(parents=True, exist_ok=True)
    (out / f"{name}.json").write_text(json.dumps(data, indent=1, sort_keys=True))


def logit_stats(got: torch.Tensor, ref: torch.Tensor) -> dict:
    d = (got.float() - ref.float()).abs()
    return {"max_abs": round(d.max().item(), 5), "rms": round(d.pow(2).mean().sqrt().item(), 5)}
