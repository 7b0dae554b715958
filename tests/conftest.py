"""Shared test setup.

``-m gpu`` tests need an MI355X (they run through ``libmk.so``); everything
else runs on the CPU. The package source directory and the repo root are put
on ``sys.path`` so tests import the product modules by name and the oracle as
``oracle.*``.
"""

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "llama1b-megakernel_amd"
for p in (str(PKG), str(REPO)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built libmk.so")


def small_dims():
    """A reduced Llama (same head_dim, GQA group and RoPE) for fast CPU tests:
    returns (product LlamaDims, oracle Dims)."""
    from mk_config import LlamaDims
    from oracle.llama_ref import Dims
    kw = dict(n_layers=2, hidden=256, n_q=4, n_kv=1, head_dim=64, inter=512, vocab=1000)
    prod = LlamaDims(n_layers=kw["n_layers"], hidden=kw["hidden"], n_q_heads=kw["n_q"],
                     n_kv_heads=kw["n_kv"], head_dim=kw["head_dim"], intermediate=kw["inter"],
                     vocab=kw["vocab"])
    return prod, Dims(**kw)


@pytest.fixture(scope="session")
def small():
    return small_dims()


@pytest.fixture(scope="session")
def llama_1b_sd():
    """Seed-0 synthetic Llama-3.2-1B weights (HF naming, bf16, CPU)."""
    from mk_weights import synthetic_state_dict
    return synthetic_state_dict(seed=0)
