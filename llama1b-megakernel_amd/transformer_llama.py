"""Multi-layer megakernel entry points, named as in the reference's
transformer_llama.py (transformer_llama.py:147-241).

``transformer_llama_megakernel_16layers(X, w_qkv, w_o, w_gu, w_down,
K_00..K_15, V_00..V_15, rope, position_ids) -> (Y, K_00..K_15, V_00..V_15)``
runs all 16 decoder layers of one token-generation step in ONE launch of the
HIP megakernel (libmk.so). As in the reference (transformer_llama.py:117-144),
each layer's fresh K/V row is scattered in place into K_i / V_i at row
``position_ids`` and the same cache tensors are returned, so a caller that
aliases them (NxDI in the reference) keeps using them.

Differences in the argument list, all load-time layout choices of this build:

* the weights are this build's packed stacks (``mk_weights.pack_for_megakernel``):
  Q/K/V concatenated in RoPE-pair row order, gate/up interleaved, gammas
  folded in. The reference also passes ``gpre_all`` / ``gpost_all``, which its
  kernel never reads (attention.py:77-81, mlp.py:80-84); they are not taken;
* ``cos`` / ``sin`` ([1,1,64] for one position) are replaced by the bf16 RoPE
  table ``rope`` [rows, 128], indexed on the device by ``position_ids``, so
  the step needs no host-side RoPE.

``transformer_llama_megakernel_1layer`` (transformer_llama.py:154-191) is the
single-layer variant, and ``_build_multilayer_kernel(n)`` builds the n-layer
entry (the reference builds 2 and 16, transformer_llama.py:196-241).
"""

from __future__ import annotations

from typing import Callable, Dict, Optional, Sequence, Tuple

import torch

import mk_lib

LLAMA_1B_NUM_LAYERS = 16
LLAMA_1B_HIDDEN = 2048
LLAMA_1B_INTERMEDIATE = 8192
LLAMA_1B_HEAD_DIM = 64
LLAMA_1B_NUM_Q_HEADS = 32
LLAMA_1B_NUM_KV_HEADS = 8
LLAMA_1B_RMS_NORM_EPS = 1e-5

_workspaces: Dict[Tuple[int, int], mk_lib.Workspace] = {}


def _workspace(device: torch.device, s_max: int) -> mk_lib.Workspace:
    key = (device.index or 0, s_max)
    if key not in _workspaces:
        _workspaces[key] = mk_lib.Workspace(1, s_max, device)
    return _workspaces[key]


def _run(X: torch.Tensor, w_qkv: torch.Tensor, w_o: torch.Tensor, w_gu: torch.Tensor, w_down: torch.Tensor,
         K: Sequence[torch.Tensor], V: Sequence[torch.Tensor], rope: torch.Tensor, position_ids: torch.Tensor,
         first_layer: int = 0) -> torch.Tensor:
    n = len(K)
    if len(V) != n or n < 1:
        raise ValueError("need the same number (>= 1) of K and V caches")
    if X.dtype != torch.bfloat16 or X.numel() != LLAMA_1B_HIDDEN:
        raise ValueError(f"X must be bf16 with {LLAMA_1B_HIDDEN} elements (batch 1), got {tuple(X.shape)}")
    for t in list(K) + list(V):
        if t.dtype != torch.bfloat16 or t.shape[-3:-2] != (LLAMA_1B_NUM_KV_HEADS,) or t.shape[-1] != LLAMA_1B_HEAD_DIM:
            raise ValueError(f"caches must be bf16 [1, 8, S, 64], got {tuple(t.shape)}")
    packed = {"w_qkv": w_qkv, "w_o": w_o, "w_gu": w_gu, "w_down": w_down, "embed": w_qkv, "norm_final": w_qkv,
              "rope": rope}
    weights = mk_lib.weights_struct(packed)
    weights.embed = None          # not used: hidden input, no lm_head
    weights.norm_final = None
    s_max = int(K[0].shape[-2])
    ws = _workspace(X.device, s_max)
    pos = position_ids.reshape(-1)[:1].to(device=X.device, dtype=torch.int32)
    Y = torch.empty(1, 1, LLAMA_1B_HIDDEN, dtype=torch.bfloat16, device=X.device)
    mk_lib.decode_step(weights, ws, K, V, pos, hidden_in=X.reshape(1, LLAMA_1B_HIDDEN).contiguous(),
                       hidden_out=Y.view(1, LLAMA_1B_HIDDEN), first_layer=first_layer, n_layers=n)
    return Y


def _build_multilayer_kernel(num_layers: int) -> Callable:
    """Entry for ``num_layers`` layers with individual K/V arguments."""

    def kernel(X, w_qkv, w_o, w_gu, w_down, *rest):
        if len(rest) != 2 * num_layers + 2:
            raise TypeError(f"expected {num_layers} K, {num_layers} V, rope, position_ids")
        K = rest[:num_layers]
        V = rest[num_layers:2 * num_layers]
        rope, position_ids = rest[2 * num_layers], rest[2 * num_layers + 1]
        Y = _run(X, w_qkv, w_o, w_gu, w_down, K, V, rope, position_ids)
        return (Y,) + tuple(K) + tuple(V)

    kernel.__name__ = f"transformer_llama_megakernel_{num_layers}L"
    return kernel


def transformer_llama_megakernel_1layer(X, w_qkv, w_o, w_gu, w_down, K_cache, V_cache, rope, position_ids,
                                        layer: int = 0):
    """Layer ``layer`` of the stacks applied to X; returns (Y, K_cache, V_cache)."""
    Y = _run(X, w_qkv, w_o, w_gu, w_down, [K_cache], [V_cache], rope, position_ids, first_layer=layer)
    return Y, K_cache, V_cache


transformer_llama_megakernel_2layers = _build_multilayer_kernel(2)
transformer_llama_megakernel_16layers = _build_multilayer_kernel(16)
