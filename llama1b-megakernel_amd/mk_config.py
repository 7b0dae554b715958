"""Llama-3.2-1B model constants and the decode-step configuration.

The megakernel is specialised for one architecture, as the reference kernel is
(nki_kernels/attention.py:19-32, nki_kernels/mlp.py:29-34,
transformer_llama.py:30-36). The values below are those constants, gathered in
one frozen dataclass instead of module globals with side effects
(llama.py:91, 157-159 sets a global flag; this build keeps no global state).
"""

from __future__ import annotations

import dataclasses


@dataclasses.dataclass(frozen=True)
class LlamaDims:
    """Architecture of the model the kernel is built for."""

    n_layers: int = 16            # transformer_llama.py:30
    hidden: int = 2048            # attention.py:20
    n_q_heads: int = 32           # attention.py:22
    n_kv_heads: int = 8           # attention.py:23
    head_dim: int = 64            # attention.py:21
    intermediate: int = 8192      # mlp.py:31
    vocab: int = 128256           # tied embeddings (llama.py:1404-1406)
    rms_eps: float = 1e-5         # attention.py:30
    rope_theta: float = 500000.0  # llama.py:897-906 (llama3 rope defaults)
    rope_factor: float = 8.0
    rope_low_freq_factor: float = 1.0
    rope_high_freq_factor: float = 4.0
    rope_original_max_pos: int = 8192

    @property
    def gqa_group(self) -> int:
        return self.n_q_heads // self.n_kv_heads

    @property
    def q_dim(self) -> int:
        return self.n_q_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    @property
    def qkv_rows(self) -> int:
        return self.q_dim + 2 * self.kv_dim


LLAMA_3_2_1B = LlamaDims()

# Bytes moved by one decode step, used for the roofline (algorithmic bytes:
# each weight read once, KV rows read only below the write position).
BF16 = 2


def layer_weight_bytes(d: LlamaDims = LLAMA_3_2_1B) -> int:
    h, i = d.hidden, d.intermediate
    return BF16 * (h * d.q_dim + 2 * h * d.kv_dim + d.q_dim * h + 3 * h * i)


def step_bytes(n_layers: int, kv_rows_read: list[int], lm_head: bool,
               d: LlamaDims = LLAMA_3_2_1B, logits_bytes: int = 4) -> int:
    """Algorithmic HBM bytes of one decode step.

    kv_rows_read[b] is the number of cache rows sequence b attends to that were
    already in the cache (its position before the step). Per sequence the step
    also writes one K and one V row per layer and reads its embedding row.
    """
    row = d.n_kv_heads * d.head_dim * BF16          # one K (or V) row of one layer
    total = n_layers * layer_weight_bytes(d)
    for t in kv_rows_read:
        total += n_layers * 2 * row * t               # K and V reads
        total += n_layers * 2 * row                   # K and V row writes
        total += d.hidden * BF16                      # embedding / hidden-in row
    if lm_head:
        total += d.vocab * d.hidden * BF16            # tied lm_head
        total += d.hidden * BF16                      # final norm gamma
        total += len(kv_rows_read) * d.vocab * logits_bytes
    return total
