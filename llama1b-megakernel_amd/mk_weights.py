"""Weights for the decode megakernel: synthetic init, checkpoint loading, packing.

Three jobs, all done once at load time, never per step:

1. ``synthetic_state_dict`` builds a Hugging Face-format Llama state dict with
   N(0, 0.02) bf16 matrices and unit RMSNorm gammas (the random-init
   convention of the reference's block tests, block_testing_utils.py:446-455,
   with gammas kept at one as HF/NxDI initialise them, llama.py:141).
2. ``load_hf_checkpoint`` reads a local safetensors checkpoint (no network).
3. ``pack_for_megakernel`` is this build's counterpart of
   ``NeuronLlamaForCausalLMMK.convert_hf_to_neuron_state_dict``
   (llama_with_megakernel.py:281-351): it folds the pre-attention and
   post-attention RMSNorm gammas into the projections that consume the normed
   activations (fp32 multiply, then bf16, as llama_with_megakernel.py:312-316
   does) and stacks the 16 layers. The layout is this build's own: row-major
   ``[out, in]`` per projection so a GEMV streams each output row as one
   contiguous run of 16-byte loads. Two row permutations serve the fused
   epilogues:

   * QKV rows are ordered in RoPE pairs ``(d, d + 32)`` of one head, so the
     two elements RoPE rotates together come out of the same workgroup;
     Q pairs first (32 heads x 32), then K pairs (8 x 32), then V pairs.
   * gate/up rows are interleaved ``(gate_i, up_i)`` so SwiGLU is computed
     in registers of the wave that produced both dot products.

   The NKI tile-transposes of the reference (llama_with_megakernel.py:44-62,
   mlp.py:37-57) describe the Trainium SBUF partition layout and are not used.

The RoPE table (``rope_table``) is the Llama-3 rotary embedding of
``Llama3RotaryEmbedding`` (llama.py:888-953) precomputed for every cache row:
fp32 inverse frequencies with llama3 smoothing, fp32 cos/sin, cast to bf16.
The kernel indexes it by the device-side position, so no host work is needed
per step.
"""

from __future__ import annotations

import concurrent.futures as _futures
import math
import os
from typing import Dict, Iterable, List, Optional, Tuple

import torch

from mk_config import LLAMA_3_2_1B, LlamaDims

INIT_STD = 0.02


def param_specs(d: LlamaDims = LLAMA_3_2_1B) -> List[Tuple[str, Tuple[int, ...], str]]:
    """HF parameter names, shapes and init kind ("normal" or "ones"), in the
    fixed order used by ``synthetic_state_dict``."""
    h, i = d.hidden, d.intermediate
    specs: List[Tuple[str, Tuple[int, ...], str]] = [("embed_tokens.weight", (d.vocab, h), "normal")]
    for l in range(d.n_layers):
        p = f"layers.{l}."
        specs += [
            (p + "self_attn.q_proj.weight", (d.q_dim, h), "normal"),
            (p + "self_attn.k_proj.weight", (d.kv_dim, h), "normal"),
            (p + "self_attn.v_proj.weight", (d.kv_dim, h), "normal"),
            (p + "self_attn.o_proj.weight", (h, d.q_dim), "normal"),
            (p + "mlp.gate_proj.weight", (i, h), "normal"),
            (p + "mlp.up_proj.weight", (i, h), "normal"),
            (p + "mlp.down_proj.weight", (h, i), "normal"),
            (p + "input_layernorm.weight", (h,), "ones"),
            (p + "post_attention_layernorm.weight", (h,), "ones"),
        ]
    specs.append(("norm.weight", (h,), "ones"))
    return specs


def _param_seed(seed: int, index: int) -> int:
    # One independent CPU generator per parameter: deterministic on every
    # machine and thread count, and lets the parameters be drawn in parallel.
    return (seed * 1_000_003 + index * 7_919 + 12_345) & 0x7FFF_FFFF_FFFF


def _draw(shape: Tuple[int, ...], kind: str, gen_seed: int) -> torch.Tensor:
    if kind == "ones":
        return torch.ones(shape, dtype=torch.bfloat16)
    g = torch.Generator(device="cpu").manual_seed(gen_seed)
    t = torch.empty(shape, dtype=torch.float32)
    t.normal_(0.0, INIT_STD, generator=g)
    return t.to(torch.bfloat16)


def synthetic_state_dict(seed: int = 0, d: LlamaDims = LLAMA_3_2_1B,
                         workers: int | None = None) -> Dict[str, torch.Tensor]:
    """Random-init HF-format state dict: N(0, 0.02) bf16 matrices, unit gammas.

    Parameter k of ``param_specs`` is drawn from its own CPU generator seeded
    with ``_param_seed(seed, k)``; fp32 ``normal_`` then round-to-nearest bf16.
    """
    specs = param_specs(d)
    if workers is None:
        workers = max(1, min(16, len(os.sched_getaffinity(0))))
    out: Dict[str, torch.Tensor] = {}
    with _futures.ThreadPoolExecutor(max_workers=workers) as ex:
        futs = {ex.submit(_draw, shape, kind, _param_seed(seed, k)): name
                for k, (name, shape, kind) in enumerate(specs)}
        for f in futs:
            out[futs[f]] = f.result()
    return {name: out[name] for name, _, _ in specs}


def load_hf_checkpoint(path: str, d: LlamaDims = LLAMA_3_2_1B) -> Dict[str, torch.Tensor]:
    """Read a local HF Llama checkpoint (``*.safetensors``) into the state-dict
    naming of ``param_specs`` (``model.`` prefix stripped). Only safetensors is
    accepted: nothing executable is ever loaded from a checkpoint.

    The kernel's lm_head is the embedding (tied weights, as Llama-3.2-1B ships
    and llama.py:1404-1406 ties them when the config asks). A checkpoint whose
    ``config.json`` sets ``tie_word_embeddings`` to false, or that holds an
    ``lm_head.weight`` different from ``embed_tokens.weight``, is refused."""
    import json
    from safetensors.torch import load_file

    cfg_path = os.path.join(path, "config.json")
    if os.path.exists(cfg_path):
        with open(cfg_path) as f:
            cfg = json.load(f)
        if cfg.get("tie_word_embeddings", True) is False:
            raise ValueError(f"{path}: tie_word_embeddings is false; the megakernel's lm_head is the embedding")

    files = sorted(f for f in os.listdir(path) if f.endswith(".safetensors"))
    if not files:
        raise FileNotFoundError(f"no .safetensors files under {path}")
    raw: Dict[str, torch.Tensor] = {}
    for f in files:
        raw.update(load_file(os.path.join(path, f)))
    sd: Dict[str, torch.Tensor] = {}
    for k, v in raw.items():
        k2 = k[len("model."):] if k.startswith("model.") else k
        sd[k2] = v.to(torch.bfloat16)
    for name, shape, _ in param_specs(d):
        if name not in sd:
            raise KeyError(f"checkpoint lacks {name}")
        if tuple(sd[name].shape) != shape:
            raise ValueError(f"{name}: shape {tuple(sd[name].shape)} != {shape}")
    lm = sd.pop("lm_head.weight", None)
    if lm is not None and not torch.equal(lm.view(torch.int16), sd["embed_tokens.weight"].view(torch.int16)):
        raise ValueError(f"{path}: lm_head.weight differs from embed_tokens.weight (untied); "
                         "the megakernel's lm_head is the embedding")
    return sd


# ----------------------------------------------------------------------------
# Packing (load-time layout for the megakernel)
# ----------------------------------------------------------------------------

def qkv_pair_rows(d: LlamaDims = LLAMA_3_2_1B) -> torch.Tensor:
    """Row order of the packed QKV matrix, as indices into cat(Wq, Wk, Wv).

    Pair p covers rows (d, d + half) of one head: Q heads first, then K
    heads, then V heads; within a head d runs 0..half-1.
    """
    half = d.head_dim // 2
    rows: List[int] = []
    base = 0
    for n_heads in (d.n_q_heads, d.n_kv_heads, d.n_kv_heads):
        for hh in range(n_heads):
            for j in range(half):
                r = base + hh * d.head_dim + j
                rows += [r, r + half]
        base += n_heads * d.head_dim
    return torch.tensor(rows, dtype=torch.long)


def fold_gamma(weight: torch.Tensor, gamma: torch.Tensor) -> torch.Tensor:
    """W' = bf16(W * gamma) over input columns, computed in fp32
    (llama_with_megakernel.py:312-316)."""
    return (weight.float() * gamma.float().unsqueeze(0)).to(torch.bfloat16)


def pack_layer(sd: Dict[str, torch.Tensor], l: int, d: LlamaDims = LLAMA_3_2_1B,
               device: str | torch.device = "cpu") -> Dict[str, torch.Tensor]:
    """Packed tensors of one layer (on ``device``)."""
    p = f"layers.{l}."
    g_in = sd[p + "input_layernorm.weight"].to(device)
    g_post = sd[p + "post_attention_layernorm.weight"].to(device)
    wq = fold_gamma(sd[p + "self_attn.q_proj.weight"].to(device), g_in)
    wk = fold_gamma(sd[p + "self_attn.k_proj.weight"].to(device), g_in)
    wv = fold_gamma(sd[p + "self_attn.v_proj.weight"].to(device), g_in)
    qkv = torch.cat([wq, wk, wv], dim=0)
    qkv = qkv.index_select(0, qkv_pair_rows(d).to(device))
    gate = fold_gamma(sd[p + "mlp.gate_proj.weight"].to(device), g_post)
    up = fold_gamma(sd[p + "mlp.up_proj.weight"].to(device), g_post)
    gu = torch.stack([gate, up], dim=1).reshape(2 * d.intermediate, d.hidden)
    return {
        "w_qkv": qkv.contiguous(),
        "w_o": sd[p + "self_attn.o_proj.weight"].to(device).contiguous(),
        "w_gu": gu.contiguous(),
        "w_down": sd[p + "mlp.down_proj.weight"].to(device).contiguous(),
    }


def mfma_tiles(w: torch.Tensor) -> torch.Tensor:
    """The MFMA tile order of a row-major bf16 matrix (or stack) [..., N, K]
    (N % 16 == 0, K % 32 == 0) that the batched kernel reads: for each 16-row
    tile and 32-column k-step a 1 KiB block, in it the 8 columns 8j..8j+7 of
    row r at 16-byte slot j*16 + r (the B operand of one
    v_mfma_f32_16x16x32_bf16, lane = slot). Same number of elements."""
    *lead, n, k = w.shape
    if n % 16 or k % 32:
        raise ValueError(f"cannot tile a [{n}, {k}] matrix (rows % 16, columns % 32)")
    t = w.reshape(*lead, n // 16, 16, k // 32, 4, 8)
    nd = len(lead)
    perm = list(range(nd)) + [nd, nd + 2, nd + 3, nd + 1, nd + 4]
    return t.permute(*perm).contiguous().reshape(w.shape)


def pack_for_megakernel(sd: Dict[str, torch.Tensor], d: LlamaDims = LLAMA_3_2_1B,
                        device: str | torch.device = "cpu",
                        rope_rows: int = 8192, tiled: Optional[bool] = None) -> Dict[str, torch.Tensor]:
    """Layer-stacked packed weights: w_qkv [L,3072,2048], w_o [L,2048,2048],
    w_gu [L,16384,2048], w_down [L,2048,8192], embed [V,2048], norm_final
    [2048], rope [rope_rows,128] (cos | sin), all bf16 on ``device``; with
    ``tiled`` (default: on a GPU) also t_qkv, t_o, t_gu, t_down, t_embed, the
    ``mfma_tiles`` copies the batched kernel streams (+2.9 GiB at full size)."""
    L = d.n_layers
    packed = {
        "w_qkv": torch.empty((L, d.qkv_rows, d.hidden), dtype=torch.bfloat16, device=device),
        "w_o": torch.empty((L, d.hidden, d.q_dim), dtype=torch.bfloat16, device=device),
        "w_gu": torch.empty((L, 2 * d.intermediate, d.hidden), dtype=torch.bfloat16, device=device),
        "w_down": torch.empty((L, d.hidden, d.intermediate), dtype=torch.bfloat16, device=device),
    }
    for l in range(L):
        for k, v in pack_layer(sd, l, d, device).items():
            packed[k][l].copy_(v)
    packed["embed"] = sd["embed_tokens.weight"].to(device).contiguous()
    packed["norm_final"] = sd["norm.weight"].to(device).contiguous()
    packed["rope"] = rope_table(rope_rows, d).to(device)
    if tiled is None:
        tiled = torch.device(device).type == "cuda"
    if tiled:
        for t, src in (("t_qkv", "w_qkv"), ("t_o", "w_o"), ("t_gu", "w_gu"), ("t_down", "w_down"), ("t_embed", "embed")):
            packed[t] = mfma_tiles(packed[src])
    return packed


def unpack_layer(packed: Dict[str, torch.Tensor], l: int,
                 d: LlamaDims = LLAMA_3_2_1B) -> Dict[str, torch.Tensor]:
    """Inverse of the row permutations of ``pack_layer`` (for tests)."""
    qkv = packed["w_qkv"][l]
    inv = torch.empty_like(qkv)
    inv[qkv_pair_rows(d).to(qkv.device)] = qkv
    q, k, v = inv.split([d.q_dim, d.kv_dim, d.kv_dim], dim=0)
    gu = packed["w_gu"][l].reshape(d.intermediate, 2, d.hidden)
    return {"q": q, "k": k, "v": v, "o": packed["w_o"][l], "gate": gu[:, 0],
            "up": gu[:, 1], "down": packed["w_down"][l]}


# ----------------------------------------------------------------------------
# RoPE table
# ----------------------------------------------------------------------------

def llama3_inv_freq(d: LlamaDims = LLAMA_3_2_1B) -> torch.Tensor:
    """fp32 inverse frequencies with llama3 smoothing (llama.py:917-936).

    Element-wise the same fp32 operations as the reference's per-frequency
    loop, evaluated on the whole vector at once.
    """
    idx = torch.arange(0, d.head_dim, 2, dtype=torch.float32)
    base = 1.0 / (d.rope_theta ** (idx / d.head_dim))
    low_wl = d.rope_original_max_pos / d.rope_low_freq_factor
    high_wl = d.rope_original_max_pos / d.rope_high_freq_factor
    wl = 2 * math.pi / base
    smooth = (d.rope_original_max_pos / wl - d.rope_low_freq_factor) / (
        d.rope_high_freq_factor - d.rope_low_freq_factor)
    mid = (1 - smooth) * base / d.rope_factor + smooth * base
    out = torch.where(wl < high_wl, base, torch.where(wl > low_wl, base / d.rope_factor, mid))
    return out.to(torch.float32)


def rope_table(rows: int, d: LlamaDims = LLAMA_3_2_1B) -> torch.Tensor:
    """bf16 [rows, 2*head_dim]: cos(pos*f) | sin(pos*f) with f = cat(inv, inv)
    (llama.py:938-953: fp32 freqs, fp32 cos/sin, cast to bf16)."""
    inv = llama3_inv_freq(d)
    pos = torch.arange(rows, dtype=torch.float32)
    freqs = pos[:, None] * inv[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return torch.cat([emb.cos(), emb.sin()], dim=-1).to(torch.bfloat16).contiguous()


def random_token_ids(n: int, seed: int = 0, d: LlamaDims = LLAMA_3_2_1B) -> torch.Tensor:
    """Uniform token ids in [0, vocab) from a CPU generator seeded ``seed``
    (a second generator, independent of the weight generators)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randint(0, d.vocab, (n,), generator=g, dtype=torch.int64)


def state_dict_fingerprint(sd: Dict[str, torch.Tensor], names: Iterable[str] | None = None):
    """SHA-256 of each tensor's bytes plus its first 16 values."""
    import hashlib
    out = {}
    for k in (names if names is not None else sd.keys()):
        t = sd[k].contiguous()
        b = t.view(torch.int16).numpy().tobytes()
        out[k] = {"sha256": hashlib.sha256(b).hexdigest(),
                  "first16": [float(x) for x in t.flatten()[:16].float()]}
    return out
