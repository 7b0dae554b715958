"""CPU oracle for the Llama-3.2-1B decode step — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker. The product
(the HIP megakernel behind ``libmk.so``) never calls it.

It restates, in plain PyTorch on the CPU, the math of the reference's
megakernel decode step and of the Llama decoder it replaces:

* layer order: pre-norm attention, residual, pre-norm MLP, residual
  (llama.py:1039-1139; transformer_llama.py:40-85);
* RMSNorm with the gamma folded into the consuming projection in fp32 then
  cast to bf16 (llama_with_megakernel.py:312-316); the kernel applies only
  ``x * rsqrt(mean(x^2) + eps)`` in fp32 and casts to bf16
  (attention.py:77-93, mlp.py:80-96);
* Q/K/V projections with fp32 accumulation cast to bf16
  (attention.py:143-158, 176-187, 189-227);
* split-half RoPE ``x*cos + rotate_half(x)*sin`` with bf16 intermediates
  (attention.py:160-174, 229-245) and llama3-scaled frequencies
  (llama.py:917-953);
* GQA attention, q head h reads kv head h // 4 (attention.py:207-210), over
  the cached rows below ``pos`` plus the fresh K/V row; single-pass softmax in
  fp32, ``exp`` cast to bf16 before the PV product, fp32 denominator,
  multiply by its reciprocal, cast to bf16 (attention.py:303-399);
* O projection (attention.py:409-448) and bf16 residual adds
  (transformer_llama.py:68-70, 82-84);
* MLP ``bf16(silu(g) * u)`` with g, u fp32 accumulators, then the down
  projection (mlp.py:98-192; llama.py:755-780);
* the in-place K/V scatter at row ``pos`` (attention.py:450-492);
* final RMSNorm as HF ``LlamaRMSNorm`` (the CPU path, llama.py:176-178):
  ``bf16(g * bf16(x * rsqrt(mean(x^2)+eps)))``, tied lm_head
  (llama.py:1404-1406) with fp32 logits, greedy argmax.

Two modes:

* ``"mk"``  — bf16 rounding at the reference kernel's points, fp32
  accumulation (the parity target for the GPU kernel);
* ``"exact"`` — float64 everywhere, no rounding (used to pin this code
  against the independent HF ``LlamaForCausalLM`` implementation).

How each piece is pinned is stated in the tests under ``tests/``.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Dict, List, Optional, Tuple

import torch


@dataclasses.dataclass(frozen=True)
class Dims:
    n_layers: int = 16
    hidden: int = 2048
    n_q: int = 32
    n_kv: int = 8
    head_dim: int = 64
    inter: int = 8192
    vocab: int = 128256
    eps: float = 1e-5
    rope_theta: float = 500000.0
    rope_factor: float = 8.0
    rope_low: float = 1.0
    rope_high: float = 4.0
    rope_orig: int = 8192


LLAMA_1B = Dims()
MASK_VALUE = -3.4028234663852886e38   # attention.py:32
SOFTMAX_SCALE_FOR = lambda hd: 1.0 / math.sqrt(hd)   # attention.py:31


def inv_freq(d: Dims) -> torch.Tensor:
    """llama3 inverse frequencies in fp32 (llama.py:917-936): the reference's
    per-frequency branch, one frequency at a time."""
    idx = torch.arange(0, d.head_dim, 2, dtype=torch.float32)
    raw = 1.0 / (d.rope_theta ** (idx / d.head_dim))
    low_wl = d.rope_orig / d.rope_low
    high_wl = d.rope_orig / d.rope_high
    vals = []
    for f in raw:
        wl = 2 * math.pi / f
        if wl < high_wl:
            vals.append(f)
        elif wl > low_wl:
            vals.append(f / d.rope_factor)
        else:
            s = (d.rope_orig / wl - d.rope_low) / (d.rope_high - d.rope_low)
            vals.append((1 - s) * f / d.rope_factor + s * f)
    return torch.tensor(vals, dtype=torch.float32)


def cos_sin(d: Dims, positions: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos, sin of shape [T, head_dim] (llama.py:938-953)."""
    f = positions.to(torch.float32)[:, None] * inv_freq(d)[None, :]
    emb = torch.cat([f, f], dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


class OracleLlama:
    """Decode/prefill restatement over an HF-format state dict."""

    def __init__(self, sd: Dict[str, torch.Tensor], d: Dims = LLAMA_1B, mode: str = "mk",
                 fold: bool = True):
        if mode not in ("mk", "exact"):
            raise ValueError(mode)
        self.d, self.mode = d, mode
        self.dt = torch.float32 if mode == "mk" else torch.float64
        dt = self.dt

        def fold_g(w, g):
            # llama_with_megakernel.py:312-316 (fp32 multiply, bf16 result)
            if mode == "mk":
                return (w.float() * g.float().unsqueeze(0)).to(torch.bfloat16).to(dt)
            return w.to(dt) * g.to(dt).unsqueeze(0)

        self.layers = []
        for l in range(d.n_layers):
            p = f"layers.{l}."
            g_in = sd[p + "input_layernorm.weight"]
            g_post = sd[p + "post_attention_layernorm.weight"]
            if fold:
                wq = fold_g(sd[p + "self_attn.q_proj.weight"], g_in)
                wk = fold_g(sd[p + "self_attn.k_proj.weight"], g_in)
                wv = fold_g(sd[p + "self_attn.v_proj.weight"], g_in)
                wg = fold_g(sd[p + "mlp.gate_proj.weight"], g_post)
                wu = fold_g(sd[p + "mlp.up_proj.weight"], g_post)
                gi = gp = None
            else:
                wq, wk, wv = (sd[p + f"self_attn.{n}_proj.weight"].to(dt) for n in "qkv")
                wg = sd[p + "mlp.gate_proj.weight"].to(dt)
                wu = sd[p + "mlp.up_proj.weight"].to(dt)
                gi, gp = g_in.to(dt), g_post.to(dt)
            self.layers.append({
                "wq_t": wq.t().contiguous(), "wk_t": wk.t().contiguous(), "wv_t": wv.t().contiguous(),
                "wo_t": sd[p + "self_attn.o_proj.weight"].to(dt).t().contiguous(),
                "wg_t": wg.t().contiguous(), "wu_t": wu.t().contiguous(),
                "wd_t": sd[p + "mlp.down_proj.weight"].to(dt).t().contiguous(),
                "g_in": gi, "g_post": gp,
            })
        self.embed = sd["embed_tokens.weight"].to(dt)
        self.embed_t = self.embed.t().contiguous()
        self.g_final = sd["norm.weight"].to(dt)
        self.scale = SOFTMAX_SCALE_FOR(d.head_dim)

    # The reference casts exp(s - max) to bf16 before the PV product
    # (attention.py:376-387); a variant with round_p = False keeps p unrounded,
    # as a split-K kernel must (its per-split maxima differ from the global one).
    round_p = True

    # -- rounding -----------------------------------------------------------
    def rnd(self, x: torch.Tensor) -> torch.Tensor:
        """bf16 rounding point (round-to-nearest-even) in mk mode; identity in exact mode."""
        if self.mode == "mk":
            return x.to(torch.bfloat16).to(self.dt)
        return x

    # -- blocks ---------------------------------------------------------------
    def norm_scale(self, x: torch.Tensor) -> torch.Tensor:
        """fp32 (or fp64) x * rsqrt(mean(x^2) + eps) over the last dim."""
        ss = (x * x).sum(-1, keepdim=True)
        return x * torch.rsqrt(ss / self.d.hidden + self.d.eps)

    def rope(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        # attention.py:160-174 / 229-245: bf16(bf16(x*cos) + bf16(rot(x)*sin))
        return self.rnd(self.rnd(x * cos) + self.rnd(rotate_half(x) * sin))

    def attention(self, q, K, V, n_valid):
        """q [T, n_q, D]; K, V [n_kv, S, D]; query t attends rows [0, n_valid[t]).

        Single pass: scores fp32 * scale, masked rows get MASK_VALUE, p = exp(s - max),
        numerator sum_j rnd(p_j) V_j, denominator sum_j p_j (fp32), times 1/denominator.
        """
        d = self.d
        n_valid = torch.as_tensor(n_valid)
        # rows at or beyond every query's limit are never read (stale or unset cache rows)
        S = int(n_valid.max())
        K, V = K[:, :S], V[:, :S]
        T = q.shape[0]
        g = d.n_q // d.n_kv
        kk = K.repeat_interleave(g, dim=0)            # [n_q, S, D]: q head h -> kv head h // g
        vv = V.repeat_interleave(g, dim=0)
        s = torch.einsum("thd,hsd->hts", q, kk) * self.scale     # [n_q, T, S]
        j = torch.arange(S)[None, :]
        mask = j >= torch.as_tensor(n_valid)[:, None]               # [T, S]
        s = s.masked_fill(mask[None], MASK_VALUE)
        m = s.max(-1, keepdim=True).values
        p = torch.exp(s - m)
        p = p.masked_fill(mask[None], 0.0)
        den = p.sum(-1, keepdim=True)
        num = torch.einsum("hts,hsd->htd", self.rnd(p) if self.round_p else p, vv)
        o = num * (1.0 / den)
        return self.rnd(o).permute(1, 0, 2)            # [T, n_q, D]

    def layer(self, l: int, h: torch.Tensor, positions: torch.Tensor, cache: Tuple[torch.Tensor, torch.Tensor]):
        """One decoder layer over T new tokens at ``positions`` (consecutive).

        h: [T, H] (bf16-valued in mk mode); cache (K, V) [n_kv, S, D] updated in place.
        """
        d, W = self.d, self.layers[l]
        T = h.shape[0]
        K, V = cache
        xn = self.norm_scale(h)
        if W["g_in"] is not None:
            xn = W["g_in"] * self.rnd(xn)
        xn = self.rnd(xn)
        q = self.rnd(xn @ W["wq_t"]).view(T, d.n_q, d.head_dim)
        k = self.rnd(xn @ W["wk_t"]).view(T, d.n_kv, d.head_dim)
        v = self.rnd(xn @ W["wv_t"]).view(T, d.n_kv, d.head_dim)
        cos, sin = self.cos_sin(positions)
        q = self.rope(q, cos[:, None, :], sin[:, None, :])
        k = self.rope(k, cos[:, None, :], sin[:, None, :])
        # in-place scatter of the fresh rows (attention.py:450-492)
        K[:, positions, :] = k.permute(1, 0, 2)
        V[:, positions, :] = v.permute(1, 0, 2)
        o = self.attention(q, K, V, positions + 1)
        attn = self.rnd(o.reshape(T, d.n_q * d.head_dim) @ W["wo_t"])
        h1 = self.rnd(h + attn)
        xn = self.norm_scale(h1)
        if W["g_post"] is not None:
            xn = W["g_post"] * self.rnd(xn)
        xn = self.rnd(xn)
        gt = xn @ W["wg_t"]
        up = xn @ W["wu_t"]
        a = self.rnd(torch.nn.functional.silu(gt) * up)
        mlp = self.rnd(a @ W["wd_t"])
        return self.rnd(h1 + mlp)

    def cos_sin(self, positions: torch.Tensor):
        c, s = cos_sin(self.d, positions)
        if self.mode == "mk":
            return c.to(torch.bfloat16).to(self.dt), s.to(torch.bfloat16).to(self.dt)
        return c.to(self.dt), s.to(self.dt)

    def final_norm(self, h: torch.Tensor) -> torch.Tensor:
        # HF LlamaRMSNorm: weight * bf16(x * rsqrt(mean(x^2)+eps))
        return self.rnd(self.g_final * self.rnd(self.norm_scale(h)))

    def logits(self, h: torch.Tensor) -> torch.Tensor:
        return self.final_norm(h) @ self.embed_t

    # -- driver -----------------------------------------------------------
    def new_cache(self, s_max: int) -> List[Tuple[torch.Tensor, torch.Tensor]]:
        d = self.d
        return [(torch.zeros(d.n_kv, s_max, d.head_dim, dtype=self.dt),
                 torch.zeros(d.n_kv, s_max, d.head_dim, dtype=self.dt)) for _ in range(d.n_layers)]

    def forward(self, tokens: Optional[torch.Tensor], start_pos: int,
                cache: List[Tuple[torch.Tensor, torch.Tensor]],
                hidden: Optional[torch.Tensor] = None, n_layers: Optional[int] = None,
                first_layer: int = 0, want_logits: bool = True):
        """Run T tokens (or T hidden rows) at positions start_pos..start_pos+T-1.

        Returns (logits [T, V] or None, hidden after the last layer [T, H]).
        """
        h = self.embed[tokens] if hidden is None else hidden.to(self.dt)
        h = self.rnd(h)
        T = h.shape[0]
        positions = torch.arange(start_pos, start_pos + T)
        n = self.d.n_layers if n_layers is None else n_layers
        for l in range(first_layer, first_layer + n):
            h = self.layer(l, h, positions, cache[l])
        return (self.logits(h) if want_logits else None), h

    def greedy(self, logits: torch.Tensor) -> torch.Tensor:
        return logits.argmax(-1)
