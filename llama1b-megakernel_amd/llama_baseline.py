"""The stock (unfused) PyTorch Llama-3.2-1B decode path, in fp32 on the GPU.

The counterpart of the reference's baseline model in ``main.py --mode
validate``: the reference compares its megakernel model with NxDI's stock
Llama (``baseline_llama.NeuronLlamaForCausalLM``, main.py:23, 568); this build
compares with this module. It is plain PyTorch operations (embedding, RMSNorm,
Llama-3 RoPE, GQA attention with a KV cache, SwiGLU MLP, tied lm_head) on
fp32 copies of the same weights, so it carries no bf16 rounding; it is only
ever used as the comparison model of validate mode, never as a stand-in for
the megakernel.
"""

from __future__ import annotations

from typing import Dict

import torch

from mk_config import LLAMA_3_2_1B, LlamaDims
from mk_weights import llama3_inv_freq


class StockLlama:
    def __init__(self, sd: Dict[str, torch.Tensor], d: LlamaDims = LLAMA_3_2_1B, device: str = "cuda",
                 s_max: int = 1024):
        self.d, self.dev = d, torch.device(device)
        f = lambda k: sd[k].to(device=self.dev, dtype=torch.float32)
        self.embed = f("embed_tokens.weight")
        self.norm = f("norm.weight")
        self.layers = []
        for l in range(d.n_layers):
            p = f"layers.{l}."
            self.layers.append({k: f(p + v) for k, v in {
                "q": "self_attn.q_proj.weight", "k": "self_attn.k_proj.weight", "v": "self_attn.v_proj.weight",
                "o": "self_attn.o_proj.weight", "g": "mlp.gate_proj.weight", "u": "mlp.up_proj.weight",
                "dn": "mlp.down_proj.weight", "n1": "input_layernorm.weight",
                "n2": "post_attention_layernorm.weight"}.items()})
        self.inv_freq = llama3_inv_freq(d).to(self.dev)
        self.K = torch.zeros(d.n_layers, d.n_kv_heads, s_max, d.head_dim, device=self.dev)
        self.V = torch.zeros_like(self.K)

    def _norm(self, x, w):
        return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.d.rms_eps))

    def _rope(self, x, pos):
        f = pos * self.inv_freq
        emb = torch.cat([f, f])
        c, s = emb.cos(), emb.sin()
        h = x.shape[-1] // 2
        return x * c + torch.cat([-x[..., h:], x[..., :h]], -1) * s

    @torch.no_grad()
    def step(self, token: int, pos: int) -> torch.Tensor:
        """One decode step; returns fp32 logits [vocab]."""
        d = self.d
        x = self.embed[token]
        for l, W in enumerate(self.layers):
            xn = self._norm(x, W["n1"])
            q = (W["q"] @ xn).view(d.n_q_heads, d.head_dim)
            k = (W["k"] @ xn).view(d.n_kv_heads, d.head_dim)
            v = (W["v"] @ xn).view(d.n_kv_heads, d.head_dim)
            q, k = self._rope(q, float(pos)), self._rope(k, float(pos))
            self.K[l, :, pos] = k
            self.V[l, :, pos] = v
            Kh = self.K[l, :, :pos + 1].repeat_interleave(d.gqa_group, 0).contiguous()
            Vh = self.V[l, :, :pos + 1].repeat_interleave(d.gqa_group, 0).contiguous()
            s = torch.matmul(Kh, q.unsqueeze(-1).contiguous()).squeeze(-1) / d.head_dim ** 0.5   # [h, S]
            o = torch.matmul(torch.softmax(s, -1).unsqueeze(1).contiguous(), Vh).reshape(-1)     # [h*D]
            x = x + W["o"] @ o
            xn = self._norm(x, W["n2"])
            x = x + W["dn"] @ (torch.nn.functional.silu(W["g"] @ xn) * (W["u"] @ xn))
        return self.embed @ self._norm(x, self.norm)
