"""Llama-3.2-1B with the MI355X decode megakernel — the model-level drop-in.

Mirrors the reference module ``llama_with_megakernel`` (selected by
``main.py --enable-nki``, main.py:546-553) and the class it exports,
``NeuronLlamaForCausalLM = NeuronLlamaForCausalLMMK``
(llama_with_megakernel.py:272-355):

* ``get_neuron_config_cls()`` / ``get_config_cls()`` / ``__init__(model_path, config)``
  / ``compile(path)`` / ``load(path)`` / ``reset()`` as used by main.py:121-175;
* ``convert_hf_to_neuron_state_dict(state_dict, config)`` — the load-time
  gamma fold + layer stacking (llama_with_megakernel.py:281-351), here producing
  this build's packed layout (``mk_weights.pack_for_megakernel``);
* the token-generation contract of the megakernel layer
  (llama_with_megakernel.py:95-185): ``forward(hidden or input_ids,
  position_ids, past_key_values) -> (logits, past_key_values)`` where the K/V
  caches are updated in place at ``position_ids`` and returned as the same
  tensors;
* ``generate(input_ids, max_new_tokens)`` — greedy decoding (the reference's
  ``do_sample=False`` / ``top_k=1`` path, main.py:57, 291, 332).

``model_path`` is a local HF checkpoint directory (safetensors) or
``"random:<seed>"`` for the synthetic N(0, 0.02) weights used by the
benchmarks. Prefill (context encoding, the reference's baseline-layer path at
llama_with_megakernel.py:194-204) runs the batched MFMA kernel over chunks of
up to 32 consecutive prompt tokens per launch (``MK_FLAG_PREFILL``: causal
attention over the cache rows, including the rows of the chunk's own earlier
tokens); ``prefill(..., batched=False)`` instead runs the decode megakernel
once per prompt token with logits skipped.

TP must be 1, as the reference asserts (llama_with_megakernel.py:147-150).
"""

from __future__ import annotations

import dataclasses
from typing import Dict, List, Optional, Sequence, Tuple

import torch

import mk_lib
from mk_config import LLAMA_3_2_1B, LlamaDims
from mk_weights import load_hf_checkpoint, pack_for_megakernel, synthetic_state_dict


@dataclasses.dataclass
class NeuronConfigLlamaMK:
    """Run-time configuration (the subset of NxDI's NeuronConfig the
    megakernel path reads; NeuronConfigLlamaMK at llama_with_megakernel.py:253-269)."""

    batch_size: int = 1
    seq_len: int = 1024                    # max_length of a generation
    max_context_length: Optional[int] = None
    max_new_tokens: Optional[int] = None
    tp_degree: int = 1
    torch_dtype: torch.dtype = torch.bfloat16
    enable_nki: bool = True
    on_device_sampling: bool = True
    device: str = "cuda"

    def __post_init__(self):
        if self.max_context_length is None:
            self.max_context_length = self.seq_len
        if self.tp_degree != 1:
            raise ValueError(f"megakernel is TP=1 only, got tp_degree={self.tp_degree}")
        if self.torch_dtype != torch.bfloat16:
            raise ValueError("the megakernel computes in bf16")

    @property
    def max_length(self) -> int:
        return self.seq_len


@dataclasses.dataclass
class LlamaInferenceConfig:
    neuron_config: NeuronConfigLlamaMK
    dims: LlamaDims = LLAMA_3_2_1B


class NeuronLlamaForCausalLMMK:
    """Llama-3.2-1B whose token-generation step is one megakernel launch."""

    @classmethod
    def get_neuron_config_cls(cls):
        return NeuronConfigLlamaMK

    @classmethod
    def get_config_cls(cls):
        return LlamaInferenceConfig

    def __init__(self, model_path: str, config: LlamaInferenceConfig):
        self.model_path = model_path
        self.config = config
        self.neuron_config = config.neuron_config
        self.on_device_sampling = True
        self.packed: Optional[Dict[str, torch.Tensor]] = None
        self._ready = False

    # -- weights -----------------------------------------------------------
    @staticmethod
    def convert_hf_to_neuron_state_dict(state_dict: Dict[str, torch.Tensor], config: LlamaInferenceConfig,
                                        device: str = "cpu") -> Dict[str, torch.Tensor]:
        """Gamma fold + layer stacking into the packed megakernel layout."""
        nc = config.neuron_config
        return pack_for_megakernel(state_dict, config.dims, device=device,
                                   rope_rows=max(nc.max_context_length, nc.seq_len))

    def load_state_dict_source(self) -> Dict[str, torch.Tensor]:
        if self.model_path.startswith("random:"):
            return synthetic_state_dict(seed=int(self.model_path.split(":", 1)[1] or 0), d=self.config.dims)
        return load_hf_checkpoint(self.model_path, self.config.dims)

    def compile(self, compiled_model_path: Optional[str] = None, debug: bool = False) -> None:
        """Pack the weights onto the device (the reference traces and compiles
        a NEFF here; the HIP kernel is compiled ahead of time into libmk.so)."""
        mk_lib.load()   # fails loudly if the native library is missing
        sd = self.load_state_dict_source()
        self.state_dict_bf16 = sd
        self.packed = self.convert_hf_to_neuron_state_dict(sd, self.config, device=self.neuron_config.device)

    def load(self, compiled_model_path: Optional[str] = None) -> None:
        if self.packed is None:
            self.compile(compiled_model_path)
        nc, d = self.neuron_config, self.config.dims
        if nc.batch_size != 1:
            raise NotImplementedError("this build runs batch 1")
        dev = torch.device(nc.device)
        self.s_max = nc.max_context_length
        # past_key_values: one [1, 8, S, 64] K and V tensor per layer, views of one allocation
        self.kv = torch.zeros(d.n_layers, 2, nc.batch_size, d.n_kv_heads, self.s_max, d.head_dim,
                              dtype=torch.bfloat16, device=dev)
        self.k_caches = [self.kv[l, 0] for l in range(d.n_layers)]
        self.v_caches = [self.kv[l, 1] for l in range(d.n_layers)]
        self.weights = mk_lib.weights_struct(self.packed)
        self.ws = mk_lib.Workspace(nc.batch_size, self.s_max, dev)
        self.pos = torch.zeros(nc.batch_size, dtype=torch.int32, device=dev)
        self.tokens = torch.zeros(nc.batch_size, dtype=torch.int32, device=dev)
        self.logits = torch.zeros(nc.batch_size, d.vocab, dtype=torch.float32, device=dev)
        self.hidden_out = torch.zeros(nc.batch_size, d.hidden, dtype=torch.bfloat16, device=dev)
        self.pf_ws: Optional[mk_lib.Workspace] = None   # batched workspace of the prefill steps (on first use)
        self.pf_pos = torch.arange(self.s_max, dtype=torch.int32, device=dev)
        self._ready = True
        self._launchers: Dict[str, mk_lib.StepLauncher] = {}

    def reset(self) -> None:
        """Start a new sequence (rows >= pos are never read, so no cache clear)."""
        self.pos.zero_()

    @property
    def past_key_values(self) -> List[Tuple[torch.Tensor, torch.Tensor]]:
        return list(zip(self.k_caches, self.v_caches))

    # -- steps ---------------------------------------------------------------
    def launcher(self, kind: str) -> mk_lib.StepLauncher:
        """Prebuilt steps on the current stream:
        "prefill": token in, K/V written, pos += 1, no lm_head;
        "decode":  token in, logits + greedy next token written back into the
                   token buffer, pos += 1 (autoregressive loop on device)."""
        if kind not in self._launchers:
            common = dict(pos=self.pos, tokens=self.tokens, flags=mk_lib.MK_FLAG_ADVANCE)
            if kind == "prefill":
                l = mk_lib.StepLauncher(self.weights, self.ws, self.k_caches, self.v_caches, **common)
            elif kind == "decode":
                l = mk_lib.StepLauncher(self.weights, self.ws, self.k_caches, self.v_caches, logits=self.logits,
                                        next_token=self.tokens, hidden_out=self.hidden_out, **common)
            elif kind == "decode_logits":   # logits only: the next token comes from mk_sample
                l = mk_lib.StepLauncher(self.weights, self.ws, self.k_caches, self.v_caches, logits=self.logits,
                                        hidden_out=self.hidden_out, **common)
            else:
                raise ValueError(kind)
            self._launchers[kind] = l
        return self._launchers[kind]

    def forward(self, input_ids: Optional[torch.Tensor] = None, position_ids: Optional[torch.Tensor] = None,
                past_key_values: Optional[Sequence[Tuple[torch.Tensor, torch.Tensor]]] = None,
                hidden_states: Optional[torch.Tensor] = None):
        """One token-generation step: (logits [B, V] fp32, past_key_values).

        ``input_ids`` [B] / [B, 1] int token ids, or ``hidden_states`` [B, 1, H]
        bf16 (the layer-0 input of the reference contract); ``position_ids`` [B]
        or [B, 1] — the row the fresh K/V is written to. ``past_key_values``
        defaults to the model's own caches; the returned caches are the same
        tensors, updated in place.
        """
        assert self._ready, "call load() first"
        kv = past_key_values if past_key_values is not None else self.past_key_values
        ks = [k for k, _ in kv]
        vs = [v for _, v in kv]
        dev = self.pos.device
        pos = position_ids.reshape(-1).to(device=dev, dtype=torch.int32)
        toks = None if input_ids is None else input_ids.reshape(-1).to(device=dev, dtype=torch.int32)
        hid = None if hidden_states is None else hidden_states.reshape(-1, self.config.dims.hidden).to(dev)
        mk_lib.decode_step(self.weights, self.ws, ks, vs, pos, tokens=toks, hidden_in=hid,
                           logits=self.logits, next_token=self.tokens)
        return self.logits, kv

    @torch.no_grad()
    def prefill(self, prompt: torch.Tensor, batched: bool = True) -> None:
        """Write the K/V rows of prompt tokens 0..n-2 (positions 0..n-2); leaves
        the last prompt token in the token buffer and pos = n - 1, so the next
        decode step processes it and yields the first generated token.

        batched: chunks of up to 32 tokens per launch of the batched kernel
        (MK_FLAG_PREFILL); otherwise one decode-kernel launch per token."""
        self.reset()
        n = int(prompt.numel())
        if n < 1 or n > self.s_max:
            raise ValueError(f"prompt of {n} tokens does not fit max_context_length {self.s_max}")
        prompt_dev = prompt.reshape(-1).to(device=self.pos.device, dtype=torch.int32)
        if batched:
            if self.pf_ws is None:
                self.pf_ws = mk_lib.Workspace(mk_lib.PREFILL_CHUNK, self.s_max, self.pos.device)
            for c0 in range(0, n - 1, mk_lib.PREFILL_CHUNK):
                m = min(mk_lib.PREFILL_CHUNK, n - 1 - c0)
                mk_lib.decode_step(self.weights, self.pf_ws, self.k_caches, self.v_caches, self.pf_pos[c0:c0 + m],
                                   tokens=prompt_dev[c0:c0 + m], flags=mk_lib.MK_FLAG_PREFILL, batch=m)
            self.pos.fill_(n - 1)
        else:
            pf = self.launcher("prefill")
            for i in range(n - 1):
                self.tokens.copy_(prompt_dev[i:i + 1])
                pf.launch()
        self.tokens.copy_(prompt_dev[n - 1:n])

    def prefill_device_error(self) -> int:
        """Device error bits of the prefill steps since the last call (0 = none)."""
        return 0 if self.pf_ws is None else self.pf_ws.read_device_error()

    @torch.no_grad()
    def decode_graph(self, n_steps: int, sampling_params: Optional[torch.Tensor] = None, seed: int = 0):
        """Capture ``n_steps`` consecutive decode steps (each followed by the
        on-device sampler if ``sampling_params`` is given) into one HIP graph.

        Every step reads its token and position from the device and writes
        them back (MK_FLAG_ADVANCE), so a replay continues from whatever state
        the model is in — e.g. right after ``prefill`` — exactly as the same
        launches issued one by one; the step's token is also appended to
        ``self.graph_tokens[:n_steps]``. The graph runs on a private stream;
        ``replay()`` orders it after the current stream's work."""
        if sampling_params is not None:
            sampling_params = sampling_params.to(device=self.pos.device, dtype=torch.float32).reshape(1, 3)
        stream = torch.cuda.Stream(device=self.pos.device)
        kw = dict(pos=self.pos, tokens=self.tokens, flags=mk_lib.MK_FLAG_ADVANCE, logits=self.logits,
                  hidden_out=self.hidden_out, stream=stream)
        if sampling_params is None:
            kw["next_token"] = self.tokens
        step = mk_lib.StepLauncher(self.weights, self.ws, self.k_caches, self.v_caches, **kw)
        self.graph_tokens = torch.zeros(n_steps, dtype=torch.int32, device=self.pos.device)
        graph = torch.cuda.CUDAGraph()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(n_steps):
                step.launch()
                if sampling_params is not None:
                    mk_lib.sample(self.logits, sampling_params, self.tokens, seed=seed, counter=self.pos)
                self.graph_tokens[i:i + 1].copy_(self.tokens)
        graph._mk_keep = (step, sampling_params, stream)
        return graph

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, return_logits: bool = False,
                 sampling_params: Optional[torch.Tensor] = None, seed: int = 0):
        """Generation for one sequence: returns the new token ids (and the
        per-step fp32 logits if requested). Greedy (the decode kernel's argmax)
        unless ``sampling_params`` [1, 3] (top_k, top_p, temperature) is given:
        then each step's logits go through the on-device sampler, whose Philox
        counter is the position of the token being produced (reproducible for
        a given seed)."""
        prompt = input_ids.reshape(-1)
        n = int(prompt.numel())
        if n + max_new_tokens - 1 > self.s_max:
            raise ValueError(f"{n} + {max_new_tokens} tokens exceed max_context_length {self.s_max}")
        self.prefill(prompt)
        dec = self.launcher("decode" if sampling_params is None else "decode_logits")
        if sampling_params is not None:
            sampling_params = sampling_params.to(device=self.pos.device, dtype=torch.float32).reshape(1, 3)
        out = torch.empty(max_new_tokens, dtype=torch.int32, device=self.pos.device)
        logits = [] if return_logits else None
        for t in range(max_new_tokens):
            dec.launch()
            if sampling_params is not None:
                mk_lib.sample(self.logits, sampling_params, self.tokens, seed=seed, counter=self.pos)
            out[t:t + 1].copy_(self.tokens)
            if return_logits:
                logits.append(self.logits.clone())
        torch.cuda.synchronize()
        bits = self.ws.read_device_error() | self.prefill_device_error()
        if bits:
            raise RuntimeError(f"megakernel device error bits 0x{bits:x}")
        if return_logits:
            return out.cpu(), torch.cat(logits).cpu()
        return out.cpu()


# Symbol main.py imports when --enable-nki is set (llama_with_megakernel.py:355).
NeuronLlamaForCausalLM = NeuronLlamaForCausalLMMK
