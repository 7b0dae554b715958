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
  ``do_sample=False`` / ``top_k=1`` path, main.py:57, 291, 332); at batch 1
  without requested logits every step runs in one launch (``decode_loop``,
  ``mk_decode_loop``).

``model_path`` is a local HF checkpoint directory (safetensors) or
``"random:<seed>"`` for the synthetic N(0, 0.02) weights used by the
benchmarks. Prefill (context encoding, the reference's baseline-layer path at
llama_with_megakernel.py:194-204) runs layer by layer on the matrix cores
(``mk_prefill``: per layer an RMSNorm, the QKV GEMM with RoPE writing the K/V
rows, causal attention, the O GEMM, an RMSNorm, the gate/up GEMM with SwiGLU
and the down GEMM, each layer's weights streamed once per chunk of prompt
tokens); ``prefill(..., method="chunks")`` runs the batched decode kernel over
up to 32 consecutive tokens per launch (``MK_FLAG_PREFILL``) and
``method="tokens"`` the decode megakernel once per prompt token.

TP must be 1, as the reference asserts (llama_with_megakernel.py:147-150).
"""

from __future__ import annotations

import dataclasses
import weakref
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


class NeuronLlamaDecoderLayerMK:
    """The layer seam (NeuronLlamaDecoderLayerMK, llama_with_megakernel.py:65-204).

    ``forward(hidden_states, attention_mask, position_ids, past_key_value,
    adapter_ids, rotary_position_ids, residual, **kwargs) -> (hidden, (K, V),
    cos, sin, residual)``:

    * token generation (``past_key_value`` given), layer 0: one launch of the
      megakernel runs all 16 layers (``transformer_llama_megakernel_16layers``)
      over the parent model's caches; the result and every layer's present
      (K, V) are stashed on the parent; cos / sin are the step's RoPE rows
      (bf16 [1, 1, 64] each);
    * token generation, layers 1..15: the stashed hidden state and this
      layer's own (K, V), so a caller that aliases each layer's cache back
      (NxDI in the reference) finds the same tensors;
    * context encoding (no ``past_key_value``): this layer alone over the
      prompt tokens, one single-layer step (``transformer_llama_megakernel_1layer``)
      per token in position order, each writing its K/V row before the next
      token attends to it. The reference runs its baseline layer here; the
      model-level ``NeuronLlamaForCausalLM.prefill`` is the fast path.

    Batch 1, TP=1 and the packed stack shapes are asserted as the reference
    asserts its own (llama_with_megakernel.py:145-162).
    """

    def __init__(self, config: "LlamaInferenceConfig", layer_idx: int):
        self.config = config
        self.layer_idx = layer_idx
        self._parent_model_ref = None        # set by the model's load()

    @property
    def _parent_model(self):
        return self._parent_model_ref() if self._parent_model_ref is not None else None

    def _check(self, parent) -> None:
        d, nc = self.config.dims, self.config.neuron_config
        assert nc.tp_degree == 1, f"megakernel is TP=1 only, got tp_degree={nc.tp_degree}"
        L, H = d.n_layers, d.hidden
        qkv = (d.n_q_heads + 2 * d.n_kv_heads) * d.head_dim
        shapes = {"w_qkv": (L, qkv, H), "w_o": (L, H, d.n_q_heads * d.head_dim),
                  "w_gu": (L, 2 * d.intermediate, H), "w_down": (L, H, d.intermediate)}
        for k, want in shapes.items():
            assert tuple(parent.packed[k].shape) == want, f"{k}.shape={tuple(parent.packed[k].shape)}, want {want}"
        assert parent.batch_size == 1, "the layer seam runs batch 1 (the reference's [1, 8, S, 64] caches)"

    def forward(self, hidden_states: torch.Tensor, attention_mask=None, position_ids=None, past_key_value=None,
                adapter_ids=None, rotary_position_ids=None, residual=None, **kwargs):
        parent = self._parent_model
        assert parent is not None, "layers need _parent_model_ref, set by NeuronLlamaForCausalLM.load()"
        import transformer_llama as tl
        p = parent.packed
        if past_key_value is not None and self.layer_idx == 0:
            self._check(parent)
            K, V = parent.k_caches, parent.v_caches
            pos = position_ids.reshape(-1)[:1].to(device=hidden_states.device, dtype=torch.int32)
            out = tl.transformer_llama_megakernel_16layers(
                hidden_states.to(torch.bfloat16), p["w_qkv"], p["w_o"], p["w_gu"], p["w_down"], *K, *V,
                p["rope"], pos)
            L = len(K)
            Y, present = out[0], [(out[1 + i], out[1 + L + i]) for i in range(L)]
            row = p["rope"][pos.long()].reshape(1, 1, -1)
            half = row.shape[-1] // 2
            parent._mk_outputs = {"hidden_states": Y, "present_kv": present}
            return Y, present[0], row[..., :half], row[..., half:], None
        if past_key_value is not None:
            st = parent._mk_outputs
            return st["hidden_states"], st["present_kv"][self.layer_idx], None, None, None
        # context encoding: this layer over the prompt, token by token
        self._check(parent)
        l = self.layer_idx
        X = hidden_states.reshape(-1, self.config.dims.hidden).to(torch.bfloat16)
        pos = position_ids.reshape(-1).to(device=X.device, dtype=torch.int32)
        if pos.numel() != X.shape[0]:
            raise ValueError(f"{pos.numel()} positions for {X.shape[0]} tokens")
        K, V = parent.k_caches[l], parent.v_caches[l]
        rows = [tl.transformer_llama_megakernel_1layer(X[t], p["w_qkv"], p["w_o"], p["w_gu"], p["w_down"], K, V,
                                                      p["rope"], pos[t:t + 1], layer=l)[0]
                for t in range(X.shape[0])]
        Y = torch.cat(rows, 1)                  # [1, n, H]
        return Y, (K, V), None, None, None

    __call__ = forward


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

    MANIFEST = "mk_compiled.json"

    def manifest(self) -> dict:
        """What a compiled model consists of in this build: the kernel library
        (compiled ahead of time) and the weights it packs at load."""
        import hashlib
        nc = self.neuron_config
        return {"abi_version": mk_lib.ABI_VERSION,
                "libmk_sha256": hashlib.sha256(mk_lib.LIB_PATH.read_bytes()).hexdigest(),
                "model_path": self.model_path, "dims": dataclasses.asdict(self.config.dims),
                "batch_size": nc.batch_size, "seq_len": nc.seq_len, "max_context_length": nc.max_context_length,
                "dtype": "bfloat16", "tp_degree": nc.tp_degree}

    def compile(self, compiled_model_path: Optional[str] = None, debug: bool = False) -> None:
        """Pack the weights onto the device. The reference traces and compiles
        a NEFF into ``compiled_model_path`` here (main.py:143); this build's
        kernel is compiled ahead of time into libmk.so, so the directory, when
        given, receives a manifest (library hash, ABI version, weights source,
        shapes) that ``load`` checks."""
        mk_lib.load()   # fails loudly if the native library is missing
        sd = self.load_state_dict_source()
        self.state_dict_bf16 = sd
        self.packed = self.convert_hf_to_neuron_state_dict(sd, self.config, device=self.neuron_config.device)
        if compiled_model_path:
            import json
            from pathlib import Path
            out = Path(compiled_model_path)
            out.mkdir(parents=True, exist_ok=True)
            (out / self.MANIFEST).write_text(json.dumps(self.manifest(), indent=1, sort_keys=True))

    def check_manifest(self, compiled_model_path: str) -> None:
        import json
        from pathlib import Path
        f = Path(compiled_model_path) / self.MANIFEST
        if not f.exists():
            raise FileNotFoundError(f"{f} is missing: call compile({compiled_model_path!r}) first")
        got, want = json.loads(f.read_text()), self.manifest()
        diff = sorted(k for k in want if got.get(k) != want[k])
        if diff:
            raise ValueError(f"{f} was compiled for another model or library (differs in {diff}): compile again")

    def load(self, compiled_model_path: Optional[str] = None) -> None:
        """Allocate the caches and workspaces (main.py:150). With a
        ``compiled_model_path`` its manifest must describe this model and
        library; a missing or stale one is an error, as loading a NEFF traced
        for other shapes would be."""
        if compiled_model_path:
            self.check_manifest(compiled_model_path)
        if self.packed is None:
            self.compile(compiled_model_path)
        nc, d = self.neuron_config, self.config.dims
        B = nc.batch_size
        if not 1 <= B <= mk_lib.PREFILL_CHUNK:
            raise ValueError(f"batch_size {B} not in [1, {mk_lib.PREFILL_CHUNK}]")
        dev = torch.device(nc.device)
        self.batch_size = B
        self.s_max = nc.max_context_length
        # past_key_values: one [B, 8, S, 64] K and V tensor per layer, views of one allocation;
        # sequence b's rows of layer l are kv[l, :, b] (its own slice: no padding between sequences)
        self.kv = torch.zeros(d.n_layers, 2, B, d.n_kv_heads, self.s_max, d.head_dim,
                              dtype=torch.bfloat16, device=dev)
        self.k_caches = [self.kv[l, 0] for l in range(d.n_layers)]
        self.v_caches = [self.kv[l, 1] for l in range(d.n_layers)]
        self.weights = mk_lib.weights_struct(self.packed)
        # batch 1 runs the GEMV kernel; batches of 2..32 the MFMA kernel
        self.ws = mk_lib.Workspace(B, self.s_max, dev)
        self.pos = torch.zeros(B, dtype=torch.int32, device=dev)
        self.tokens = torch.zeros(B, dtype=torch.int32, device=dev)
        self.logits = torch.zeros(B, d.vocab, dtype=torch.float32, device=dev)
        self.hidden_out = torch.zeros(B, d.hidden, dtype=torch.bfloat16, device=dev)
        self.pf_ws: Optional[mk_lib.Workspace] = None   # batched workspace of the 32-token prefill steps (on first use)
        self.pf_layers_ws: Optional[torch.Tensor] = None  # mk_prefill's workspace (on first use)
        self.ws1: Optional[mk_lib.Workspace] = None     # batch-1 workspace of token-by-token prefill (B > 1)
        self.pf_pos = torch.arange(self.s_max, dtype=torch.int32, device=dev)
        self._ready = True
        self._launchers: Dict[str, mk_lib.StepLauncher] = {}
        # the layer seam (NeuronLlamaModelMK.init_model installs the same parent weakrefs,
        # llama_with_megakernel.py:210-250)
        self.layers = [NeuronLlamaDecoderLayerMK(self.config, i) for i in range(d.n_layers)]
        for layer in self.layers:
            layer._parent_model_ref = weakref.ref(self)
        self._mk_outputs: Optional[dict] = None

    def reset(self) -> None:
        """Start new sequences (rows >= pos are never read, so no cache clear)."""
        self.pos.zero_()

    @property
    def past_key_values(self) -> List[Tuple[torch.Tensor, torch.Tensor]]:
        return list(zip(self.k_caches, self.v_caches))

    def seq_caches(self, b: int) -> Tuple[List[torch.Tensor], List[torch.Tensor]]:
        """Per-layer K and V caches of sequence b alone ([1, 8, S, 64] views)."""
        return ([self.kv[l, 0, b:b + 1] for l in range(self.kv.shape[0])],
                [self.kv[l, 1, b:b + 1] for l in range(self.kv.shape[0])])

    # -- steps ---------------------------------------------------------------
    def launcher(self, kind: str) -> mk_lib.StepLauncher:
        """Prebuilt steps over the whole batch on the current stream:
        "prefill": token in, K/V written, pos += 1, no lm_head;
        "decode":  token in, logits + greedy next token written back into the
                   token buffer, pos += 1 (autoregressive loop on device);
        "decode_logits": logits only (the next token comes from mk_sample)."""
        if kind not in self._launchers:
            common = dict(pos=self.pos, tokens=self.tokens, flags=mk_lib.MK_FLAG_ADVANCE, batch=self.batch_size)
            if kind == "prefill":
                l = mk_lib.StepLauncher(self.weights, self.ws, self.k_caches, self.v_caches, **common)
            elif kind == "decode":
                l = mk_lib.StepLauncher(self.weights, self.ws, self.k_caches, self.v_caches, logits=self.logits,
                                        next_token=self.tokens, hidden_out=self.hidden_out, **common)
            elif kind == "decode_logits":
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
        or [B, 1] — the row each sequence's fresh K/V is written to (sequences
        may sit at different positions). ``past_key_values`` defaults to the
        model's own caches ([B, 8, S, 64] per layer); the returned caches are
        the same tensors, updated in place. B may be smaller than the loaded
        batch size: the first B sequences of the caches step.
        """
        assert self._ready, "call load() first"
        kv = past_key_values if past_key_values is not None else self.past_key_values
        ks = [k for k, _ in kv]
        vs = [v for _, v in kv]
        dev = self.pos.device
        pos = position_ids.reshape(-1).to(device=dev, dtype=torch.int32)
        toks = None if input_ids is None else input_ids.reshape(-1).to(device=dev, dtype=torch.int32)
        hid = None if hidden_states is None else hidden_states.reshape(-1, self.config.dims.hidden).to(dev)
        nb = int(pos.numel())
        if not 1 <= nb <= self.batch_size:
            raise ValueError(f"{nb} positions for a model loaded with batch_size {self.batch_size}")
        mk_lib.decode_step(self.weights, self.ws, ks, vs, pos, tokens=toks, hidden_in=hid,
                           logits=self.logits[:nb], next_token=self.tokens[:nb], batch=nb)
        return self.logits[:nb], kv

    @torch.no_grad()
    def layer_stack_forward(self, hidden_states: torch.Tensor, position_ids: torch.Tensor,
                            past_key_values: Optional[Sequence[Tuple[torch.Tensor, torch.Tensor]]] = None):
        """The decoder-layer loop of NxDI's model forward over the layer seam:
        each layer called with (hidden, position_ids, its past_key_value), the
        returned hidden state fed to the next. Token generation passes the
        caches (the megakernel runs in layer 0); context encoding passes
        ``past_key_values=None`` with the prompt's hidden states [1, n, H] and
        positions [1, n]. Returns the hidden state after the last layer (before
        the final norm) and the per-layer present (K, V)."""
        assert self._ready, "call load() first"
        h, present = hidden_states, []
        for i, layer in enumerate(self.layers):
            kv = None if past_key_values is None else past_key_values[i]
            h, kv_out, _, _, _ = layer(h, position_ids=position_ids, past_key_value=kv)
            present.append(kv_out)
        return h, present

    def _prompts(self, input_ids) -> List[torch.Tensor]:
        """The batch's prompts as 1-D tensors: [n] (batch 1), [B, n], or a list
        of B 1-D tensors of their own lengths (no padding: every sequence has
        its own cache slice and position)."""
        if isinstance(input_ids, torch.Tensor):
            ps = [input_ids.reshape(-1)] if input_ids.dim() <= 1 else list(input_ids)
        else:
            ps = [torch.as_tensor(p).reshape(-1) for p in input_ids]
        if len(ps) != self.batch_size:
            raise ValueError(f"{len(ps)} prompts for a model loaded with batch_size {self.batch_size}")
        for p in ps:
            if not 1 <= int(p.numel()) <= self.s_max:
                raise ValueError(f"prompt of {int(p.numel())} tokens does not fit max_context_length {self.s_max}")
        return ps

    PREFILL_METHODS = ("layers", "chunks", "tokens")

    @torch.no_grad()
    def prefill(self, prompt, method: str = "layers", batched: Optional[bool] = None) -> None:
        """For each sequence b, write the K/V rows of its prompt tokens 0..n_b-2
        into its own cache slice; leaves its last prompt token in the token
        buffer and pos[b] = n_b - 1, so the next decode step processes it and
        yields the first generated token.

        method "layers" (default): ``mk_prefill``, layer by layer on the matrix
        cores, each layer's weights streamed once per chunk of up to 4096
        tokens; "chunks": launches of the batched decode kernel over up to 32
        consecutive tokens (MK_FLAG_PREFILL); "tokens": one decode-kernel launch
        per token. ``batched`` (earlier interface): True = "chunks", False =
        "tokens"."""
        if batched is not None:
            method = "chunks" if batched else "tokens"
        if method not in self.PREFILL_METHODS:
            raise ValueError(f"prefill method {method!r} not in {self.PREFILL_METHODS}")
        prompts = self._prompts(prompt)
        self.reset()
        dev = self.pos.device
        last = []
        for b, p in enumerate(prompts):
            n = int(p.numel())
            prompt_dev = p.to(device=dev, dtype=torch.int32)
            kc, vc = self.seq_caches(b)
            if method == "layers":
                if n > 1:
                    if self.pf_layers_ws is None:
                        self.pf_layers_ws = mk_lib.prefill_workspace(min(self.s_max, 4096), dev)
                    mk_lib.prefill(self.weights, prompt_dev[:n - 1], kc, vc, 0, self.pf_layers_ws)
            elif method == "chunks":
                if self.pf_ws is None:
                    self.pf_ws = mk_lib.Workspace(mk_lib.PREFILL_CHUNK, self.s_max, dev)
                for c0 in range(0, n - 1, mk_lib.PREFILL_CHUNK):
                    m = min(mk_lib.PREFILL_CHUNK, n - 1 - c0)
                    mk_lib.decode_step(self.weights, self.pf_ws, kc, vc, self.pf_pos[c0:c0 + m],
                                       tokens=prompt_dev[c0:c0 + m], flags=mk_lib.MK_FLAG_PREFILL, batch=m)
            elif self.batch_size == 1:   # "tokens"
                pf = self.launcher("prefill")
                for i in range(n - 1):
                    self.tokens.copy_(prompt_dev[i:i + 1])
                    pf.launch()
            else:
                if self.ws1 is None:
                    self.ws1 = mk_lib.Workspace(1, self.s_max, dev)
                pos1 = torch.zeros(1, dtype=torch.int32, device=dev)
                tok1 = torch.zeros(1, dtype=torch.int32, device=dev)
                pf = mk_lib.StepLauncher(self.weights, self.ws1, kc, vc, pos1, tokens=tok1,
                                         flags=mk_lib.MK_FLAG_ADVANCE)
                for i in range(n - 1):
                    tok1.copy_(prompt_dev[i:i + 1])
                    pf.launch()
            last.append(prompt_dev[n - 1:n])
        self.pos.copy_(torch.tensor([int(p.numel()) - 1 for p in prompts], dtype=torch.int32))
        self.tokens.copy_(torch.cat(last))

    def prefill_device_error(self) -> int:
        """Device error bits of the prefill steps since the last call (0 = none)."""
        bits = 0
        for ws in (self.pf_ws, self.ws1):
            if ws is not None:
                bits |= ws.read_device_error()
        return bits

    def _sampling_rows(self, sampling_params: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
        if sampling_params is None:
            return None
        sp = sampling_params.to(device=self.pos.device, dtype=torch.float32).reshape(-1, 3)
        if sp.shape[0] == 1 and self.batch_size > 1:
            sp = sp.expand(self.batch_size, 3)
        if sp.shape[0] != self.batch_size:
            raise ValueError(f"sampling parameters for {sp.shape[0]} rows, batch {self.batch_size}")
        return sp.contiguous()

    @torch.no_grad()
    def decode_graph(self, n_steps: int, sampling_params: Optional[torch.Tensor] = None, seed: int = 0):
        """Capture ``n_steps`` consecutive decode steps of the whole batch (each
        followed by the on-device sampler if ``sampling_params`` is given) into
        one HIP graph.

        Every step reads its tokens and positions from the device and writes
        them back (MK_FLAG_ADVANCE), so a replay continues from whatever state
        the model is in — e.g. right after ``prefill`` — exactly as the same
        launches issued one by one; step i's tokens are also written to
        ``self.graph_tokens[i]``. The graph runs on a private stream;
        ``replay()`` orders it after the current stream's work."""
        sampling_params = self._sampling_rows(sampling_params)
        stream = torch.cuda.Stream(device=self.pos.device)
        kw = dict(pos=self.pos, tokens=self.tokens, flags=mk_lib.MK_FLAG_ADVANCE, logits=self.logits,
                  hidden_out=self.hidden_out, stream=stream, batch=self.batch_size)
        if sampling_params is None:
            kw["next_token"] = self.tokens
        step = mk_lib.StepLauncher(self.weights, self.ws, self.k_caches, self.v_caches, **kw)
        self.graph_tokens = torch.zeros(n_steps, self.batch_size, dtype=torch.int32, device=self.pos.device)
        graph = torch.cuda.CUDAGraph()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(n_steps):
                step.launch()
                if sampling_params is not None:
                    mk_lib.sample(self.logits, sampling_params, self.tokens, seed=seed, counter=self.pos)
                self.graph_tokens[i].copy_(self.tokens)
        graph._mk_keep = (step, sampling_params, stream)
        self.ws.register_graph(graph)            # the workspace is not released while the graph lives
        return graph

    @torch.no_grad()
    def decode_loop(self, n_steps: int, step_clock: Optional[torch.Tensor] = None,
                    tokens_out: Optional[torch.Tensor] = None, check: bool = True) -> torch.Tensor:
        """``n_steps`` greedy decode steps of a batch-1 model in ONE launch of the
        persistent kernel (``mk_decode_loop``): each step feeds its argmax to
        the next on the device, continuing from the model's current token and
        position exactly as ``n_steps`` launches of ``launcher("decode")``
        would (same tokens, caches, pos, and the last step's logits). Returns the
        generated token ids (int32 [n_steps], on the device; ``tokens_out`` if
        given); ``step_clock`` (int64 [n_steps + 1]) receives the device wall
        clock at each step boundary (``mk_wall_clock_hz`` ticks per second).
        ``check`` reads the position back to refuse a range past the cache on
        the host (a synchronisation); without it the device refuses such a
        range (``MK_DEVERR_POS``, nothing written)."""
        if self.batch_size != 1:
            raise ValueError(f"the decode loop runs batch 1 (model batch {self.batch_size})")
        if check:
            p = int(self.pos[0])
            if p + n_steps > self.s_max:
                raise ValueError(f"{n_steps} steps from position {p} exceed max_context_length {self.s_max}")
        out = tokens_out if tokens_out is not None else torch.empty(n_steps, dtype=torch.int32,
                                                                     device=self.pos.device)
        dec = self.launcher("decode")   # the same arguments, prebuilt
        if torch.cuda.current_stream(self.pos.device).cuda_stream == dec.stream_ptr:
            dec.loop(n_steps, tokens_out=out, step_clock=step_clock)
        else:
            mk_lib.decode_loop(self.weights, self.ws, self.k_caches, self.v_caches, self.pos, self.tokens, n_steps,
                               tokens_out=out, step_clock=step_clock, logits=self.logits, next_token=self.tokens,
                               hidden_out=self.hidden_out, flags=mk_lib.MK_FLAG_ADVANCE)
        return out

    @torch.no_grad()
    def generate(self, input_ids, max_new_tokens: int, return_logits: bool = False,
                 sampling_params: Optional[torch.Tensor] = None, seed: int = 0):
        """Generation for the batch's sequences (prompts as in ``prefill``):
        returns the new token ids, [max_new_tokens] for a 1-D prompt of a
        batch-1 model, else [B, max_new_tokens] (and the per-step fp32 logits,
        [steps, V] or [B, steps, V], if requested). Greedy (the kernel's argmax)
        unless ``sampling_params`` ([1, 3] or [B, 3]: top_k, top_p,
        temperature) is given: then each step's logits go through the
        on-device sampler, whose Philox counter is the position of the token
        being produced (reproducible for a given seed)."""
        prompts = self._prompts(input_ids)
        for p in prompts:
            if int(p.numel()) + max_new_tokens - 1 > self.s_max:
                raise ValueError(f"{int(p.numel())} + {max_new_tokens} tokens exceed max_context_length {self.s_max}")
        self.prefill(prompts)
        sampling_params = self._sampling_rows(sampling_params)
        B = self.batch_size
        logits = [] if return_logits else None
        if B == 1 and sampling_params is None and not return_logits:
            # greedy batch 1 with nothing to read between steps: one launch
            out = self.decode_loop(max_new_tokens).view(max_new_tokens, 1)
        else:
            dec = self.launcher("decode" if sampling_params is None else "decode_logits")
            out = torch.empty(max_new_tokens, B, dtype=torch.int32, device=self.pos.device)
            for t in range(max_new_tokens):
                dec.launch()
                if sampling_params is not None:
                    mk_lib.sample(self.logits, sampling_params, self.tokens, seed=seed, counter=self.pos)
                out[t].copy_(self.tokens)
                if return_logits:
                    logits.append(self.logits.clone())
        torch.cuda.synchronize()
        bits = self.ws.read_device_error() | self.prefill_device_error()
        if bits:
            raise RuntimeError(f"megakernel device error bits 0x{bits:x}")
        flat = B == 1 and isinstance(input_ids, torch.Tensor) and input_ids.dim() <= 1
        toks = out.t().cpu()
        if flat:
            toks = toks[0]
        if not return_logits:
            return toks
        lg = torch.stack(logits, 1).cpu()      # [B, steps, V]
        return toks, (lg[0] if flat else lg)


# Symbol main.py imports when --enable-nki is set (llama_with_megakernel.py:355).
NeuronLlamaForCausalLM = NeuronLlamaForCausalLMMK
