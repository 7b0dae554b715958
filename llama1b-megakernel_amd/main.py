"""Driver with the reference's CLI (main.py:34-105, 538-669) for this build.

  python main.py --mode generate [--enable-nki] [--prompt TEXT ... | --prompt-ids 1,2,3 ... | --prompt-len 384]
                 [--max-new-tokens N] [--model-path random:0 | /path/to/hf_checkpoint] [--tokenizer-path DIR]
  python main.py --mode validate --enable-nki [...]
  python main.py --mode benchmark --enable-nki [...]

Prompts. As in the reference (main.py:56, 538-540) every ``--prompt`` is one
sequence of the batch and the batch size is their number. Text prompts are
encoded with the checkpoint's own tokenizer, read from a local directory only
(``--tokenizer-path``, default ``--model-path``; the reference's
load_tokenizer, main.py:114-118, with the pad token set to EOS). The
reference pads a batch of prompts to one length (main.py:217, 277); here each
sequence has its own cache slice and position, so prompts keep their own
lengths and need no padding or attention mask (the same positions and causal
attention a left-padded, masked sequence sees). ``--prompt-ids`` gives a
prompt as token ids instead (repeatable); with no prompt at all,
``--batch-size`` random prompts of ``--prompt-len`` ids are drawn (seeds 0..).

* generate: generation with the megakernel model (the reference's
  run_generation, main.py:360-375), greedy unless --top-k/--top-p/--temperature
  ask for on-device sampling; with a tokenizer the outputs are decoded.
* validate: the megakernel model against the stock PyTorch path
  (llama_baseline.StockLlama, fp32) on the same weights and token ids, with
  teacher forcing after a divergence as in check_accuracy_logits
  (main.py:274-357): per-step logit error and greedy agreement; the criteria
  are those of tests/test_gpu_decode.py (bf16 noise floor, see there). The
  reference's tol_map and divergence tolerance (main.py:51, 544) are reported
  as restated checks (mk_validate).
* benchmark: e2e / context-encoding / token-generation latency percentiles and
  throughput in the shape of NxDI's benchmark report (main.py:178-271),
  written to benchmark_report.json.

``--enable-nki`` selects the megakernel model (llama_with_megakernel), as in
the reference (main.py:546-553); without it generate runs the stock path.
``--tp-degree`` must be 1 (llama_with_megakernel.py:147-150).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path
from typing import List, Optional

import torch

sys.path.insert(0, str(Path(__file__).resolve().parent))

BENCHMARK_REPORT_FILENAME = "benchmark_report.json"


def _torch_dtype(name: str) -> torch.dtype:
    """The reference parses --torch-dtype / --rpl-reduce-dtype with NxDI's
    to_torch_dtype (main.py:66, 75): a dtype name such as "bfloat16"."""
    key = str(name).lower().replace("torch.", "")
    table = {"bfloat16": torch.bfloat16, "bf16": torch.bfloat16, "float16": torch.float16, "fp16": torch.float16,
             "half": torch.float16, "float32": torch.float32, "fp32": torch.float32, "float": torch.float32,
             "float64": torch.float64, "double": torch.float64}
    if key not in table:
        raise argparse.ArgumentTypeError(f"unknown torch dtype {name!r}")
    return table[key]


def _flag_bool(v) -> bool:
    """--do-sample / --enable-bucketing take a value as in the reference
    (main.py:62, 89). The reference's ``type=bool`` reads any non-empty string,
    "False" included, as True; here "0", "false" and "no" read as False."""
    return str(v).lower() in ("1", "true", "yes", "y", "on")


def parse_args(argv=None):
    """Every flag of the reference's parser (main.py:34-105), plus this build's
    own (benchmark mode, --prompt-ids, --prompt-len, --tokenizer-path, --seed,
    --graph, --num-runs, --report-path). Flags for Neuron features this build
    has no counterpart for are accepted; a value this build cannot honour is
    refused by check_args with a message naming the flag."""
    ap = argparse.ArgumentParser()
    # ASPLOS contest specific (main.py:37-41)
    ap.add_argument("--mode", choices=["generate", "validate", "benchmark", "evaluate_single", "evaluate_all"],
                    required=True)
    ap.add_argument("--llama", type=str, default="llama",
                    help="model module: llama (the stock path, or the megakernel with --enable-nki) "
                         "or llama_with_megakernel")
    ap.add_argument("--enable-nki", action="store_true", help="run the megakernel model (llama_with_megakernel)")
    ap.add_argument("--base-latency", type=float, default=526.15, help="contest scoring only (evaluate_*)")
    ap.add_argument("--base-throughput", type=float, default=134.61, help="contest scoring only (evaluate_*)")
    # Model path (main.py:44-47)
    ap.add_argument("--model-path", default="random:0",
                    help="local HF checkpoint directory (safetensors) or random:<seed>")
    ap.add_argument("--compiled-model-path", default=None,
                    help="directory for the compiled-model manifest and the tokenizer (the reference writes its "
                         "traced NEFF there)")
    # Evaluation (main.py:49-53)
    ap.add_argument("--benchmark", action="store_true", help="accepted (a NeuronConfig field; no effect in main.py)")
    ap.add_argument("--divergence-difference-tol", type=float, default=None,
                    help="validate: logit gap under which a greedy divergence is a tie (default 0.001)")
    ap.add_argument("--tol-map", type=str, default=None,
                    help="validate: {top_k: (atol, rtol)} as a Python literal (default: the reference's, main.py:544)")
    ap.add_argument("--num-tokens-to-check", type=int, default=None)
    # Generation (main.py:55-63)
    ap.add_argument("--prompt", dest="prompts", action="append", default=None, help="text prompt (repeatable)")
    ap.add_argument("--prompt-ids", action="append", default=None,
                    help="comma-separated token ids of one prompt (repeatable)")
    ap.add_argument("--prompt-len", type=int, default=384, help="random prompt length (seed 0) if no prompt")
    ap.add_argument("--tokenizer-path", default=None,
                    help="local tokenizer directory (default: --model-path when it is a directory)")
    ap.add_argument("--top-k", type=int, default=1)
    ap.add_argument("--top-p", type=float, default=1.0)
    ap.add_argument("--temperature", type=float, default=1.0)
    ap.add_argument("--global-topk", type=int, default=None,
                    help="candidate cap of the on-device sampler (at most 1024, the built-in cap)")
    ap.add_argument("--do-sample", type=_flag_bool, default=True)
    ap.add_argument("--dynamic", action="store_true", help="accepted (a generation-config field; no effect here)")
    ap.add_argument("--pad-token-id", type=int, default=2,
                    help="accepted: prompts are not padded here (each sequence keeps its own length)")
    ap.add_argument("--seed", type=int, default=0, help="Philox key of the on-device sampler")
    # Basic config (main.py:65-77)
    ap.add_argument("--torch-dtype", type=_torch_dtype, default=torch.bfloat16)
    ap.add_argument("--batch-size", type=int, default=1, help="random prompts drawn when no prompt is given")
    ap.add_argument("--padding-side", type=str, default=None, choices=[None, "left", "right"],
                    help="tokenizer padding side (prompts are not padded here)")
    ap.add_argument("--seq-len", type=int, default=1024,
                    help="cache rows per sequence = max_length (the reference's default 64 fails its own "
                         "megakernel's asserts, llama_with_megakernel.py:159-162)")
    ap.add_argument("--n-active-tokens", type=int, default=None, help="accepted (NxDI tracing shape)")
    ap.add_argument("--n-positions", type=int, default=None, help="positions of the model; must be >= --seq-len")
    ap.add_argument("--max-context-length", type=int, default=None)
    ap.add_argument("--max-new-tokens", type=int, default=None,
                    help="default: up to --seq-len (seq_len minus the longest prompt, as the reference's max_length)")
    ap.add_argument("--max-length", type=int, default=None,
                    help="accepted; set to --seq-len as the reference does (main.py:543)")
    ap.add_argument("--rpl-reduce-dtype", type=_torch_dtype, default=None,
                    help="accepted: the TP all-reduce dtype; TP=1 has no all-reduce")
    ap.add_argument("--output-logits", action="store_true",
                    help="generate: also return the per-step logits and print their summary")
    ap.add_argument("--vocab-parallel", action="store_true", help="accepted: no vocabulary split at TP=1")
    # Attention (main.py:79-82)
    ap.add_argument("--fused-qkv", action="store_true", help="accepted: Q, K and V are always one fused GEMV")
    ap.add_argument("--sequence-parallel-enabled", action="store_true", help="accepted: no sequence split at TP=1")
    ap.add_argument("--flash-decoding-enabled", action="store_true",
                    help="accepted: decode attention is always split over the KV length")
    # On device sampling (main.py:84-85)
    ap.add_argument("--on-device-sampling", action="store_true",
                    help="accepted for the reference's CLI; sampling always runs on the GPU here")
    # Bucketing (main.py:87-91)
    ap.add_argument("--enable-bucketing", type=_flag_bool, default=True,
                    help="accepted: no traced buckets (every length runs the same kernel)")
    ap.add_argument("--bucket-n-active-tokens", action="store_true", help="accepted (no traced buckets)")
    ap.add_argument("--context-encoding-buckets", nargs="+", type=int, default=None,
                    help="accepted; each bucket must fit --seq-len")
    ap.add_argument("--token-generation-buckets", nargs="+", type=int, default=None,
                    help="accepted; each bucket must fit --seq-len")
    # Parallelism (main.py:93-94)
    ap.add_argument("--tp-degree", type=int, default=1,
                    help="must be 1 (llama_with_megakernel.py:147-150; the reference's default 2 fails there)")
    # Kernels (main.py:96-103)
    ap.add_argument("--qkv-kernel-enabled", action="store_true", help="accepted: the megakernel fuses QKV")
    ap.add_argument("--attn-kernel-enabled", action="store_true", help="accepted: the megakernel fuses attention")
    ap.add_argument("--mlp-kernel-enabled", action="store_true", help="accepted: the megakernel fuses the MLP")
    ap.add_argument("--quantized-mlp-kernel-enabled", action="store_true",
                    help="refused: this build computes in bf16 only")
    ap.add_argument("--rmsnorm-quantize-kernel-enabled", action="store_true",
                    help="refused: this build computes in bf16 only")
    ap.add_argument("--quantized-kernel-lower-bound", type=float, default=1200.0,
                    help="accepted (used only with the quantized MLP kernel)")
    ap.add_argument("--mlp-kernel-fuse-residual-add", action="store_true",
                    help="accepted: the residual add is always fused")
    # this build's benchmark mode
    ap.add_argument("--graph", action="store_true", help="benchmark: replay the decode steps as one HIP graph")
    ap.add_argument("--decode-loop", action="store_true",
                    help="benchmark: greedy batch-1 token generation as one mk_decode_loop launch (per-step latencies "
                         "from the device clock at the step boundaries)")
    ap.add_argument("--num-runs", type=int, default=5)
    ap.add_argument("--report-path", default=BENCHMARK_REPORT_FILENAME)
    args = ap.parse_args(argv)
    check_args(args)
    return args


MODULES = ("llama", "llama_with_megakernel")


def check_args(args) -> None:
    """Refuse values this build cannot honour, with the flag named (the
    reference's own asserts, llama_with_megakernel.py:145-162, plus this
    build's bf16-only kernels)."""
    if args.mode in ("evaluate_single", "evaluate_all"):
        raise SystemExit(f"--mode {args.mode} scores the reference's ASPLOS contest (trn1 baselines, the NKI "
                         "share of the traced HLO, prompts.txt with a real checkpoint; main.py:586-669): out of "
                         "scope for this build. Use --mode validate for accuracy and --mode benchmark for latency.")
    if args.llama not in MODULES:
        raise SystemExit(f"--llama {args.llama!r}: this build has the modules {', '.join(MODULES)}")
    if args.llama == "llama_with_megakernel":
        args.enable_nki = True
    if args.torch_dtype != torch.bfloat16:
        raise SystemExit(f"--torch-dtype {args.torch_dtype}: the megakernel computes in bfloat16 only")
    if args.quantized_mlp_kernel_enabled or args.rmsnorm_quantize_kernel_enabled:
        raise SystemExit("--quantized-mlp-kernel-enabled / --rmsnorm-quantize-kernel-enabled: "
                         "this build computes in bfloat16 only (no quantized kernels)")
    if args.tp_degree != 1:
        raise SystemExit(f"--tp-degree {args.tp_degree}: the megakernel is TP=1 only "
                         "(llama_with_megakernel.py:147-150)")
    if args.n_positions is not None and args.n_positions < args.seq_len:
        raise SystemExit(f"--n-positions {args.n_positions} < --seq-len {args.seq_len}")
    for name in ("context_encoding_buckets", "token_generation_buckets"):
        for b in getattr(args, name) or []:
            if not 1 <= b <= args.seq_len:
                raise SystemExit(f"--{name.replace('_', '-')} {b}: buckets must lie in [1, --seq-len]")
    if args.max_new_tokens is not None and args.max_new_tokens < 1:
        raise SystemExit("--max-new-tokens must be >= 1")
    if args.divergence_difference_tol is not None and args.divergence_difference_tol < 0:
        raise SystemExit("--divergence-difference-tol must be >= 0")
    args.max_length = args.seq_len             # main.py:543
    from mk_validate import parse_tol_map
    try:
        args.tol_map_parsed = parse_tol_map(args.tol_map)
    except ValueError as e:
        raise SystemExit(f"--tol-map: {e}")


def max_new_tokens(args, prompts) -> int:
    """--max-new-tokens, or what fills --seq-len after the longest prompt (the
    reference generates up to max_length = seq_len, main.py:543)."""
    if args.max_new_tokens is not None:
        return args.max_new_tokens
    n = args.seq_len - max(int(p.numel()) for p in prompts) + 1
    if n < 1:
        raise SystemExit(f"a prompt of {max(int(p.numel()) for p in prompts)} tokens fills --seq-len {args.seq_len}")
    return n


def tokenizer_dir(args) -> Optional[str]:
    if args.tokenizer_path:
        return args.tokenizer_path
    if not args.model_path.startswith("random:") and os.path.isdir(args.model_path):
        return args.model_path
    return None


def load_tokenizer(path: str, padding_side: Optional[str] = None, compiled_model_path: Optional[str] = None):
    """The checkpoint's tokenizer from a local directory (main.py:114-118):
    no network, pad token = EOS, a copy saved into the compiled-model
    directory when one is given (as the reference does)."""
    from transformers import AutoTokenizer
    kw = {"padding_side": padding_side} if padding_side else {}
    tok = AutoTokenizer.from_pretrained(path, local_files_only=True, **kw)
    if tok.pad_token is None:
        tok.pad_token = tok.eos_token
    if compiled_model_path:
        tok.save_pretrained(compiled_model_path)
    return tok


def args_tokenizer(args):
    """The tokenizer main.py's modes use, or None (random weights, no
    tokenizer directory)."""
    d = tokenizer_dir(args)
    return load_tokenizer(d, args.padding_side, args.compiled_model_path) if d else None


REFERENCE_DEFAULT_PROMPT = "I believe the meaning of life is"     # main.py:538-539


def encode_prompts(args, tokenizer=None) -> List[torch.Tensor]:
    """The batch's prompts as 1-D int64 token-id tensors (see the module doc)."""
    prompts: List[torch.Tensor] = []
    if args.prompts:
        if tokenizer is None:
            d = tokenizer_dir(args)
            if d is None:
                raise SystemExit("--prompt needs a tokenizer: give --tokenizer-path (a local directory)")
            tokenizer = load_tokenizer(d, args.padding_side)
        for text in args.prompts:
            ids = tokenizer(text)["input_ids"]
            if not ids:
                raise SystemExit(f"prompt {text!r} encodes to no tokens")
            prompts.append(torch.tensor(ids, dtype=torch.int64))
    for s in args.prompt_ids or []:
        prompts.append(torch.tensor([int(x) for x in s.split(",")], dtype=torch.int64))
    if not prompts and tokenizer is not None:
        ids = tokenizer(REFERENCE_DEFAULT_PROMPT)["input_ids"]
        prompts = [torch.tensor(ids, dtype=torch.int64)]
    if not prompts:
        from mk_weights import random_token_ids
        prompts = [random_token_ids(args.prompt_len, seed=b) for b in range(args.batch_size)]
    return prompts


def sampling_params(args, batch: int = 1):
    """[B, 3] device tensor (top_k, top_p, temperature), or None for greedy
    (top_k == 1 or do_sample false), as the reference's generation config."""
    import mk_lib
    if not args.do_sample or args.top_k == 1:
        return None
    if args.global_topk is not None and not 1 <= args.global_topk <= mk_lib.SAMPLE_MAX_TOPK:
        raise SystemExit(f"--global-topk must be in [1, {mk_lib.SAMPLE_MAX_TOPK}]")
    k = args.top_k
    if args.global_topk is not None and (k <= 0 or k > args.global_topk):
        k = args.global_topk
    return mk_lib.prepare_sampling_params(batch, k, args.top_p, args.temperature)


def prepare_inference(args, batch: int):
    """Model construction, compile (weight packing) and load, timed as the
    reference's prepare_inference does (main.py:121-175); batch_size is the
    number of prompts (main.py:538-540)."""
    from llama_with_megakernel import LlamaInferenceConfig, NeuronConfigLlamaMK, NeuronLlamaForCausalLM
    nc = NeuronConfigLlamaMK(batch_size=batch, seq_len=args.seq_len,
                             max_context_length=args.max_context_length or args.seq_len,
                             tp_degree=args.tp_degree)
    model = NeuronLlamaForCausalLM(args.model_path, LlamaInferenceConfig(nc))
    t0 = time.monotonic()
    model.compile(args.compiled_model_path)
    model.load(args.compiled_model_path)
    print(f"model ready in {time.monotonic() - t0:.1f}s (weights packed on the GPU), batch {batch}", flush=True)
    return model


def _state_dict(args):
    from mk_weights import load_hf_checkpoint, synthetic_state_dict
    if args.model_path.startswith("random:"):
        return synthetic_state_dict(int(args.model_path.split(":")[1] or 0))
    return load_hf_checkpoint(args.model_path)


def run_generation(args):
    tokenizer = args_tokenizer(args)
    prompts = encode_prompts(args, tokenizer)
    B = len(prompts)
    n_new = max_new_tokens(args, prompts)
    lg = None
    if args.enable_nki:
        model = prepare_inference(args, B)
        out = model.generate(prompts, n_new, sampling_params=sampling_params(args, B), seed=args.seed,
                             return_logits=args.output_logits)
        if args.output_logits:
            out, lg = out
            if lg.dim() == 2:
                lg = lg[None]
    else:
        if sampling_params(args) is not None:
            raise SystemExit("the stock path decodes greedily; sampling needs --enable-nki")
        from llama_baseline import StockLlama
        base = StockLlama(_state_dict(args), s_max=args.seq_len)
        rows = []
        for ids in prompts:
            for p in range(len(ids) - 1):
                base.step(int(ids[p]), p)
            tok, row = int(ids[-1]), []
            lrow = []
            for t in range(n_new):
                step = base.step(tok, len(ids) - 1 + t).float().cpu()
                tok = int(step.argmax())
                row.append(tok)
                if args.output_logits:
                    lrow.append(step)
            rows.append(row)
            if args.output_logits:
                lg = (lg or []) + [torch.stack(lrow)]
        out = torch.tensor(rows)
        if args.output_logits:
            lg = torch.stack(lg)
    if out.dim() == 1:
        out = out[None]
    for b in range(B):
        print(f"Output {b}: token ids {out[b].tolist()}")
        if lg is not None:
            print(f"Output {b}: logits [{lg.shape[1]}, {lg.shape[2]}] fp32; per-step max "
                  f"{[round(float(x), 3) for x in lg[b].max(-1).values]}")
        if tokenizer is not None:
            print(f"Output {b}: {tokenizer.decode(out[b].tolist(), skip_special_tokens=True)!r}")
    return out


def run_accuracy_check(args) -> bool:
    """The reference's validate mode (check_accuracy_logits, main.py:274-357)
    for this build: the megakernel model's greedy generation, teacher-forced
    through the stock fp32 path on the same weights, compared step by step.
    Pass rule: validate_pass; the reference's tol_map / divergence tolerance
    (--tol-map, --divergence-difference-tol) are reported as restated checks."""
    from llama_baseline import StockLlama
    from mk_validate import REFERENCE_DIVERGENCE_TOL, divergences, topk_tolerance
    tokenizer = args_tokenizer(args)
    prompts = encode_prompts(args, tokenizer)
    model = prepare_inference(args, len(prompts))
    n_new = max_new_tokens(args, prompts)
    toks, logits = model.generate(prompts, n_new, return_logits=True)   # [B, T], [B, T, V]
    n_check = min(args.num_tokens_to_check or n_new, n_new)
    if args.num_tokens_to_check is not None:
        print(f"Validating logits for first {n_check} tokens")
    base = StockLlama(model.state_dict_bf16, s_max=model.s_max)
    worst, worst_rms, first_div = 0.0, 0.0, None
    got_all, refs_all, agree, gaps = [], [], [], []
    for b, ids in enumerate(prompts):
        seq = torch.cat([ids, toks[b].long()])
        for p in range(len(ids) - 1):
            base.step(int(seq[p]), p)
        for t in range(n_check):
            ref = base.step(int(seq[len(ids) - 1 + t]), len(ids) - 1 + t).cpu()
            refs_all.append(ref)
            got_all.append(logits[b, t])
            dd = (logits[b, t] - ref).abs()
            worst = max(worst, dd.max().item())
            worst_rms = max(worst_rms, dd.pow(2).mean().sqrt().item())
            same = int(ref.argmax()) == int(toks[b, t])
            if not same and first_div is None:
                first_div = (b, t)
            top2 = ref.topk(2).values
            agree.append(same)
            gaps.append(float(top2[0] - top2[1]))
    ok, st = validate_pass(agree, gaps, worst, worst_rms)
    print(f"validate: {len(prompts)} sequence(s) x {n_check} tokens, teacher-forced greedy agreement "
          f"{st['all'] * 100:.2f}%; where the baseline's top-2 gap >= {CLEAR_GAP}: {st['clear'] * 100:.2f}% of "
          f"{st['n_clear']} (floor {CLEAR_FLOOR * 100:.0f}%); where >= {DECIDED_GAP}: {st['decided'] * 100:.2f}% of "
          f"{st['n_decided']} (floor {DECIDED_FLOOR * 100:.0f}%); first divergence at (sequence, step) {first_div}; "
          f"logits max|d| {worst:.3e}, worst per-step rms {worst_rms:.3e}")
    # the reference's logit_validation parameters (main.py:51, 544) as restated checks; reported,
    # not part of the pass rule (their rtol on near-zero logits is below the bf16 noise floor)
    got_all, refs_all = torch.stack(got_all), torch.stack(refs_all)
    tol = REFERENCE_DIVERGENCE_TOL if args.divergence_difference_tol is None else args.divergence_difference_tol
    tm = topk_tolerance(got_all, refs_all, args.tol_map_parsed)
    dv = divergences(got_all, refs_all, tol)
    print("validate: tol_map (restated; steps passing / worst ratio): " +
          ", ".join(f"{k} {v['steps_passing'] * 100:.1f}% / {v['worst_ratio']:.2f}" for k, v in tm.items()) +
          f"; greedy divergences {dv['steps']}, {dv['within_tol']} within divergence_difference_tol {tol}")
    return ok


# Validate pass rule. Two correct bf16 implementations of the step disagree on
# the greedy token wherever the top-2 logits are closer than their rounding
# noise (per-step logit rms ~0.02): with random-init weights the CPU oracle and
# its own fp64-accumulation variant disagree on 44 of the 640 config-3
# positions, all with a top-2 gap below 0.1, and those flips cluster along the
# trajectory (tests/golden/c3_self_agreement.json). A floor on the agreement
# over ALL positions therefore fails correct runs: 28 of the 593 48-position
# windows of that fixture fall below even a floor three binomial deviations
# under the mean. Near-ties are excluded instead: the agreement must be >= 90%
# where the baseline's top-2 gap is >= 0.03 (every window of >= 24 positions of
# the fixture passes) and >= 99% where it is >= 0.1 (100% in the fixture).
CLEAR_GAP, CLEAR_FLOOR = 0.03, 0.90
DECIDED_GAP, DECIDED_FLOOR = 0.1, 0.99
MAX_ABS_BOUND, RMS_BOUND = 0.2, 0.03


def validate_pass(agree, gaps, worst_max_abs: float = 0.0, worst_rms: float = 0.0):
    """(passed, stats) of validate mode's rule for per-position greedy
    agreement flags and the baseline's top-2 logit gaps at those positions."""
    def rate(th):
        sel = [a for a, g in zip(agree, gaps) if g >= th]
        return (sum(sel) / len(sel) if sel else 1.0), len(sel)
    clear, n_clear = rate(CLEAR_GAP)
    decided, n_decided = rate(DECIDED_GAP)
    st = {"all": sum(agree) / max(len(agree), 1), "clear": clear, "n_clear": n_clear, "decided": decided,
          "n_decided": n_decided}
    ok = (worst_max_abs <= MAX_ABS_BOUND and worst_rms <= RMS_BOUND and clear >= CLEAR_FLOOR
          and decided >= DECIDED_FLOOR)
    return ok, st


def generate_report(latencies_ms: List[float], tokens: int) -> dict:
    """Percentiles and throughput of one latency list (the fields of NxDI's
    generate_report as main.py:178-271 prints them): ``tokens`` is the number
    of tokens one latency sample covers, batch included."""
    lat_s = sorted(latencies_ms)
    pct = lambda q: lat_s[min(len(lat_s) - 1, int(q * len(lat_s)))]
    return {"latency_ms_p50": pct(0.5), "latency_ms_p90": pct(0.9), "latency_ms_p95": pct(0.95),
            "latency_ms_p99": pct(0.99), "latency_ms_p100": lat_s[-1], "latency_ms_avg": statistics.mean(lat_s),
            "throughput": tokens / (statistics.mean(lat_s) / 1e3)}


def benchmark_sampling(args):
    """The reference's benchmark_sampling / generate_report (main.py:178-271):
    e2e, context encoding (prefill) and per-step token generation latencies
    over num_runs runs after one warm-up run. With --graph the token-generation
    steps of a run replay one captured HIP graph (the per-step latency is then
    the run's generation time / steps); with --decode-loop (greedy, batch 1)
    they run as one mk_decode_loop launch and the per-step latencies are the
    device clock's intervals between step boundaries."""
    import mk_lib
    prompts = encode_prompts(args, args_tokenizer(args))
    B = len(prompts)
    loop = getattr(args, "decode_loop", False)
    greedy = not args.do_sample or args.top_k == 1
    if loop and (not greedy or B != 1 or args.graph):
        raise SystemExit("--decode-loop runs greedy batch-1 generation (no sampling, one prompt, no --graph)")
    model = prepare_inference(args, B)
    n_new = max_new_tokens(args, prompts)
    sp = sampling_params(args, B)
    if loop:
        clk = torch.zeros(n_new + 1, dtype=torch.int64, device=model.pos.device)
        toks_out = torch.empty(n_new, dtype=torch.int32, device=model.pos.device)
        hz = mk_lib.load().mk_wall_clock_hz(model.pos.device.index or 0)
    dec = model.launcher("decode" if sp is None else "decode_logits")
    graph = model.decode_graph(n_new, sampling_params=sp, seed=args.seed) if args.graph else None
    e2e, cte, tkg = [], [], []
    for r in range(args.num_runs + 1):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        model.prefill(prompts)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(n_new + 1)]
        if loop:
            model.decode_loop(n_new, step_clock=clk, tokens_out=toks_out, check=False)
        elif graph is not None:
            ev[0].record()
            graph.replay()
            ev[n_new].record()
        else:
            ev[0].record()
            for i in range(n_new):
                dec.launch()
                if sp is not None:
                    mk_lib.sample(model.logits, sp, model.tokens, seed=args.seed, counter=model.pos)
                ev[i + 1].record()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        if r == 0:
            continue            # warm-up run
        e2e.append((t2 - t0) * 1e3)
        cte.append((t1 - t0) * 1e3)
        if loop:
            tkg += ((clk[1:] - clk[:-1]).double() * 1e3 / hz).cpu().tolist()
        elif graph is not None:
            tkg += [ev[0].elapsed_time(ev[n_new]) / n_new] * n_new
        else:
            tkg += [ev[i].elapsed_time(ev[i + 1]) for i in range(n_new)]
    bits = model.ws.read_device_error() | model.prefill_device_error()
    if bits:
        raise RuntimeError(f"megakernel device error bits 0x{bits:x}")
    n_prompt = sum(int(p.numel()) for p in prompts)
    report = {"e2e_model": generate_report(e2e, n_prompt + B * n_new),
              "context_encoding_model": generate_report(cte, n_prompt),
              "token_generation_model": generate_report(tkg, B),
              "config": {"batch": B, "prompt_lengths": [int(p.numel()) for p in prompts], "max_new_tokens": n_new,
                         "graph": bool(args.graph), "decode_loop": bool(loop), "num_runs": args.num_runs,
                         "model_path": args.model_path}}
    print(json.dumps(report, indent=4))
    Path(args.report_path).write_text(json.dumps(report))
    return report


def main(argv=None):
    args = parse_args(argv)
    if args.mode == "generate":
        run_generation(args)
    elif args.mode == "validate":
        if not args.enable_nki:
            raise SystemExit("validate compares the megakernel model (--enable-nki) with the stock path")
        ok = run_accuracy_check(args)
        print(f"Validation {'passed' if ok else 'failed'}.")
        return 0 if ok else 1
    elif args.mode == "benchmark":
        if not args.enable_nki:
            raise SystemExit("benchmark measures the megakernel model (--enable-nki)")
        benchmark_sampling(args)
    return 0


if __name__ == "__main__":
    sys.exit(main())
