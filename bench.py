#!/usr/bin/env python3
"""Benchmark: bs=1 Llama-3.2-1B decode on one MI355X (BASELINE.json metric).

Workload ("C3"): random-init bf16 weights (seed 0),
a 384-token uniform-random prompt prefilled into a 1024-row KV cache on the
GPU (``mk_prefill``: layer by layer on the matrix cores, each layer's weights
streamed once for the whole prompt; its latency is reported as prefill_ms),
then greedy decode. A *step* is one decode step — 16 layers + final norm + tied
lm_head + argmax of the persistent megakernel for one token, the token and
position fed back on the device. One step at position 383 gives the first
token; then K steps are timed from position 384 (K <= 640, so the timed steps
cover KV lengths 384..384+K-1), each way the library runs them:

* loop (the headline ``value``): all K steps in ONE launch of the kernel
  (``mk_decode_loop``, what ``model.generate`` runs for greedy batch 1): an
  on-device step barrier, each step's argmax read by the next; after a
  warm-up loop of W steps and a rewind of the state. Step latencies p50/p90
  from the device wall clock at the step boundaries;
* launch (``per_launch``): one launch per step, W warm-up launches, K back to
  back, then the same K again with a HIP event after each for the latency
  percentiles. The loop's last token and logits equal the K launches' (the
  steps are bitwise the same): ``per_launch.loop_last_step_equal`` records it.

Printed (one JSON line on stdout): tok/s over the timed region (host clock,
synchronised on both sides), ms per step, p50/p90 step latency, the HBM
roofline of the megakernel (algorithmic bytes per step / mean step time from
HIP events around the timed launches, vs 8 TB/s), and a CPU baseline: the
oracle's fp32 decode step timed on this host's cores on a bounded sample.

``--config c4`` / ``--config c5`` time the batched step instead (BASELINE
configs 4 and 5; not the headline line). C4: batch 8 through the model seam
(``NeuronLlamaForCausalLM`` with batch_size 8), each sequence an independent
uniform-random prompt of length uniform in [512, 3840] (seed 0, so that 256
steps fit the 4096-row caches) prefilled on the GPU into its own cache slice,
then greedy steps at every sequence's own position. C5: batch 32 at KV
lengths 8064..8191 of 8192-row caches whose rows below each start position
hold N(0,1) bf16 values instead of prefilled K/V (BASELINE config 5 allows
this to save 258k tokens of prefill; the step's cost does not depend on the
values). tok/s counts every sequence's token.

CPU baselines (every config): the oracle's decode step (fp32 accumulation,
bf16 rounding points; one sequence at a time) timed on the host cores, on a
bounded sample stated in ``sample``; threads = the CPU share the process may
use (its affinity mask, capped by ``OMP_NUM_THREADS``, which the GPU pool sets
to its per-GPU share), with the CPU model string.

``traffic`` is not measured inside a bench run: it is the HBM bytes per step
of the same kernel and workload from two ``rocprofv3 --pmc`` runs (FETCH_SIZE,
WRITE_SIZE, scaled by a plain-copy calibration), read from the committed
``profiles/*_traffic.json`` named in ``traffic_source``.

``--config c2`` times BASELINE config 2 instead: one decoder layer (layer 0 of
the seed-0 weights) as its own launch of the decode kernel (``mk_layer_step``
seam), batch 1, a 1024-row KV cache of N(0,1) bf16 values, the step at position
1023 and an N(0,1) input row; it reports µs per layer launch and HBM GB/s, and
its CPU baseline (the oracle's layer, timed on the host) doubles as the check:
the max-abs error of the GPU layer against it.

``--gpus N`` with N > 1 exits: this benchmark runs on one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "llama1b-megakernel_amd"))
sys.path.insert(1, str(REPO))

HBM_PEAK_GBS = 8000.0
# HBM bytes per decode step measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
# (scaled by the plain-copy calibration), one file per kernel and workload
TRAFFIC_JSON = {
    "c3": REPO / "profiles" / "mk_decode_kernel_c3_bs1_traffic.json",
    "c4": REPO / "profiles" / "mk_batch_kernel_c4_traffic.json",
    "c5": REPO / "profiles" / "mk_batch_kernel_c5_traffic.json",
}
PROMPT = 384
S_MAX = 1024
BATCH_CONFIGS = {
    "c4": dict(batch=8, s_max=4096, steps=256, lo=512, hi=3840),
    "c5": dict(batch=32, s_max=8192, steps=128, lo=8192 - 128, hi=8192 - 128),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def timed_steps(launch, K: int):
    """Time K back-to-back launches with HIP events only around the whole
    run (an event recorded between two launches puts a marker packet between
    the kernels, which costs several us per step on this stack), bracketed by
    synchronisations; returns (host wall s, mean ms per step from the events)."""
    import torch
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    e0.record()
    for _ in range(K):
        launch()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    return wall, e0.elapsed_time(e1) / K


def step_latencies(launch, K: int, reset):
    """After the timed run: reset the state and run the same K steps again
    with an event after each, for the per-step latency percentiles (each
    interval includes its event marker)."""
    import torch
    reset()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(K + 1)]
    torch.cuda.synchronize()
    evs[0].record()
    for i in range(K):
        launch()
        evs[i + 1].record()
    torch.cuda.synchronize()
    return [evs[i].elapsed_time(evs[i + 1]) for i in range(K)]


def cpu_threads() -> int:
    """Host threads for the CPU baseline: the affinity mask, capped by
    OMP_NUM_THREADS (the GPU pool sets it to the CPU share of one GPU)."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, n)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def traffic_of(config: str):
    """(HBM bytes per step, source) from the committed rocprofv3 counter summary, or (None, None)."""
    f = TRAFFIC_JSON.get(config)
    if f is None or not f.exists():
        return None, None
    return int(json.loads(f.read_text())["traffic_bytes_per_step"]), str(f.relative_to(REPO))


def cpu_baseline(sd, positions, s_max: int, steps_per_seq: int, budget_s: float, what: str):
    """The oracle's decode step (fp32 accumulation, bf16 rounding points) on the
    host cores: for each of ``steps_per_seq`` rounds, one step of every
    sequence in ``positions`` (its start position + round), over one
    synthetic N(0,1) bf16 cache of ``s_max`` rows (a step reads only rows
    below its position, so the sequences can share it). Stops early after
    ``budget_s`` seconds of steps."""
    import torch
    from oracle.llama_ref import OracleLlama
    threads = cpu_threads()
    torch.set_num_threads(threads)
    t0 = time.perf_counter()
    o = OracleLlama(sd, mode="mk")
    g = torch.Generator().manual_seed(1)
    cache = [(torch.randn(8, s_max, 64, generator=g).to(torch.bfloat16).float(),
              torch.randn(8, s_max, 64, generator=g).to(torch.bfloat16).float()) for _ in range(16)]
    log(f"[cpu] oracle ready in {time.perf_counter() - t0:.1f}s, {threads} threads ({cpu_model()})")
    tok = torch.tensor([17])
    o.forward(tok, positions[0], cache)              # warm-up step
    o.forward(tok, positions[0], cache)
    times, done = [], []
    t_start = time.perf_counter()
    for r in range(steps_per_seq):
        for p in positions:
            t = time.perf_counter()
            logits, _ = o.forward(tok, p + r, cache)
            tok = logits.argmax(-1)
            times.append(time.perf_counter() - t)
            done.append(p + r)
            if time.perf_counter() - t_start > budget_s:
                break
        if time.perf_counter() - t_start > budget_s:
            break
    total = sum(times)
    return {
        "value": round(len(times) / total, 3), "unit": "tok/s", "cores": threads, "kind": "port",
        "cpu_model": cpu_model(),
        "sample": f"{len(times)} oracle decode steps ({what}; fp32 accumulation, bf16 rounding points, one "
                  f"sequence per step) at positions {min(done)}..{max(done)} over a synthetic N(0,1) bf16 KV "
                  f"cache of {s_max} rows, after 2 warm-up steps; p50 {statistics.median(times) * 1e3:.1f} ms/step",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=640)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-steps", type=int, default=48, help="C3 CPU baseline steps (>= 32)")
    ap.add_argument("--cpu-budget-s", type=float, default=30.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--c3-mode", choices=["loop", "launch", "both"], default="both",
                    help="C3 steps as one mk_decode_loop launch (loop), one launch per step (launch), or both "
                         "(the loop is the headline; the per-launch figures go to per_launch)")
    ap.add_argument("--config", choices=["c2", "c3", "c4", "c5"], default="c3",
                    help="c3: the headline bs=1 decode; c2: one decoder layer; c4/c5: the batched configurations")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run 10 plain device copies of BYTES (HBM counter calibration for rocprofv3)")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        src = torch.ones(args.copy_calibration // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": args.copy_calibration, "dispatches": 10}))
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU; --gpus {args.gpus} is not supported by this build", file=sys.stderr)
        sys.exit(2)
    if args.config == "c2":
        run_layer(args)
        return
    if args.config != "c3":
        run_batched(args, BATCH_CONFIGS[args.config])
        return
    if not 1 <= args.steps <= S_MAX - PROMPT:
        sys.exit(f"--steps must be in [1, {S_MAX - PROMPT}]")

    import torch
    import mk_lib
    from mk_config import step_bytes
    from llama_with_megakernel import NeuronLlamaForCausalLM, NeuronConfigLlamaMK, LlamaInferenceConfig
    from mk_weights import random_token_ids

    t0 = time.perf_counter()
    cfg = LlamaInferenceConfig(NeuronConfigLlamaMK(seq_len=S_MAX, max_context_length=S_MAX))
    model = NeuronLlamaForCausalLM("random:0", cfg)
    model.compile()
    model.load()
    log(f"[bench] weights packed in {time.perf_counter() - t0:.1f}s; grid = {mk_lib.load().mk_grid_size(0)} WGs")

    prompt = random_token_ids(PROMPT, seed=0)
    model.prefill(prompt)                        # warm-up (first use allocates the prefill workspace)
    torch.cuda.synchronize()
    tp = time.perf_counter()
    model.prefill(prompt)                        # context encoding: 383 prompt tokens, layer by layer
    torch.cuda.synchronize()
    prefill_ms = (time.perf_counter() - tp) * 1e3
    if model.prefill_device_error():
        sys.exit("device error in the prefill steps")
    dec = model.launcher("decode")
    dec.launch()                                 # position 383 -> first generated token
    torch.cuda.synchronize()
    pos0 = model.pos.clone()
    tok0 = model.tokens.clone()
    assert int(pos0.item()) == PROMPT

    if args.c3_mode != "loop":
        for _ in range(args.warmup):
            dec.launch()
    torch.cuda.synchronize()
    model.pos.copy_(pos0)
    model.tokens.copy_(tok0)
    torch.cuda.synchronize()

    K = args.steps

    def reset():
        model.pos.copy_(pos0)
        model.tokens.copy_(tok0)
        torch.cuda.synchronize()

    per_launch = None
    if args.c3_mode in ("launch", "both"):
        # one launch per step (the reference's call pattern): K back-to-back
        # launches, then the same K again with an event after each for the
        # latency percentiles
        wall1, mean1 = timed_steps(dec.launch, K)
        ref_state = (model.tokens.clone(), model.logits.clone())
        step_ms1 = step_latencies(dec.launch, K, reset)
        per_launch = {"value": round(K / wall1, 2), "ms_per_step": round(wall1 * 1e3 / K, 4),
                      "p50_step_ms": round(statistics.median(step_ms1), 4),
                      "p90_step_ms": round(sorted(step_ms1)[int(0.9 * (K - 1))], 4),
                      "kernel_ms_per_step": round(mean1, 4)}
    loop = None
    if args.c3_mode in ("loop", "both"):
        # the greedy loop: all K steps in one launch (mk_decode_loop), the same
        # per-step work; step latencies from the device clock at the step
        # boundaries
        reset()
        if args.warmup:
            model.decode_loop(args.warmup)
        reset()
        clk = torch.zeros(K + 1, dtype=torch.int64, device="cuda")
        toks_out = torch.empty(K, dtype=torch.int32, device="cuda")
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t_start = time.perf_counter()
        e0.record()
        # (the step range was checked above: K <= S_MAX - PROMPT)
        model.decode_loop(K, step_clock=clk, tokens_out=toks_out, check=False)
        e1.record()
        torch.cuda.synchronize()
        wall2 = time.perf_counter() - t_start
        mean2 = e0.elapsed_time(e1) / K
        hz = mk_lib.load().mk_wall_clock_hz(0)
        step_ms2 = ((clk[1:] - clk[:-1]).double() * 1e3 / hz).cpu().tolist()
        if per_launch is not None:
            # the loop's steps are the single launches' computation bit for bit
            per_launch["loop_last_step_equal"] = bool(torch.equal(model.tokens, ref_state[0])
                                                      and torch.equal(model.logits, ref_state[1]))
            if not per_launch["loop_last_step_equal"]:
                log("[bench] WARNING: the decode loop's last token / logits differ from K single launches")
        loop = {"value": round(K / wall2, 2), "ms_per_step": round(wall2 * 1e3 / K, 4),
                "p50_step_ms": round(statistics.median(step_ms2), 4),
                "p90_step_ms": round(sorted(step_ms2)[int(0.9 * (K - 1))], 4),
                "kernel_ms_per_step": round(mean2, 4)}
    bits = model.ws.read_device_error()
    if bits:
        sys.exit(f"device error bits 0x{bits:x}")
    head = loop if loop is not None else per_launch
    bytes_per_step = sum(step_bytes(16, [PROMPT + i], lm_head=True) for i in range(K)) / K
    achieved = bytes_per_step / (head["kernel_ms_per_step"] * 1e-3) / 1e9
    if per_launch is not None:
        a1 = bytes_per_step / (per_launch["kernel_ms_per_step"] * 1e-3) / 1e9
        per_launch.update(achieved_gbs=round(a1, 1), frac=round(a1 / HBM_PEAK_GBS, 4))

    traffic, traffic_src = traffic_of("c3")
    how = ("all K steps in one launch of mk_decode_kernel (mk_decode_loop: an on-device step barrier, each "
           "step's argmax fed to the next)" if loop is not None else "one launch of mk_decode_kernel per step")
    result = {
        "metric": "bs=1 decode tok/s + p50 step latency, Llama-3.2-1B ctx1024; HBM GB/s",
        "value": head["value"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "p50_step_ms": head["p50_step_ms"],
        "p90_step_ms": head["p90_step_ms"],
        "prefill_ms": round(prefill_ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) bf16 weights seed 0, uniform-random prompt ids seed 0)",
        "config": {"workload": "C3: Llama-3.2-1B decode, batch 1, 384-token prompt prefilled to a 1024-row "
                               f"KV cache, greedy steps at KV lengths {PROMPT}..{PROMPT + K - 1}",
                   "batch": 1, "prompt": PROMPT, "max_context_length": S_MAX, "n_layers": 16,
                   "steps_run_as": how},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                     "bytes_per_step": int(bytes_per_step), "kernel": "mk_decode_kernel"},
        "per_launch": per_launch,
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        del model
        torch.cuda.empty_cache()
        from mk_weights import synthetic_state_dict
        sd = synthetic_state_dict(seed=0)
        result["cpu_baseline"] = cpu_baseline(sd, [PROMPT + 1], S_MAX, args.cpu_steps, args.cpu_budget_s,
                                              "C3 shapes, batch 1")
    print(json.dumps(result), flush=True)


def run_layer(args):
    """one decoder layer launch at KV position 1023."""
    import torch
    import mk_lib
    from mk_config import LlamaDims, step_bytes
    from mk_weights import pack_for_megakernel, synthetic_state_dict

    S, POS = S_MAX, S_MAX - 1
    dp = LlamaDims(n_layers=1)
    sd = synthetic_state_dict(seed=0, d=dp)
    packed = pack_for_megakernel(sd, dp, device="cuda", rope_rows=S)
    w = mk_lib.weights_struct(packed)
    g = torch.Generator().manual_seed(2)
    hidden = torch.randn(1, 2048, generator=g).to(torch.bfloat16)
    k0 = torch.randn(1, 8, S, 64, generator=g).to(torch.bfloat16)
    v0 = torch.randn(1, 8, S, 64, generator=g).to(torch.bfloat16)
    kc, vc = k0.cuda(), v0.cuda()
    ws = mk_lib.Workspace(1, S, torch.device("cuda"))
    pos = torch.tensor([POS], dtype=torch.int32, device="cuda")
    out = torch.empty(1, 2048, dtype=torch.bfloat16, device="cuda")
    step = mk_lib.StepLauncher(w, ws, [kc], [vc], pos, hidden_in=hidden.cuda(), hidden_out=out)
    for _ in range(args.warmup):
        step.launch()          # every launch recomputes the same layer (row POS rewritten identically)
    torch.cuda.synchronize()
    K = args.steps
    wall, mean_ms = timed_steps(step.launch, K)
    us = [v * 1e3 for v in step_latencies(step.launch, K, lambda: None)]
    bits = ws.read_device_error()
    if bits:
        sys.exit(f"device error bits 0x{bits:x}")
    mean_us = mean_ms * 1e3
    nbytes = step_bytes(1, [POS], lm_head=False) + 2048 * 2   # + the hidden_out row
    achieved = nbytes / (mean_us * 1e-6) / 1e9
    result = {
        "metric": "single decoder layer us per launch (Llama-3.2-1B layer, batch 1, KV length 1024); HBM GB/s",
        "value": round(mean_us, 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / K, 4),
        "p50_us": round(statistics.median(us), 2),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) bf16 layer weights seed 0, N(0,1) bf16 input and KV cache)",
        "config": {"workload": "C2: one Llama-3.2-1B decoder layer as its own launch, batch 1, KV cache "
                               f"[1,8,{S},64], step at position {POS}", "batch": 1, "kv_rows": S, "n_layers": 1},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "bytes_per_step": int(nbytes),
                     "kernel": "mk_decode_kernel (one layer, no lm_head)"},
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        # the oracle's layer on the host cores: timed, and the reference for the max-abs check
        from oracle.llama_ref import Dims, OracleLlama
        threads = cpu_threads()
        torch.set_num_threads(threads)
        o = OracleLlama(sd, Dims(n_layers=1), mode="mk")
        times, ref = [], None
        for _ in range(22):
            cache = [(k0[0].float().clone(), v0[0].float().clone())]
            t = time.perf_counter()
            _, ref = o.forward(None, POS, cache, hidden=hidden.float(), want_logits=False)
            times.append(time.perf_counter() - t)
        times = times[2:]                       # 2 warm-up runs
        err = (out.cpu().float() - ref).abs().max().item()
        result["max_abs_err_vs_oracle"] = round(err, 5)
        result["cpu_baseline"] = {
            "value": round(statistics.median(times) * 1e6, 1), "unit": "us", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{len(times)} runs of the oracle's decoder layer (fp32 accumulation, bf16 rounding "
                      f"points) at position {POS} after 2 warm-up runs, median",
        }
    print(json.dumps(result), flush=True)


def run_batched(args, cfg):
    """A batched decode configuration (BASELINE configs 4 and 5)."""
    import torch
    import mk_lib
    from mk_config import LLAMA_3_2_1B, step_bytes
    from mk_weights import random_token_ids

    B, S, K = cfg["batch"], cfg["s_max"], min(args.steps, cfg["steps"])
    g = torch.Generator().manual_seed(0)
    lens = [int(torch.randint(cfg["lo"], cfg["hi"] + 1, (1,), generator=g)) for _ in range(B)]
    t0 = time.perf_counter()
    prefill_ms = None
    if args.config == "c4":
        # the model seam: one prompt per sequence, prefilled on the GPU into its own cache slice
        from llama_with_megakernel import LlamaInferenceConfig, NeuronConfigLlamaMK, NeuronLlamaForCausalLM
        model = NeuronLlamaForCausalLM("random:0", LlamaInferenceConfig(
            NeuronConfigLlamaMK(batch_size=B, seq_len=S, max_context_length=S)))
        model.compile()
        model.load()
        sd = model.state_dict_bf16
        prompts = [random_token_ids(n, seed=100 + b) for b, n in enumerate(lens)]
        model.prefill(prompts)                       # warm-up (allocates the prefill workspace)
        torch.cuda.synchronize()
        tp = time.perf_counter()
        model.prefill(prompts)
        torch.cuda.synchronize()
        prefill_ms = (time.perf_counter() - tp) * 1e3
        if model.prefill_device_error():
            sys.exit("device error in the prefill steps")
        step, ws, pos, toks = model.launcher("decode"), model.ws, model.pos, model.tokens
        starts = [n - 1 for n in lens]
        data = ("synthetic (random-init N(0,0.02) bf16 weights seed 0; one uniform-random prompt per sequence, "
                "prefilled on the GPU)")
        workload = (f"C4: Llama-3.2-1B decode, batch 8, independent prompts of lengths {min(lens)}..{max(lens)} "
                    f"prefilled into {S}-row KV caches, {K} greedy steps")
    else:
        from mk_weights import pack_for_megakernel, synthetic_state_dict
        sd = synthetic_state_dict(seed=0)
        packed = pack_for_megakernel(sd, LLAMA_3_2_1B, device="cuda", rope_rows=S)
        w = mk_lib.weights_struct(packed)
        # caches: N(0,1) bf16 (rows at and above a sequence's start are rewritten by the steps)
        kv = torch.empty(16, 2, B, 8, S, 64, dtype=torch.bfloat16, device="cuda")
        gd = torch.Generator(device="cuda").manual_seed(1)
        for l in range(16):
            kv[l].normal_(generator=gd)
        ws = mk_lib.Workspace(B, S, torch.device("cuda"))
        starts = lens
        pos = torch.tensor(starts, dtype=torch.int32, device="cuda")
        toks = random_token_ids(B, seed=0).to(device="cuda", dtype=torch.int32)
        logits = torch.empty(B, LLAMA_3_2_1B.vocab, dtype=torch.float32, device="cuda")
        step = mk_lib.StepLauncher(w, ws, [kv[l, 0] for l in range(16)], [kv[l, 1] for l in range(16)], pos,
                                   tokens=toks, logits=logits, next_token=toks, flags=mk_lib.MK_FLAG_ADVANCE,
                                   batch=B)
        data = ("synthetic (random-init N(0,0.02) bf16 weights seed 0, N(0,1) bf16 KV cache below each start "
                "position, uniform-random token ids)")
        workload = (f"C5: Llama-3.2-1B decode, batch {B}, {S}-row KV caches, start positions "
                    f"{min(starts)}..{max(starts)}, {K} greedy steps")
    torch.cuda.synchronize()
    log(f"[bench] {args.config}: batch {B}, cache rows {S}, start positions {min(starts)}..{max(starts)}; "
        f"ready in {time.perf_counter() - t0:.1f}s")
    pos0, tok0 = pos.clone(), toks.clone()
    for _ in range(min(args.warmup, K)):
        step.launch()
    torch.cuda.synchronize()
    pos.copy_(pos0)
    toks.copy_(tok0)

    def reset():
        pos.copy_(pos0)
        toks.copy_(tok0)
        torch.cuda.synchronize()

    wall, mean_ms = timed_steps(step.launch, K)
    step_ms = step_latencies(step.launch, K, reset)
    bits = ws.read_device_error()
    if bits:
        sys.exit(f"device error bits 0x{bits:x}")
    bytes_per_step = sum(step_bytes(16, [p + i for p in starts], lm_head=True) for i in range(K)) / K
    achieved = bytes_per_step / (mean_ms * 1e-3) / 1e9
    traffic, traffic_src = traffic_of(args.config)
    result = {
        "metric": f"batched decode tok/s (all sequences), Llama-3.2-1B, {args.config.upper()}; HBM GB/s",
        "value": round(B * K / wall, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / K, 4),
        "p50_step_ms": round(statistics.median(step_ms), 4),
        "p90_step_ms": round(sorted(step_ms)[int(0.9 * (K - 1))], 4),
        "prefill_ms": None if prefill_ms is None else round(prefill_ms, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": data,
        "config": {"workload": workload, "batch": B, "max_context_length": S, "start_positions": starts,
                   "n_layers": 16},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                     "bytes_per_step": int(bytes_per_step),
                     "kernel": f"mk_batch_kernel<{1 if B <= 16 else 2}>"},
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        if args.config == "c4":
            del model
        torch.cuda.empty_cache()
        if args.config == "c4":
            result["cpu_baseline"] = cpu_baseline(sd, starts, S, 2, args.cpu_budget_s,
                                                  "C4 shapes: each of the 8 sequences' start positions, 2 rounds")
        else:
            result["cpu_baseline"] = cpu_baseline(sd, starts[::8], S, 4, args.cpu_budget_s,
                                                  "C5 shapes: 4 of the 32 sequences' start positions, 4 rounds")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
