"""GPU parity of the full batched decode step at BASELINE configs 4 and 5.

Config 4: batch 8, each sequence at its own position, start positions uniform
in [512, 3840] (the benchmark's seed-0 draw), 4096-row caches; 3 consecutive
steps with MK_FLAG_ADVANCE and the greedy token fed back on the device.
Config 5: batch 32, 8192-row caches, positions 8066..8190 (one launch of
``mk_batch_kernel<2>``: two 16-token MFMA tiles, the 2-D down projection, the
lm_head of the 32-token kernel); 2 consecutive steps.

Both: 16 layers + final norm + tied lm_head + argmax, seed-0 Llama-3.2-1B
weights (the MFMA-tiled copies, as the benchmark runs them), caches filled with
N(0,1) bf16 values (BASELINE config 5 allows synthetic KV). For every
sequence of every step, the CPU oracle runs the same step from the GPU's own
cache (bf16 copied before the launch) with the same token and position, and:

* logits within the outer caps of the batch-1 tests (max-abs 0.15, rms 0.03);
* on a subset of sequences of every step (FLOOR_SEQS), a floor measured on
  that state: the oracle against its own fp64-accumulation variants from the
  same cache (tests/noise_variants.py), with p rounded to bf16 as the
  reference does and with p kept fp32 as this split-K kernel does;
  rms(GPU - oracle) must be within 1.3x the second (the spread of a correct
  implementation of the kernel's algorithm; measured 0.92-1.06x, against
  1.15-1.65x of the first), and both ratios are recorded;
* ``next_token`` equals the argmax of the step's own logits; the oracle's
  argmax agrees wherever the oracle's top-2 gap is >= 0.1 (the decided
  positions of the C3 test);
* the K/V scatter is position-exact: in every layer and head, row ``pos[b]``
  of sequence b is the only cache row that changed; layer 0's fresh K row is
  within 2 bf16 ulps of the oracle's (a cancelling RoPE sum turns one ulp of a
  term into two), V within 1;
* ``pos`` advanced by one per sequence.

Measured numbers go to c4.json and c5.json (``record_parity`` in gpu_common).
"""

import os

import pytest
import torch

from gpu_common import bf16_ulp, logit_stats, need_gpu, packed_on_device, record_parity, say

pytestmark = pytest.mark.gpu

STEP_MAX_TOL = 0.15
STEP_RMS_TOL = 0.03
DECIDED_GAP = 0.1
FLOOR_RATIO = 1.3
FLOOR_SEQS = {"c4": (0, 3, 5, 7), "c5": (0, 11, 22, 31)}


@pytest.fixture(scope="module")
def full():
    need_gpu()
    import mk_lib
    from mk_config import LLAMA_3_2_1B
    from mk_weights import synthetic_state_dict
    from oracle.llama_ref import OracleLlama
    torch.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    sd = synthetic_state_dict(seed=0)
    packed = packed_on_device(sd, LLAMA_3_2_1B, rope_rows=8192)
    assert all(k in packed for k in mk_lib.TILED_KEYS)
    return dict(w=mk_lib.weights_struct(packed), packed=packed, oracle=OracleLlama(sd, mode="mk"), sd=sd)


def variant(f):
    """The fp64-accumulation oracle (built once; its round_p is set per run)."""
    if "variant" not in f:
        from noise_variants import FP64Accumulate
        f["variant"] = FP64Accumulate(f["sd"])
    return f["variant"]


def c4_starts():
    """The benchmark's C4 start positions (bench.py: uniform in [512, 3840], seed 0)."""
    g = torch.Generator().manual_seed(0)
    return [int(torch.randint(512, 3840 + 1, (1,), generator=g)) for _ in range(8)]


def run_config(f, name, B, S, starts, n_steps):
    import mk_lib
    from mk_weights import random_token_ids
    kv = torch.empty(16, 2, B, 8, S, 64, dtype=torch.bfloat16, device="cuda")
    gd = torch.Generator(device="cuda").manual_seed(1)
    for l in range(16):
        kv[l].normal_(generator=gd)
    ws = mk_lib.Workspace(B, S, torch.device("cuda"))
    pos = torch.tensor(starts, dtype=torch.int32, device="cuda")
    toks = random_token_ids(B, seed=7).to(device="cuda", dtype=torch.int32)
    logits = torch.empty(B, 128256, dtype=torch.float32, device="cuda")
    step = mk_lib.StepLauncher(f["w"], ws, [kv[l, 0] for l in range(16)], [kv[l, 1] for l in range(16)], pos,
                               tokens=toks, logits=logits, next_token=toks, flags=mk_lib.MK_FLAG_ADVANCE, batch=B)
    o = f["oracle"]
    rec = {"config": name, "batch": B, "s_max": S, "steps": []}
    worst_max = worst_rms = worst_ratio = 0.0
    n_dec = n_dec_ok = n_all = n_all_ok = 0
    for s in range(n_steps):
        pos_in, tok_in = pos.cpu().tolist(), toks.cpu().tolist()
        say(f"[{name}] step {s}: batch {B}, positions {min(pos_in)}..{max(pos_in)}")
        kv_before = kv.clone()
        step.launch()
        torch.cuda.synchronize()
        assert ws.read_device_error() == 0
        lg, nxt = logits.cpu(), toks.cpu()
        assert pos.cpu().tolist() == [p + 1 for p in pos_in]
        # scatter: per layer, the changed (sequence, row) pairs are exactly (b, pos_in[b])
        for l in range(16):
            ch = (kv[l] != kv_before[l]).any(-1).any(0).any(1)     # [B, S]
            got = ch.nonzero().tolist()
            assert got == [[b, pos_in[b]] for b in range(B)], (name, s, l, got[:8])
        srec = []
        for b in range(B):
            p = pos_in[b]
            cache = [(kv_before[l, 0, b].float().cpu(), kv_before[l, 1, b].float().cpu()) for l in range(16)]
            ref, _ = o.forward(torch.tensor([tok_in[b]]), p, cache)
            ref = ref[0]
            st = logit_stats(lg[b], ref)
            top2 = ref.topk(2).values
            gap = float(top2[0] - top2[1])
            agree = int(ref.argmax()) == int(nxt[b])
            st.update(seq=b, pos=p, gpu_token=int(nxt[b]), oracle_token=int(ref.argmax()), top2_gap=round(gap, 4))
            srec.append(st)
            worst_max, worst_rms = max(worst_max, st["max_abs"]), max(worst_rms, st["rms"])
            assert st["max_abs"] <= STEP_MAX_TOL and st["rms"] <= STEP_RMS_TOL, (name, s, b, st)
            if b in FLOOR_SEQS[name]:
                from noise_variants import rms
                v = variant(f)
                floors = {}
                for key, round_p in (("floor_fp64", True), ("floor_fp64_fp32p", False)):
                    v.round_p = round_p
                    vc = [(kv_before[l, 0, b].double().cpu(), kv_before[l, 1, b].double().cpu()) for l in range(16)]
                    floors[key] = rms(ref, v.forward(torch.tensor([tok_in[b]]), p, vc)[0][0])
                gpu_rms = rms(lg[b], ref)
                st.update({k: round(x, 5) for k, x in floors.items()})
                st["ratio_fp64"] = round(gpu_rms / floors["floor_fp64"], 3)
                st["ratio_fp64_fp32p"] = round(gpu_rms / floors["floor_fp64_fp32p"], 3)
                say(f"[{name}] step {s} seq {b}: rms {gpu_rms:.4f}, floor (fp64 acc) {floors['floor_fp64']:.4f}, "
                    f"floor (fp64 acc, fp32 p) {floors['floor_fp64_fp32p']:.4f}, ratios {st['ratio_fp64']:.2f} / "
                    f"{st['ratio_fp64_fp32p']:.2f}")
                worst_ratio = max(worst_ratio, st["ratio_fp64_fp32p"])
                assert gpu_rms <= FLOOR_RATIO * floors["floor_fp64_fp32p"], (name, s, b, st)
            assert int(nxt[b]) == int(lg[b].argmax()), (name, s, b)
            n_all += 1
            n_all_ok += agree
            if gap >= DECIDED_GAP:
                n_dec += 1
                n_dec_ok += agree
                assert agree, (name, s, b, st)
            # layer 0's fresh rows (same embedding input as the oracle's)
            for idx, ulps in ((0, 2.0), (1, 1.0)):
                got_row = kv[0, idx, b, :, p].float().cpu()
                ref_row = cache[0][idx][:, p]
                assert torch.all((got_row - ref_row).abs() <= ulps * bf16_ulp(ref_row) + 1e-6), (name, s, b, idx)
        del kv_before
        rec["steps"].append(srec)
    rec.update(worst_max_abs=worst_max, worst_rms=worst_rms, greedy_agreement=n_all_ok / n_all,
               decided_positions=n_dec, decided_agreement=(n_dec_ok / n_dec) if n_dec else None,
               worst_floor_ratio=worst_ratio,
               tolerances={"max_abs": STEP_MAX_TOL, "rms": STEP_RMS_TOL, "decided_gap": DECIDED_GAP,
                           "rms_vs_floor_fp64_fp32p": FLOOR_RATIO})
    say(f"[{name}] {n_steps} steps x {B} sequences: logits worst max|d| {worst_max:.3e}, worst rms {worst_rms:.3e}; "
        f"greedy agreement {n_all_ok}/{n_all}, on decided positions {n_dec_ok}/{n_dec}")
    record_parity(name, rec)
    ws.release()
    return rec


@pytest.mark.timeout(600)
def test_c4_batch8_ragged_full_step(full):
    run_config(full, "c4", 8, 4096, c4_starts(), n_steps=3)


@pytest.mark.timeout(900)
def test_c5_batch32_8k_full_step(full):
    starts = [8190 - 4 * b for b in range(32)]
    run_config(full, "c5", 32, 8192, starts, n_steps=2)
