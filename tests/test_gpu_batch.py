"""GPU parity of the batched decode step (mk_batch.hip, batch 1..32) with the oracle.

BASELINE configs 4 and 5 decode batches of independent sequences at ragged
positions (per-sequence cache rows, per-sequence split-K attention). The
batched kernel computes the projections with MFMA tiles whose summation order
differs from the batch-1 kernel's, so results are compared with the oracle
(and with the batch-1 kernel) at the same tolerances as the batch-1 tests:

* one decoder layer, batch sizes 1, 2, 5, 16, 17 (first two-tile batch) and
  32, every sequence at its own position (0, 31, 32, ... up to s_max-1): each
  sequence's output hidden within 2^-5 * max(|ref|, |x|, 1) of the oracle ("mk"
  rounding; x the layer input), with an rms no larger than 1.5x the oracle's
  own bf16-vs-float64 departure; the K/V scatter position-exact per sequence
  (only row pos[b] of sequence b changes, in every kv head) and the written
  rows within 1 bf16 ulp;
* the full 16-layer step with lm_head at batch 4, each sequence prefilled to a
  different length by the batch-1 kernel in its own slice of the batched
  cache: per-sequence logits within the per-step bounds of the batch-1 decode
  tests (max-abs 0.15, rms 0.03; see tests/test_gpu_decode.py for the bf16
  noise floor they sit on), next_token the argmax of the step's own logits,
  the same logits as the batch-1 kernel from the same state within those
  bounds, and the scatter position-exact over all 16 layers;
* the same full step at batch 20 (the two-tile kernel with a partial second
  tile): every sequence against the batch-1 kernel, two against the oracle;
* bitwise repeatability, MK_FLAG_ADVANCE on every sequence, and a step with
  one position out of range refused as a whole (error bit, nothing written).
"""

import os

import pytest
import torch

from gpu_common import bf16_ulp, need_gpu, packed_on_device, say

pytestmark = pytest.mark.gpu

S = 256
STEP_MAX_TOL = 0.15
STEP_RMS_TOL = 0.03


def ragged_positions(batch: int, s_max: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    fixed = [0, 31, 32, 127, 128, s_max - 1]
    pos = [fixed[b] if b < len(fixed) else int(torch.randint(0, s_max, (1,), generator=g)) for b in range(batch)]
    return pos


# ---------------------------------------------------------------------------
# one layer
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def layer1():
    need_gpu()
    from mk_config import LlamaDims
    from mk_weights import synthetic_state_dict
    from oracle.llama_ref import Dims, OracleLlama
    torch.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    dp = LlamaDims(n_layers=1)
    sd = synthetic_state_dict(seed=0, d=dp)
    packed = packed_on_device(sd, dp, rope_rows=S)
    d = Dims(n_layers=1)
    return packed, OracleLlama(sd, d, mode="mk"), OracleLlama(sd, d, mode="exact")


def run_batched_layer(packed, hidden, kc, vc, pos_list, ws_batch=None):
    import mk_lib
    B = len(pos_list)
    w = mk_lib.weights_struct(packed)
    ws = mk_lib.Workspace(ws_batch or max(B, 2), S, torch.device("cuda"))
    pos = torch.tensor(pos_list, dtype=torch.int32, device="cuda")
    out = torch.empty(B, 2048, dtype=torch.bfloat16, device="cuda")
    mk_lib.decode_step(w, ws, [kc], [vc], pos, hidden_in=hidden, hidden_out=out, n_layers=1, batch=B)
    torch.cuda.synchronize()
    return out, ws


@pytest.mark.parametrize("batch", [1, 2, 5, 16, 17, 32])
def test_batched_layer_matches_oracle(layer1, batch):
    packed, o_mk, o_exact = layer1
    pos_list = ragged_positions(batch, S, seed=batch)
    say(f"[blayer] batch={batch} pos={pos_list}")
    g = torch.Generator().manual_seed(1000 + batch)
    hidden = torch.randn(batch, 2048, generator=g).to(torch.bfloat16)
    k0 = torch.randn(batch, 8, S, 64, generator=g).to(torch.bfloat16)
    v0 = torch.randn(batch, 8, S, 64, generator=g).to(torch.bfloat16)
    kc, vc = k0.cuda(), v0.cuda()
    out, ws = run_batched_layer(packed, hidden.cuda(), kc, vc, pos_list)
    assert ws.read_device_error() == 0
    got_all, k1, v1 = out.cpu().float(), kc.cpu(), vc.cpu()
    worst_ulps, worst_ratio = 0.0, 0.0
    for b, p in enumerate(pos_list):
        cache = [(k0[b].float().clone(), v0[b].float().clone())]
        _, ref = o_mk.forward(None, p, cache, hidden=hidden[b:b + 1].float(), want_logits=False)
        _, exact = o_exact.forward(None, p, [(k0[b].double(), v0[b].double())], hidden=hidden[b:b + 1].double(),
                                   want_logits=False)
        ref, exact = ref[0], exact[0]
        got = got_all[b]
        diff = (got - ref).abs()
        # elementwise: a few bf16 ulps at the scale of the residual sum's operands (where the
        # layer input and the layer's contribution nearly cancel, the result is small while
        # the roundings happened at |x|; the batch-1 kernel shows the same values there)
        scale = torch.maximum(ref.abs(), hidden[b].float().abs()).clamp_min(1.0)
        worst_ulps = max(worst_ulps, (diff / bf16_ulp(scale)).max().item())
        assert torch.all(diff <= 2.0 ** -5 * scale), (b, p, diff.max().item())
        rms_gpu = (got.double() - ref.double()).pow(2).mean().sqrt().item()
        rms_bf16 = (ref.double() - exact).pow(2).mean().sqrt().item()
        worst_ratio = max(worst_ratio, rms_gpu / max(rms_bf16, 1e-12))
        assert rms_gpu <= 1.5 * rms_bf16 + 1e-6, (b, p, rms_gpu, rms_bf16)
        # scatter: only row p of sequence b changed, written rows match the oracle's
        mask = torch.ones(S, dtype=torch.bool)
        mask[p] = False
        assert torch.equal(k1[b][:, mask].view(torch.int16), k0[b][:, mask].view(torch.int16)), (b, p)
        assert torch.equal(v1[b][:, mask].view(torch.int16), v0[b][:, mask].view(torch.int16)), (b, p)
        for got_row, ref_row in ((k1[b][:, p].float(), cache[0][0][:, p]), (v1[b][:, p].float(), cache[0][1][:, p])):
            dd = (got_row - ref_row).abs()
            assert torch.all(dd <= bf16_ulp(ref_row) + 1e-6), (b, p)
            assert (dd > 0).float().mean().item() < 0.05, (b, p)
    say(f"[blayer] batch={batch}: max ulps (at the operands' scale) {worst_ulps:.2f}, worst rms ratio vs bf16 floor {worst_ratio:.2f}")


@pytest.mark.parametrize("batch", [5, 32])
def test_batched_tiled_weights_bitwise_equal_row_major(layer1, batch):
    """The MFMA-tiled weight copies only change where each B operand is read
    from: every MFMA gets the same lane data, so the layer output, the K/V
    rows, the lm_head logits and the argmax are bit-identical to a run on the
    row-major stacks (batch 5: one 16-row tile; batch 32: two tiles and the
    2-D down projection)."""
    import mk_lib
    packed = layer1[0]
    assert all(k in packed for k in mk_lib.TILED_KEYS)
    pos_list = ragged_positions(batch, S, seed=50 + batch)
    say(f"[tiled] batch={batch} pos={pos_list}")
    g = torch.Generator().manual_seed(2000 + batch)
    hidden = torch.randn(batch, 2048, generator=g).to(torch.bfloat16).cuda()
    k0 = torch.randn(batch, 8, S, 64, generator=g).to(torch.bfloat16)
    v0 = torch.randn(batch, 8, S, 64, generator=g).to(torch.bfloat16)
    runs = []
    for tiled in (True, False):
        w = mk_lib.weights_struct(packed, tiled=tiled)
        assert (w.t_gu is not None) == tiled
        ws = mk_lib.Workspace(max(batch, 2), S, torch.device("cuda"))
        kc, vc = k0.cuda(), v0.cuda()
        pos = torch.tensor(pos_list, dtype=torch.int32, device="cuda")
        out = torch.empty(batch, 2048, dtype=torch.bfloat16, device="cuda")
        logits = torch.empty(batch, mk_lib.VOCAB, dtype=torch.float32, device="cuda")
        nxt = torch.empty(batch, dtype=torch.int32, device="cuda")
        mk_lib.decode_step(w, ws, [kc], [vc], pos, hidden_in=hidden, hidden_out=out, logits=logits,
                           next_token=nxt, n_layers=1, batch=batch)
        torch.cuda.synchronize()
        assert ws.read_device_error() == 0
        runs.append((out.cpu().view(torch.int16), kc.cpu().view(torch.int16), vc.cpu().view(torch.int16),
                     logits.cpu().view(torch.int32), nxt.cpu()))
    for name, a, b in zip(("hidden", "k", "v", "logits", "next"), *runs):
        assert torch.equal(a, b), name


def test_batched_layer_bad_position_refused(layer1):
    import mk_lib
    packed, _, _ = layer1
    B = 3
    g = torch.Generator().manual_seed(77)
    hidden = torch.randn(B, 2048, generator=g).to(torch.bfloat16).cuda()
    kc = torch.randn(B, 8, S, 64, generator=g).to(torch.bfloat16).cuda()
    vc = torch.randn(B, 8, S, 64, generator=g).to(torch.bfloat16).cuda()
    k0, v0 = kc.clone(), vc.clone()
    w = mk_lib.weights_struct(packed)
    ws = mk_lib.Workspace(B, S, torch.device("cuda"))
    pos = torch.tensor([5, S, 9], dtype=torch.int32, device="cuda")
    out = torch.full((B, 2048), 7.0, dtype=torch.bfloat16, device="cuda")
    mk_lib.decode_step(w, ws, [kc], [vc], pos, hidden_in=hidden, hidden_out=out, n_layers=1, batch=B,
                       flags=mk_lib.MK_FLAG_ADVANCE)
    bits = ws.read_device_error()
    assert bits & mk_lib.MK_DEVERR_POS
    assert torch.equal(kc.view(torch.int16), k0.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), v0.view(torch.int16))
    assert torch.all(out.float() == 7.0)
    assert pos.tolist() == [5, S, 9]
    assert ws.read_device_error() == 0
    # the workspace is still usable
    pos.copy_(torch.tensor([5, 6, 9], dtype=torch.int32))
    mk_lib.decode_step(w, ws, [kc], [vc], pos, hidden_in=hidden, hidden_out=out, n_layers=1, batch=B)
    assert ws.read_device_error() == 0
    assert not torch.all(out.float() == 7.0)


def test_batch_larger_than_workspace_is_refused(layer1):
    import mk_lib
    packed, _, _ = layer1
    w = mk_lib.weights_struct(packed)
    ws = mk_lib.Workspace(4, S, torch.device("cuda"))
    kc = torch.zeros(5, 8, S, 64, dtype=torch.bfloat16, device="cuda")
    hidden = torch.zeros(5, 2048, dtype=torch.bfloat16, device="cuda")
    pos = torch.zeros(5, dtype=torch.int32, device="cuda")
    out = torch.empty(5, 2048, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(mk_lib.MkError) as ei:
        mk_lib.decode_step(w, ws, [kc], [kc], pos, hidden_in=hidden, hidden_out=out, n_layers=1, batch=5)
    assert ei.value.code == -3


# ---------------------------------------------------------------------------
# full 16-layer step
# ---------------------------------------------------------------------------

PROMPT_LENS = [37, 100, 5, 150]


@pytest.fixture(scope="module")
def full16():
    need_gpu()
    import mk_lib
    from mk_config import LLAMA_3_2_1B
    from mk_weights import random_token_ids, synthetic_state_dict
    from oracle.llama_ref import OracleLlama
    torch.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    sd = synthetic_state_dict(seed=0)
    packed = packed_on_device(sd, LLAMA_3_2_1B, rope_rows=S)
    w = mk_lib.weights_struct(packed)
    B = len(PROMPT_LENS)
    kv = torch.zeros(16, 2, B, 8, S, 64, dtype=torch.bfloat16, device="cuda")
    prompts = [random_token_ids(n, seed=50 + b) for b, n in enumerate(PROMPT_LENS)]
    # prefill each sequence with the batch-1 kernel in its own slice of the batched cache
    ws1 = mk_lib.Workspace(1, S, torch.device("cuda"))
    for b, ids in enumerate(prompts):
        pos = torch.zeros(1, dtype=torch.int32, device="cuda")
        tok = torch.zeros(1, dtype=torch.int32, device="cuda")
        l = mk_lib.StepLauncher(w, ws1, [kv[i, 0, b:b + 1] for i in range(16)], [kv[i, 1, b:b + 1] for i in range(16)],
                                pos, tokens=tok, flags=mk_lib.MK_FLAG_ADVANCE)
        ids_dev = ids.to(device="cuda", dtype=torch.int32)
        for i in range(len(ids) - 1):
            tok.copy_(ids_dev[i:i + 1])
            l.launch()
    torch.cuda.synchronize()
    assert ws1.read_device_error() == 0
    oracle = OracleLlama(sd, mode="mk")
    return dict(w=w, packed=packed, kv=kv, prompts=prompts, oracle=oracle, ws1=ws1)


def batched_step(f, ws=None, flags=0):
    """One batched step from the prefilled state: each sequence's last prompt token at pos len-1."""
    import mk_lib
    B = len(PROMPT_LENS)
    ws = ws or mk_lib.Workspace(B, S, torch.device("cuda"))
    kv = f["kv"]
    pos = torch.tensor([n - 1 for n in PROMPT_LENS], dtype=torch.int32, device="cuda")
    toks = torch.tensor([int(p[-1]) for p in f["prompts"]], dtype=torch.int32, device="cuda")
    logits = torch.zeros(B, 128256, dtype=torch.float32, device="cuda")
    nxt = torch.full((B,), -5, dtype=torch.int32, device="cuda")
    hid = torch.zeros(B, 2048, dtype=torch.bfloat16, device="cuda")
    mk_lib.decode_step(f["w"], ws, [kv[i, 0] for i in range(16)], [kv[i, 1] for i in range(16)], pos, tokens=toks,
                       logits=logits, next_token=nxt, hidden_out=hid, batch=B, flags=flags)
    torch.cuda.synchronize()
    assert ws.read_device_error() == 0
    return logits.cpu(), nxt.cpu(), hid.cpu(), pos.cpu()


def test_batched_step_matches_oracle(full16):
    f = full16
    kv = f["kv"]
    kv_before = kv.clone()
    logits, nxt, _, _ = batched_step(f)
    kv_after = kv.clone()
    kv.copy_(kv_before)   # later tests start from the prefilled state
    o = f["oracle"]
    for b, n in enumerate(PROMPT_LENS):
        p = n - 1
        cache = [(kv_before[l, 0, b].float().cpu(), kv_before[l, 1, b].float().cpu()) for l in range(16)]
        ref, _ = o.forward(torch.tensor([int(f["prompts"][b][-1])]), p, cache)
        d = (logits[b] - ref[0]).abs()
        say(f"[bstep] seq {b} pos {p}: logits max|d| {d.max():.3e} rms {d.pow(2).mean().sqrt():.3e}; "
            f"argmax gpu {int(nxt[b])} oracle {int(ref[0].argmax())}")
        assert d.max().item() <= STEP_MAX_TOL
        assert d.pow(2).mean().sqrt().item() <= STEP_RMS_TOL
        assert int(nxt[b]) == int(logits[b].argmax())
        # scatter: in every layer only row p of sequence b changed
        changed = (kv_after[:, :, b] != kv_before[:, :, b]).view(16, 2, 8, S, 64).any(-1)   # [16, 2, 8, S]
        rows = changed.any(0).any(0).any(0).nonzero().flatten().tolist()
        assert rows == [p], (b, rows)


def test_batched_step_matches_batch1_kernel(full16):
    import mk_lib
    f = full16
    kv = f["kv"]
    kv_before = kv.clone()
    logits, nxt, hid, _ = batched_step(f)
    kv.copy_(kv_before)
    for b, n in enumerate(PROMPT_LENS):
        pos = torch.tensor([n - 1], dtype=torch.int32, device="cuda")
        tok = torch.tensor([int(f["prompts"][b][-1])], dtype=torch.int32, device="cuda")
        lg = torch.zeros(1, 128256, dtype=torch.float32, device="cuda")
        mk_lib.decode_step(f["w"], f["ws1"], [kv[i, 0, b:b + 1] for i in range(16)],
                           [kv[i, 1, b:b + 1] for i in range(16)], pos, tokens=tok, logits=lg)
        torch.cuda.synchronize()
        d = (logits[b] - lg[0].cpu()).abs()
        say(f"[bstep] seq {b}: batched vs batch-1 kernel logits max|d| {d.max():.3e} rms {d.pow(2).mean().sqrt():.3e}")
        assert d.max().item() <= STEP_MAX_TOL
        assert d.pow(2).mean().sqrt().item() <= STEP_RMS_TOL
    kv.copy_(kv_before)


def test_batched_step_bitwise_repeatable_and_advances(full16):
    import mk_lib
    f = full16
    kv = f["kv"]
    kv_before = kv.clone()
    ws = mk_lib.Workspace(len(PROMPT_LENS), S, torch.device("cuda"))
    outs = []
    for _ in range(2):
        kv.copy_(kv_before)
        logits, nxt, hid, pos = batched_step(f, ws=ws, flags=mk_lib.MK_FLAG_ADVANCE)
        outs.append((logits, nxt, hid, kv.clone()))
        assert pos.tolist() == [n for n in PROMPT_LENS]
    kv.copy_(kv_before)
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[0][2].view(torch.int16), outs[1][2].view(torch.int16))
    assert torch.equal(outs[0][3].view(torch.int16), outs[1][3].view(torch.int16))


def test_batched_step_two_tiles_partial(full16):
    """A full 16-layer step at batch 20: the two-token-tile kernel (batches
    17..32, its own translation unit) with a partial second tile (tokens 16..19;
    rows 20..31 of the tile are MFMA padding). Each sequence's logits against the
    batch-1 kernel's step from the same cache slice and, for two sequences,
    against the oracle; next_token is each row's argmax, and only row pos of each
    sequence's slice changes."""
    import mk_lib
    from mk_weights import random_token_ids
    f = full16
    lens = [3, 17, 40, 9, 25, 1, 60, 12, 33, 5, 48, 21, 2, 70, 14, 8, 29, 55, 6, 41]
    B = len(lens)
    w = f["w"]
    kv = torch.zeros(16, 2, B, 8, S, 64, dtype=torch.bfloat16, device="cuda")
    prompts = [random_token_ids(n, seed=900 + b) for b, n in enumerate(lens)]
    pos1 = torch.zeros(1, dtype=torch.int32, device="cuda")
    tok1 = torch.zeros(1, dtype=torch.int32, device="cuda")
    for b, ids in enumerate(prompts):   # prefill: the batch-1 kernel, one launch per prompt token
        pos1.zero_()
        l = mk_lib.StepLauncher(w, f["ws1"], [kv[i, 0, b:b + 1] for i in range(16)],
                                [kv[i, 1, b:b + 1] for i in range(16)], pos1, tokens=tok1,
                                flags=mk_lib.MK_FLAG_ADVANCE)
        ids_dev = ids.to(device="cuda", dtype=torch.int32)
        for i in range(len(ids) - 1):
            tok1.copy_(ids_dev[i:i + 1])
            l.launch()
    torch.cuda.synchronize()
    assert f["ws1"].read_device_error() == 0
    kv_before = kv.clone()
    ws = mk_lib.Workspace(B, S, torch.device("cuda"))
    pos = torch.tensor([n - 1 for n in lens], dtype=torch.int32, device="cuda")
    toks = torch.tensor([int(p[-1]) for p in prompts], dtype=torch.int32, device="cuda")
    logits = torch.zeros(B, 128256, dtype=torch.float32, device="cuda")
    nxt = torch.full((B,), -5, dtype=torch.int32, device="cuda")
    mk_lib.decode_step(w, ws, [kv[i, 0] for i in range(16)], [kv[i, 1] for i in range(16)], pos, tokens=toks,
                       logits=logits, next_token=nxt, batch=B)
    torch.cuda.synchronize()
    assert ws.read_device_error() == 0
    kv_after = kv.clone()
    logits, nxt = logits.cpu(), nxt.cpu()
    worst = 0.0
    for b, n in enumerate(lens):
        p = n - 1
        assert int(nxt[b]) == int(logits[b].argmax()), b
        changed = (kv_after[:, :, b] != kv_before[:, :, b]).any(-1)   # [16, 2, 8, S]
        assert changed.any(0).any(0).any(0).nonzero().flatten().tolist() == [p], b
        kv[:, :, b].copy_(kv_before[:, :, b])
        pos1.fill_(p)
        tok1.fill_(int(prompts[b][-1]))
        lg = torch.zeros(1, 128256, dtype=torch.float32, device="cuda")
        mk_lib.decode_step(w, f["ws1"], [kv[i, 0, b:b + 1] for i in range(16)], [kv[i, 1, b:b + 1] for i in range(16)],
                           pos1, tokens=tok1, logits=lg)
        torch.cuda.synchronize()
        d = (logits[b] - lg[0].cpu()).abs()
        worst = max(worst, d.max().item())
        assert d.max().item() <= STEP_MAX_TOL and d.pow(2).mean().sqrt().item() <= STEP_RMS_TOL, b
    o = f["oracle"]
    for b in (6, 19):   # one row of each token tile against the oracle
        p = lens[b] - 1
        cache = [(kv_before[l, 0, b].float().cpu(), kv_before[l, 1, b].float().cpu()) for l in range(16)]
        ref, _ = o.forward(torch.tensor([int(prompts[b][-1])]), p, cache)
        d = (logits[b] - ref[0]).abs()
        say(f"[bstep] batch 20, seq {b} pos {p}: oracle max|d| {d.max():.3e} rms {d.pow(2).mean().sqrt():.3e}")
        assert d.max().item() <= STEP_MAX_TOL and d.pow(2).mean().sqrt().item() <= STEP_RMS_TOL, b
    say(f"[bstep] batch 20 (two tiles): worst max|d| against the batch-1 kernel {worst:.3e}")
