"""GPU parity at long KV lengths: attention items that span several full
128-row groups, so the online softmax rescales across groups.

The other layer tests use 256-row caches (batched) and the C3 trajectory
splits 1024 rows over 8 items of at most 128 rows, so each of their items is
one group. Here the caches hold 4096 rows and the positions reach 4095:
  * batch-1 kernel (``mk_decode_kernel``): 8 splits of up to 512 rows, four
    full groups per item;
  * batched kernel (``mk_batch_kernel``): items sized from all sequences'
    lengths, 128-row multiples, several groups each, ragged lengths.
Same bounds as the 256-row layer tests: elementwise within 2^-5 of the
operands' scale, rms(GPU - oracle) within 1.5x the oracle's own bf16-vs-fp64
departure, and the K/V scatter position-exact, bit for bit outside row pos.
"""

import os

import pytest
import torch

from gpu_common import bf16_ulp, need_gpu, packed_on_device, say

pytestmark = pytest.mark.gpu

S = 4096


@pytest.fixture(scope="module")
def layer_long():
    need_gpu()
    from mk_config import LlamaDims
    from mk_weights import synthetic_state_dict
    from oracle.llama_ref import Dims, OracleLlama
    torch.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    dp = LlamaDims(n_layers=1)
    sd = synthetic_state_dict(seed=3, d=dp)
    packed = packed_on_device(sd, dp, rope_rows=S)
    d = Dims(n_layers=1)
    return packed, OracleLlama(sd, d, mode="mk"), OracleLlama(sd, d, mode="exact")


def run_layer(packed, hidden, kc, vc, pos_list, ws_batch):
    import mk_lib
    B = len(pos_list)
    w = mk_lib.weights_struct(packed)
    ws = mk_lib.Workspace(ws_batch, S, torch.device("cuda"))
    pos = torch.tensor(pos_list, dtype=torch.int32, device="cuda")
    out = torch.empty(B, 2048, dtype=torch.bfloat16, device="cuda")
    mk_lib.decode_step(w, ws, [kc], [vc], pos, hidden_in=hidden, hidden_out=out, n_layers=1, batch=B)
    torch.cuda.synchronize()
    return out, ws


@pytest.mark.parametrize("pos_list,ws_batch", [
    ([4095], 1),                      # batch-1 kernel: 8 items of 512 rows (4 full groups each)
    ([2000], 1),                      # batch-1 kernel: items of 224-256 rows (7-8 groups of 32)
    ([4095, 600, 2047, 3071], 4),     # batched kernel, ragged
    ([1500, 4095, 129, 3333, 2600, 4000, 700, 3900], 8),
])
def test_long_context_layer_matches_oracle(layer_long, pos_list, ws_batch):
    packed, o_mk, o_exact = layer_long
    B = len(pos_list)
    say(f"[long] ws_batch={ws_batch} pos={pos_list}")
    g = torch.Generator().manual_seed(77 + sum(pos_list))
    hidden = torch.randn(B, 2048, generator=g).to(torch.bfloat16)
    k0 = torch.randn(B, 8, S, 64, generator=g).to(torch.bfloat16)
    v0 = torch.randn(B, 8, S, 64, generator=g).to(torch.bfloat16)
    kc, vc = k0.cuda(), v0.cuda()
    out, ws = run_layer(packed, hidden.cuda(), kc, vc, pos_list, ws_batch)
    assert ws.read_device_error() == 0
    got_all, k1, v1 = out.cpu().float(), kc.cpu(), vc.cpu()
    worst_ratio = 0.0
    for b, p in enumerate(pos_list):
        cache = [(k0[b].float().clone(), v0[b].float().clone())]
        _, ref = o_mk.forward(None, p, cache, hidden=hidden[b:b + 1].float(), want_logits=False)
        _, exact = o_exact.forward(None, p, [(k0[b].double(), v0[b].double())], hidden=hidden[b:b + 1].double(),
                                   want_logits=False)
        ref, exact = ref[0], exact[0]
        got = got_all[b]
        diff = (got - ref).abs()
        scale = torch.maximum(ref.abs(), hidden[b].float().abs()).clamp_min(1.0)
        assert torch.all(diff <= 2.0 ** -5 * scale), (b, p, diff.max().item())
        rms_gpu = (got.double() - ref.double()).pow(2).mean().sqrt().item()
        rms_bf16 = (ref.double() - exact).pow(2).mean().sqrt().item()
        worst_ratio = max(worst_ratio, rms_gpu / max(rms_bf16, 1e-12))
        assert rms_gpu <= 1.5 * rms_bf16 + 1e-6, (b, p, rms_gpu, rms_bf16)
        mask = torch.ones(S, dtype=torch.bool)
        mask[p] = False
        assert torch.equal(k1[b][:, mask].view(torch.int16), k0[b][:, mask].view(torch.int16)), (b, p)
        assert torch.equal(v1[b][:, mask].view(torch.int16), v0[b][:, mask].view(torch.int16)), (b, p)
        # V: the projection rounded once, within 1 bf16 ulp. K: after RoPE,
        # bf16(bf16(a*cos) + bf16(-b*sin)); where the two terms nearly cancel,
        # one ulp of a term (from the projection's fp32 summation order) is
        # two ulps of the result, so K is held to 2 ulps.
        for got_row, ref_row, ulps in ((k1[b][:, p].float(), cache[0][0][:, p], 2),
                                       (v1[b][:, p].float(), cache[0][1][:, p], 1)):
            dd = (got_row - ref_row).abs()
            assert torch.all(dd <= ulps * bf16_ulp(ref_row) + 1e-6), (b, p, ulps)
            assert (dd > 0).float().mean().item() < 0.05, (b, p)
    say(f"[long] ws_batch={ws_batch}: worst rms ratio vs bf16 floor {worst_ratio:.2f}")


# ---------------------------------------------------------------------------
# The C5 shape: batch 32 over 8192-row caches (``mk_batch_kernel<2>``: two
# 16-token MFMA tiles; every (sequence, kv head) one attention item of up to
# 64 groups whose output is written directly, no split merge), MFMA-tiled
# weights as the benchmark runs them. Positions: the last 128 rows of the
# cache (the C5 bench's range), the cache's last row, and ragged ones down to 0.
# ---------------------------------------------------------------------------

S5 = 8192
C5_POSITIONS = ([8191, 8190, 8189, 8160, 8128, 8127, 8100, 8064] + list(range(8065, 8192, 8))[:16]
                + [0, 1, 127, 128, 129, 4095, 6000, 7000])


@pytest.fixture(scope="module")
def layer_c5():
    need_gpu()
    import mk_lib
    from mk_config import LlamaDims
    from mk_weights import synthetic_state_dict
    from oracle.llama_ref import Dims, OracleLlama
    torch.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    dp = LlamaDims(n_layers=1)
    sd = synthetic_state_dict(seed=5, d=dp)
    packed = packed_on_device(sd, dp, rope_rows=S5)
    assert all(k in packed for k in mk_lib.TILED_KEYS)
    d = Dims(n_layers=1)
    return packed, OracleLlama(sd, d, mode="mk"), OracleLlama(sd, d, mode="exact")


def test_c5_shape_layer_matches_oracle(layer_c5):
    import mk_lib
    packed, o_mk, o_exact = layer_c5
    pos_list = C5_POSITIONS
    B = len(pos_list)
    assert B == 32 and len(set(pos_list)) == 32
    say(f"[long] C5 shape: batch {B}, s_max {S5}, positions {min(pos_list)}..{max(pos_list)}")
    g = torch.Generator().manual_seed(5)
    hidden = torch.randn(B, 2048, generator=g).to(torch.bfloat16)
    gd = torch.Generator(device="cuda").manual_seed(55)
    kc = torch.empty(B, 8, S5, 64, dtype=torch.bfloat16, device="cuda").normal_(generator=gd)
    vc = torch.empty(B, 8, S5, 64, dtype=torch.bfloat16, device="cuda").normal_(generator=gd)
    k0, v0 = kc.cpu(), vc.cpu()
    w = mk_lib.weights_struct(packed)
    ws = mk_lib.Workspace(B, S5, torch.device("cuda"))
    pos = torch.tensor(pos_list, dtype=torch.int32, device="cuda")
    out = torch.empty(B, 2048, dtype=torch.bfloat16, device="cuda")
    mk_lib.decode_step(w, ws, [kc], [vc], pos, hidden_in=hidden.cuda(), hidden_out=out, n_layers=1, batch=B)
    torch.cuda.synchronize()
    assert ws.read_device_error() == 0
    got_all = out.cpu().float()
    # position-exact scatter over the whole batch: the changed (sequence, row) pairs
    ch = ((kc.cpu() != k0).any(-1) | (vc.cpu() != v0).any(-1)).any(1)       # [B, S]
    assert ch.nonzero().tolist() == [[b, p] for b, p in enumerate(pos_list)]
    k1, v1 = kc.cpu(), vc.cpu()
    worst_ratio, worst_ulps = 0.0, 0.0
    for b, p in enumerate(pos_list):
        cache = [(k0[b].float().clone(), v0[b].float().clone())]
        _, ref = o_mk.forward(None, p, cache, hidden=hidden[b:b + 1].float(), want_logits=False)
        _, exact = o_exact.forward(None, p, [(k0[b].double(), v0[b].double())], hidden=hidden[b:b + 1].double(),
                                   want_logits=False)
        ref, exact = ref[0], exact[0]
        diff = (got_all[b] - ref).abs()
        scale = torch.maximum(ref.abs(), hidden[b].float().abs()).clamp_min(1.0)
        assert torch.all(diff <= 2.0 ** -5 * scale), (b, p, diff.max().item())
        worst_ulps = max(worst_ulps, (diff / scale).max().item() * 2 ** 8)
        rms_gpu = (got_all[b].double() - ref.double()).pow(2).mean().sqrt().item()
        rms_bf16 = (ref.double() - exact).pow(2).mean().sqrt().item()
        worst_ratio = max(worst_ratio, rms_gpu / max(rms_bf16, 1e-12))
        assert rms_gpu <= 1.5 * rms_bf16 + 1e-6, (b, p, rms_gpu, rms_bf16)
        for got_row, ref_row, ulps in ((k1[b][:, p].float(), cache[0][0][:, p], 2),
                                       (v1[b][:, p].float(), cache[0][1][:, p], 1)):
            dd = (got_row - ref_row).abs()
            assert torch.all(dd <= ulps * bf16_ulp(ref_row) + 1e-6), (b, p, ulps)
            assert (dd > 0).float().mean().item() < 0.05, (b, p)
    say(f"[long] C5 shape: worst rms ratio vs bf16 floor {worst_ratio:.2f}, worst |d| {worst_ulps:.2f} / 256 of scale")
    from gpu_common import record_parity
    record_parity("c5_layer", {"config": "C5 shape, one layer", "batch": B, "s_max": S5, "positions": pos_list,
                               "worst_rms_ratio_vs_bf16_floor": round(worst_ratio, 3),
                               "worst_abs_diff_in_256ths_of_scale": round(worst_ulps, 3),
                               "tolerances": {"elementwise": "2^-5 * max(|ref|, |hidden|, 1)",
                                              "rms_vs_floor": 1.5, "k_row_ulps": 2, "v_row_ulps": 1}})
