"""GPU parity of one fused decoder layer (BASELINE config 2 shapes) against the oracle.

Layer 0 of seed-0 synthetic weights, hidden ~ N(0,1), K/V cache [1,8,1024,64]
bf16 ~ N(0,1), pos = 1023 and a few other positions (384 and 900: eight KV
splits of unequal sizes, 1-2 and 3-4 groups of 32 rows), run through
``mk_layer_step`` / ``mk_decode_step`` in libmk.so and compared with
``OracleLlama`` in "mk" mode (same bf16 rounding points, fp32 accumulation):

* output hidden within 2^-6 * max(|ref|, 1) elementwise (a few bf16 ulps:
  summation order differs, so intermediates may round to the neighbouring
  bf16, and the kernel's split-K softmax keeps p in fp32), and the rms of the
  GPU-oracle difference no larger than 1.5x the rms by which the bf16 oracle
  itself departs from float64 math ("exact" mode) on the same inputs;
* the K/V scatter is position-exact: every cache byte outside row ``pos`` of
  each kv head is unchanged, and the written rows match the oracle's
  RoPE'd K and V within 1 bf16 ulp (almost all bit-exact);
* two runs give bitwise identical results;
* an out-of-range position is refused on the device (error bit, no writes).
"""

import pytest
import torch

from gpu_common import bf16_ulp, need_gpu, new_caches, packed_on_device, say

pytestmark = pytest.mark.gpu

S = 1024


@pytest.fixture(scope="module")
def layer_setup():
    need_gpu()
    from mk_config import LlamaDims
    from mk_weights import synthetic_state_dict
    from oracle.llama_ref import Dims
    dp = LlamaDims(n_layers=1)
    sd = synthetic_state_dict(seed=0, d=dp)
    packed = packed_on_device(sd, dp, rope_rows=S)
    return sd, packed, Dims(n_layers=1)


def run_layer(packed, hidden, kc, vc, pos_val, ws=None):
    import mk_lib
    w = mk_lib.weights_struct(packed)
    if ws is None:
        ws = mk_lib.Workspace(1, S, torch.device("cuda"))
    pos = torch.tensor([pos_val], dtype=torch.int32, device="cuda")
    out = torch.empty(1, 2048, dtype=torch.bfloat16, device="cuda")
    mk_lib.decode_step(w, ws, kc, vc, pos, hidden_in=hidden, hidden_out=out, n_layers=1)
    torch.cuda.synchronize()
    return out, ws


def oracle_layer(sd, d, hidden_cpu, k0, v0, pos_val, mode="mk"):
    from oracle.llama_ref import OracleLlama
    o = OracleLlama(sd, d, mode=mode)
    dt = o.dt
    cache = [(k0[0].to(dt).clone(), v0[0].to(dt).clone())]
    _, h = o.forward(None, pos_val, cache, hidden=hidden_cpu.to(dt), want_logits=False)
    return h, cache


@pytest.mark.parametrize("pos_val", [1023, 0, 63, 64, 500, 384, 900])
def test_layer_matches_oracle(layer_setup, pos_val):
    sd, packed, d = layer_setup
    say(f"[layer] pos={pos_val}")
    g = torch.Generator().manual_seed(100 + pos_val)
    hidden = torch.randn(1, 2048, generator=g).to(torch.bfloat16)
    kc, vc = new_caches(1, S, fill="randn", seed=pos_val)
    k0, v0 = kc[0].cpu(), vc[0].cpu()
    out, ws = run_layer(packed, hidden.cuda(), kc, vc, pos_val)
    assert ws.read_device_error() == 0
    ref, cache = oracle_layer(sd, d, hidden, k0, v0, pos_val)
    got = out.cpu().float()
    diff = (got - ref).abs()
    ulp = bf16_ulp(ref)
    say(f"[layer] pos={pos_val} max|d|={diff.max().item():.3e} max ulps={(diff / ulp).max().item():.2f} "
        f"frac!=0: {(diff > 0).float().mean().item():.4f}")
    assert torch.all(diff <= 2.0 ** -6 * ref.abs().clamp_min(1.0))
    exact, _ = oracle_layer(sd, d, hidden, k0, v0, pos_val, mode="exact")
    rms_gpu = (got.double() - ref.double()).pow(2).mean().sqrt().item()
    rms_bf16 = (ref.double() - exact).pow(2).mean().sqrt().item()
    say(f"[layer] pos={pos_val} rms(gpu-mk)={rms_gpu:.3e} rms(mk-exact)={rms_bf16:.3e}")
    assert rms_gpu <= 1.5 * rms_bf16 + 1e-6

    # scatter: only row pos changed, in every kv head
    k1, v1 = kc[0].cpu(), vc[0].cpu()
    mask = torch.ones(S, dtype=torch.bool)
    mask[pos_val] = False
    assert torch.equal(k1[0][:, mask].view(torch.int16), k0[0][:, mask].view(torch.int16))
    assert torch.equal(v1[0][:, mask].view(torch.int16), v0[0][:, mask].view(torch.int16))
    kr_ref, vr_ref = cache[0][0][:, pos_val], cache[0][1][:, pos_val]
    for got_row, ref_row in ((k1[0][:, pos_val].float(), kr_ref), (v1[0][:, pos_val].float(), vr_ref)):
        dd = (got_row - ref_row).abs()
        assert torch.all(dd <= bf16_ulp(ref_row) + 1e-6)
        assert (dd > 0).float().mean().item() < 0.05


def test_layer_is_deterministic(layer_setup):
    sd, packed, d = layer_setup
    hidden = torch.randn(1, 2048, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).cuda()
    outs, caches = [], []
    for _ in range(2):
        kc, vc = new_caches(1, S, fill="randn", seed=3)
        out, _ = run_layer(packed, hidden, kc, vc, 777)
        outs.append(out.cpu())
        caches.append((kc[0].cpu(), vc[0].cpu()))
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert torch.equal(caches[0][0].view(torch.int16), caches[1][0].view(torch.int16))
    assert torch.equal(caches[0][1].view(torch.int16), caches[1][1].view(torch.int16))


def test_out_of_range_position_is_refused_on_device(layer_setup):
    sd, packed, d = layer_setup
    hidden = torch.randn(1, 2048, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).cuda()
    kc, vc = new_caches(1, S, fill="randn", seed=4)
    k0 = kc[0].clone()
    import mk_lib
    w = mk_lib.weights_struct(packed)
    ws = mk_lib.Workspace(1, S, torch.device("cuda"))
    pos = torch.tensor([S], dtype=torch.int32, device="cuda")
    out = torch.full((1, 2048), 7.0, dtype=torch.bfloat16, device="cuda")
    mk_lib.decode_step(w, ws, kc, vc, pos, hidden_in=hidden, hidden_out=out, n_layers=1)
    bits = ws.read_device_error()
    assert bits & mk_lib.MK_DEVERR_POS
    assert torch.equal(kc[0].view(torch.int16), k0.view(torch.int16))
    assert torch.all(out.float() == 7.0)
    assert ws.read_device_error() == 0   # cleared
    # the workspace is still usable afterwards
    out2, _ = run_layer(packed, hidden, kc, vc, 5, ws=ws)
    assert ws.read_device_error() == 0
