"""GPU parity of the prefill (context-encoding) paths.

The reference encodes the prompt with its baseline layer path before the
megakernel takes over token generation (llama_with_megakernel.py:194-204;
NxDI's context-encoding model). This build has three ways to do it:

* "layers" (``mk_prefill``, the default): layer by layer on the matrix cores,
  every layer's weights streamed once per chunk of prompt tokens;
* "chunks": launches of the batched decode kernel with MK_FLAG_PREFILL over
  up to 32 consecutive tokens of one sequence sharing one cache (token b
  attends to cache rows [0, pos[b]), including the rows the chunk's earlier
  tokens write in the same launch);
* "tokens": one decode-megakernel launch per prompt token.

Checks (70-token prompt, S = 256):

* K/V rows written = exactly rows 0..n-2 of every layer and kv head; the rest
  of the cache keeps its bytes (a N(0,1) pattern);
* the written rows against the CPU oracle's prefill of the same tokens
  ("mk" rounding): layer 0 within 1 bf16 ulp for V and 2 for K after RoPE
  (its input is the embedding row, the same for every implementation; a
  cancelling RoPE sum turns one ulp of a term into two), every layer's rows within an rms
  of 4% of the rows' own rms and a max-abs of 5% of their max |value|: the
  bf16 rounding noise that the deeper layers accumulate along independently
  rounded trajectories (the token-by-token path sits at 2.05% rms at its
  worst layer, max-abs 0.10 on K values of a few units; the decode tests allow
  5% for a fresh row computed from the same state);
* the first decode step from the prefilled cache: logits within the
  trajectory bound of the decode tests (max-abs 0.2) of the oracle's step from
  the oracle's own cache, and within the per-step bounds (0.15 / 0.03) of the
  oracle's step from the GPU's cache;
* the three paths agree within the same bounds;
* "layers": the hidden state after the last layer (``hidden_out``) within the
  same relative bounds of the oracle's; chunked runs (a workspace for 32
  tokens, and a call continued at start_pos 40) equal the one-chunk run bit
  for bit (each token's rows depend only on its own row of every GEMM and on
  the keys in the same order);
* bitwise repeatability; non-consecutive positions refused as a whole
  (MK_DEVERR_PREFILL, nothing written); MK_FLAG_PREFILL on a batch-1
  workspace refused with MK_ERR_UNSUPPORTED.
"""

import os

import pytest
import torch

from gpu_common import bf16_ulp, need_gpu, say

pytestmark = pytest.mark.gpu

S = 256
N_PROMPT = 70
STEP_MAX_TOL = 0.15
STEP_RMS_TOL = 0.03
TRAJ_TOL = 0.2
KV_RMS_REL = 0.04
KV_MAX_REL = 0.05


@pytest.fixture(scope="module")
def setup():
    need_gpu()
    from llama_with_megakernel import LlamaInferenceConfig, NeuronConfigLlamaMK, NeuronLlamaForCausalLM
    from mk_weights import random_token_ids
    from oracle.llama_ref import OracleLlama
    torch.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    cfg = LlamaInferenceConfig(NeuronConfigLlamaMK(seq_len=S, max_context_length=S))
    model = NeuronLlamaForCausalLM("random:0", cfg)
    model.compile()
    model.load()
    ids = random_token_ids(N_PROMPT, seed=21)
    oracle = OracleLlama(model.state_dict_bf16, mode="mk")
    ocache = oracle.new_cache(S)
    oracle.forward(ids[:N_PROMPT - 1], 0, ocache, want_logits=False)   # rows 0..n-2
    ref_logits, _ = oracle.forward(ids[N_PROMPT - 1:], N_PROMPT - 1, ocache)
    return dict(model=model, ids=ids, oracle=oracle, ocache=ocache, ref_logits=ref_logits[0])


def fill_pattern(model):
    g = torch.Generator(device="cuda").manual_seed(7)
    model.kv.normal_(generator=g)
    return model.kv.clone()


def kv_rows_vs_oracle(model, ocache, n_rows, tag):
    worst = 0.0
    for l in range(16):
        for j, name in ((0, "K"), (1, "V")):
            got = model.kv[l, j, 0, :, :n_rows].float().cpu()
            ref = ocache[l][j][:, :n_rows].float()
            d = (got - ref).abs()
            rel = (d.pow(2).mean().sqrt() / ref.pow(2).mean().sqrt()).item()
            worst = max(worst, rel)
            if l == 0:
                # V: the projection rounded once, within 1 ulp. K: after RoPE,
                # bf16(bf16(a*cos) + bf16(-b*sin)); where the two terms nearly
                # cancel, one ulp of a term is two of the result (as in the decode tests)
                ulps = 2.0 if name == "K" else 1.0
                ratio = d / (bf16_ulp(ref) + 1e-6)
                say(f"[prefill] {tag}: layer 0 {name}: max |d|/ulp {ratio.max():.2f}, "
                    f"> 1 ulp at {(ratio > 1).float().mean():.2e}, nonzero at {(d > 0).float().mean():.2e}")
                assert (d <= ulps * bf16_ulp(ref) + 1e-6).all(), f"{tag}: layer 0 {name} beyond {ulps} ulp"
                assert (d > 0).float().mean().item() < 0.05, f"{tag}: layer 0 {name}"
            assert rel <= KV_RMS_REL, f"{tag}: layer {l} {name} rms rel {rel:.3e}"
            assert d.max().item() <= KV_MAX_REL * ref.abs().max().item(), f"{tag}: layer {l} {name} max|d| {d.max():.3e}"
    say(f"[prefill] {tag}: K/V rows 0..{n_rows - 1} vs oracle, worst rms rel {worst:.3e}")


@pytest.mark.parametrize("method", ["layers", "chunks"])
def test_prefill_writes_exactly_the_prompt_rows(setup, method):
    m = setup["model"]
    before = fill_pattern(m)
    m.prefill(setup["ids"], method=method)
    torch.cuda.synchronize()
    assert m.prefill_device_error() == 0
    assert int(m.pos.item()) == N_PROMPT - 1
    assert int(m.tokens.item()) == int(setup["ids"][-1])
    changed = (m.kv != before).view(16, 2, 8, S, 64).any(-1).any(0).any(0).any(0)
    rows = changed.nonzero().flatten().tolist()
    assert rows == list(range(N_PROMPT - 1)), rows[:8]
    untouched = m.kv[:, :, :, :, N_PROMPT - 1:]
    assert torch.equal(untouched.view(torch.int16), before[:, :, :, :, N_PROMPT - 1:].view(torch.int16))


@pytest.mark.parametrize("method", ["layers", "chunks", "tokens"])
def test_prefill_matches_oracle(setup, method):
    m = setup["model"]
    m.kv.zero_()
    m.prefill(setup["ids"], method=method)
    torch.cuda.synchronize()
    assert m.prefill_device_error() == 0
    tag = method
    kv_rows_vs_oracle(m, setup["ocache"], N_PROMPT - 1, tag)
    m.launcher("decode").launch()
    torch.cuda.synchronize()
    assert m.ws.read_device_error() == 0
    lg = m.logits[0].cpu()
    d = (lg - setup["ref_logits"]).abs()
    say(f"[prefill] {tag}: first decode step vs oracle trajectory: max|d| {d.max():.3e} "
        f"rms {d.pow(2).mean().sqrt():.3e}; argmax gpu {int(lg.argmax())} oracle {int(setup['ref_logits'].argmax())}")
    assert d.max().item() <= TRAJ_TOL
    # same state: the oracle's step from the GPU's own cache
    cache = [(m.kv[l, 0, 0].float().cpu(), m.kv[l, 1, 0].float().cpu()) for l in range(16)]
    ref = setup["oracle"].forward(torch.tensor([int(setup["ids"][-1])]), N_PROMPT - 1, cache)[0][0]
    d = (lg - ref).abs()
    say(f"[prefill] {tag}: step vs oracle from the GPU cache: max|d| {d.max():.3e} rms {d.pow(2).mean().sqrt():.3e}")
    assert d.max().item() <= STEP_MAX_TOL
    assert d.pow(2).mean().sqrt().item() <= STEP_RMS_TOL


@pytest.mark.parametrize("method", ["layers", "chunks"])
def test_prefill_matches_token_by_token(setup, method):
    m = setup["model"]
    m.kv.zero_()
    m.prefill(setup["ids"], method="tokens")
    torch.cuda.synchronize()
    kv_step = m.kv[:, :, 0, :, :N_PROMPT - 1].float().clone()
    m.kv.zero_()
    m.prefill(setup["ids"], method=method)
    torch.cuda.synchronize()
    kv_b = m.kv[:, :, 0, :, :N_PROMPT - 1].float()
    for l in range(16):
        d = (kv_b[l] - kv_step[l]).abs()
        rel = (d.pow(2).mean().sqrt() / kv_step[l].pow(2).mean().sqrt()).item()
        assert rel <= KV_RMS_REL and d.max().item() <= KV_MAX_REL * kv_step[l].abs().max().item(), (l, rel)
    say(f"[prefill] {method} vs token-by-token K/V: layer 15 rms rel "
        f"{((kv_b[15] - kv_step[15]).pow(2).mean().sqrt() / kv_step[15].pow(2).mean().sqrt()).item():.3e}")


@pytest.mark.parametrize("method", ["layers", "chunks"])
def test_prefill_is_bitwise_repeatable(setup, method):
    m = setup["model"]
    outs = []
    for _ in range(2):
        m.kv.zero_()
        m.prefill(setup["ids"], method=method)
        torch.cuda.synchronize()
        outs.append(m.kv.clone())
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def test_layers_prefill_chunking_and_hidden_state(setup):
    """mk_prefill over the whole prompt: hidden_out against the oracle; chunks
    of 32 tokens and a continuation at start_pos 40 equal one chunk bit for bit."""
    import mk_lib
    m = setup["model"]
    n = N_PROMPT
    toks = setup["ids"].to(device="cuda", dtype=torch.int32)
    kc, vc = m.seq_caches(0)
    big = mk_lib.prefill_workspace(256, "cuda")
    hid = torch.empty(n, 2048, dtype=torch.bfloat16, device="cuda")
    m.kv.zero_()
    mk_lib.prefill(m.weights, toks, kc, vc, 0, big, hidden_out=hid)
    torch.cuda.synchronize()
    one = m.kv.clone()
    # the hidden state of every prompt token after the last layer, against the oracle's
    o = setup["oracle"]
    _, ref_h = o.forward(setup["ids"], 0, o.new_cache(S), want_logits=False)
    got_h = hid.float().cpu()
    d = (got_h - ref_h).abs()
    rel = (d.pow(2).mean().sqrt() / ref_h.pow(2).mean().sqrt()).item()
    say(f"[prefill] layers: hidden_out vs oracle rms rel {rel:.3e}, max|d| {d.max():.3e} "
        f"(max |h| {ref_h.abs().max():.2f})")
    assert rel <= KV_RMS_REL and d.max().item() <= KV_MAX_REL * ref_h.abs().max().item()
    # 32-token chunks (a workspace for 32 tokens)
    small = mk_lib.prefill_workspace(32, "cuda")
    m.kv.zero_()
    mk_lib.prefill(m.weights, toks, kc, vc, 0, small)
    torch.cuda.synchronize()
    assert torch.equal(m.kv.view(torch.int16), one.view(torch.int16))
    # two calls: tokens 0..39, then 40..69 from start_pos 40
    m.kv.zero_()
    mk_lib.prefill(m.weights, toks[:40], kc, vc, 0, big)
    mk_lib.prefill(m.weights, toks[40:].contiguous(), kc, vc, 40, big)
    torch.cuda.synchronize()
    assert torch.equal(m.kv.view(torch.int16), one.view(torch.int16))


def test_prefill_refuses_non_consecutive_positions(setup):
    import mk_lib
    m = setup["model"]
    before = fill_pattern(m)
    if m.pf_ws is None:
        m.pf_ws = mk_lib.Workspace(mk_lib.PREFILL_CHUNK, m.s_max, m.pos.device)
    pos = torch.tensor([3, 4, 6, 7], dtype=torch.int32, device="cuda")
    toks = setup["ids"][:4].to(device="cuda", dtype=torch.int32)
    mk_lib.decode_step(m.weights, m.pf_ws, m.k_caches, m.v_caches, pos, tokens=toks, flags=mk_lib.MK_FLAG_PREFILL,
                       batch=4)
    torch.cuda.synchronize()
    bits = m.pf_ws.read_device_error()
    assert bits & mk_lib.MK_DEVERR_PREFILL, bits
    assert torch.equal(m.kv.view(torch.int16), before.view(torch.int16))


def test_prefill_flag_needs_batched_workspace(setup):
    import mk_lib
    m = setup["model"]
    pos = torch.tensor([0], dtype=torch.int32, device="cuda")
    toks = setup["ids"][:1].to(device="cuda", dtype=torch.int32)
    with pytest.raises(mk_lib.MkError) as e:
        mk_lib.decode_step(m.weights, m.ws, m.k_caches, m.v_caches, pos, tokens=toks, flags=mk_lib.MK_FLAG_PREFILL,
                           batch=1)
    assert e.value.code == -4


@pytest.mark.timeout(300)
@pytest.mark.parametrize("n", [200, 383, 1500])
def test_layers_prefill_matches_chunks(n):
    """Prompts whose "layers" prefill takes each GEMM path: 200 tokens (the QKV
    projection split over K in 4 parts, O and down in 8), 383 (QKV in 2, O and
    down in 4), 1500 (12 row tiles of 128 tokens occupy the device: every
    projection unsplit, the residual add in the GEMM epilogue). Their K/V rows
    agree with the "chunks" method's within the same relative bounds as the
    70-token prompt's against the oracle, and so does the first decode step
    from each cache (per-step bounds)."""
    from llama_with_megakernel import LlamaInferenceConfig, NeuronConfigLlamaMK, NeuronLlamaForCausalLM
    from mk_weights import random_token_ids
    S2 = 2048
    cfg = LlamaInferenceConfig(NeuronConfigLlamaMK(seq_len=S2, max_context_length=S2))
    m = NeuronLlamaForCausalLM("random:0", cfg)
    m.compile()
    m.load()
    ids = random_token_ids(n, seed=33)
    res = {}
    for method in ("chunks", "layers"):
        m.kv.zero_()
        m.prefill(ids, method=method)
        m.launcher("decode_logits").launch()
        torch.cuda.synchronize()
        assert m.prefill_device_error() == 0 and m.ws.read_device_error() == 0
        res[method] = (m.kv[:, :, 0, :, :n - 1].float().clone(), m.logits[0].cpu().clone())
    (kv_c, lg_c), (kv_l, lg_l) = res["chunks"], res["layers"]
    worst = 0.0
    for l in range(16):
        d = (kv_l[l] - kv_c[l]).abs()
        rel = (d.pow(2).mean().sqrt() / kv_c[l].pow(2).mean().sqrt()).item()
        worst = max(worst, rel)
        assert rel <= KV_RMS_REL and d.max().item() <= KV_MAX_REL * kv_c[l].abs().max().item(), (l, rel)
    d = (lg_l - lg_c).abs()
    say(f"[prefill] {n} tokens, layers vs chunks: K/V worst rms rel {worst:.3e}; first step logits "
        f"max|d| {d.max():.3e} rms {d.pow(2).mean().sqrt():.3e}")
    assert d.max().item() <= STEP_MAX_TOL and d.pow(2).mean().sqrt().item() <= STEP_RMS_TOL
