"""The allocation-free decode step (``mk_decode_step_noalloc``) against ``mk_decode_step``.

Both run the batch-1 megakernel; the allocation-free entry point keeps the
kernel's control block and exchange sets in the library's static scratch
instead of a caller workspace plus an exchange area that ``mk_workspace_init``
allocates. From the same inputs the two give bit-identical results: the fp32
logits, the greedy next token, the hidden state after the last layer, every
K/V cache byte (the fresh rows written at ``pos`` and nothing else) and the
advanced position. Checked on consecutive calls that share the scratch:

1. a 512-row cache at position 300 (token input, lm_head);
2. a smaller input right after it: a 64-row cache at position 17;
3. the layer-stack seam (hidden state in, no lm_head) at position 5;
4. a step with the position out of range (forced from the host): nothing is
   written, next_token reads -1 and the position does not advance;
5. the first input again: equal to call 1's results, so every earlier call
   (the refused one included) left the scratch ready;
6. a refused step without next_token (the layer-stack seam): its fault is in
   the sticky error word that mk_read_device_error(NULL, ...) returns.

The first test runs before any eager allocation-free call of the process: it
captures three allocation-free steps into a HIP graph on a side stream (so the
scratch's first fill is recorded into the graph, and the library fills again
on the next eager call), replays it twice and compares each replay bit for
bit with three mk_decode_step steps from the same inputs, then checks that an
eager allocation-free call after the capture is still bit-exact.
"""

import pytest
import torch

from gpu_common import need_gpu, packed_on_device, say

pytestmark = pytest.mark.gpu

VOCAB = 128256


@pytest.fixture(scope="module")
def packed2():
    need_gpu()
    from mk_config import LlamaDims
    from mk_weights import synthetic_state_dict
    dp = LlamaDims(n_layers=2)
    sd = synthetic_state_dict(seed=0, d=dp)
    return packed_on_device(sd, dp, rope_rows=512)


def make_case(s_max, pos, seed, token=None):
    g = torch.Generator().manual_seed(seed)
    ks = [torch.randn(1, 8, s_max, 64, generator=g).to(torch.bfloat16) for _ in range(2)]
    vs = [torch.randn(1, 8, s_max, 64, generator=g).to(torch.bfloat16) for _ in range(2)]
    hidden = torch.randn(1, 2048, generator=g).to(torch.bfloat16)
    return dict(s_max=s_max, pos=pos, ks=ks, vs=vs, token=token, hidden=hidden)


def run(packed, case, noalloc, ws=None):
    """One step from the case's inputs (fresh device copies); returns the outputs on the CPU."""
    import mk_lib
    w = mk_lib.weights_struct(packed)
    ks = [k.cuda() for k in case["ks"]]
    vs = [v.cuda() for v in case["vs"]]
    pos = torch.tensor([case["pos"]], dtype=torch.int32, device="cuda")
    hid = torch.zeros(1, 2048, dtype=torch.bfloat16, device="cuda")
    kw = dict(hidden_out=hid, flags=mk_lib.MK_FLAG_ADVANCE)
    logits = nxt = None
    if case["token"] is not None:
        kw["tokens"] = torch.tensor([case["token"]], dtype=torch.int32, device="cuda")
        logits = torch.full((1, VOCAB), float("nan"), dtype=torch.float32, device="cuda")
        nxt = torch.full((1,), -7, dtype=torch.int32, device="cuda")
        kw.update(logits=logits, next_token=nxt)
    else:
        kw["hidden_in"] = case["hidden"].cuda()
    if noalloc:
        mk_lib.decode_step_noalloc(w, ks, vs, pos, **kw)
    else:
        mk_lib.decode_step(w, ws, ks, vs, pos, **kw)
    torch.cuda.synchronize()
    out = dict(hidden=hid.cpu().view(torch.int16), pos=pos.cpu(),
               k=[k.cpu().view(torch.int16) for k in ks], v=[v.cpu().view(torch.int16) for v in vs])
    if logits is not None:
        out.update(logits=logits.cpu().view(torch.int32), next=nxt.cpu())
    return out


def assert_same(a, b, what):
    assert a.keys() == b.keys()
    for key in a:
        if isinstance(a[key], list):
            for l, (x, y) in enumerate(zip(a[key], b[key])):
                assert torch.equal(x, y), (what, key, l)
        else:
            assert torch.equal(a[key], b[key]), (what, key)


def _loop_state(case):
    ks = [k.cuda() for k in case["ks"]]
    vs = [v.cuda() for v in case["vs"]]
    pos = torch.tensor([case["pos"]], dtype=torch.int32, device="cuda")
    tok = torch.tensor([case["token"]], dtype=torch.int32, device="cuda")
    logits = torch.zeros(1, VOCAB, dtype=torch.float32, device="cuda")
    hid = torch.zeros(1, 2048, dtype=torch.bfloat16, device="cuda")
    return ks, vs, pos, tok, logits, hid


def _snapshot(ks, vs, pos, tok, logits, hid, toks):
    torch.cuda.synchronize()
    return dict(k=[k.cpu().view(torch.int16) for k in ks], v=[v.cpu().view(torch.int16) for v in vs],
                pos=pos.cpu(), tok=tok.cpu(), logits=logits.cpu().view(torch.int32), hidden=hid.cpu().view(torch.int16),
                toks=torch.stack([t.cpu() for t in toks]))


def test_noalloc_under_graph_capture_first(packed2):
    import mk_lib
    w = mk_lib.weights_struct(packed2)
    case = make_case(256, 100, seed=5, token=4321)
    adv = mk_lib.MK_FLAG_ADVANCE
    # reference: three workspace steps, each step's token fed back on the device
    ks, vs, pos, tok, logits, hid = _loop_state(case)
    ws = mk_lib.Workspace(1, 256, torch.device("cuda"))
    toks = []
    for _ in range(3):
        mk_lib.decode_step(w, ws, ks, vs, pos, tokens=tok, hidden_out=hid, logits=logits, next_token=tok, flags=adv)
        toks.append(tok.clone())
    ref = _snapshot(ks, vs, pos, tok, logits, hid, toks)
    assert ws.read_device_error() == 0
    ws.release()
    assert int(ref["pos"]) == 103

    ks, vs, pos, tok, logits, hid = _loop_state(case)
    init = [t.clone() for t in ks + vs] + [pos.clone(), tok.clone()]
    gtoks = torch.zeros(3, 1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    say("[noalloc] capturing 3 allocation-free steps (first allocation-free use in the process)")
    with torch.cuda.graph(graph, stream=stream):
        for i in range(3):
            mk_lib.decode_step_noalloc(w, ks, vs, pos, tokens=tok, hidden_out=hid, logits=logits, next_token=tok,
                                       flags=adv)
            gtoks[i].copy_(tok)

    def restore():
        for dst, src in zip(ks + vs + [pos, tok], init):
            dst.copy_(src)
        logits.zero_()
        hid.zero_()
        torch.cuda.synchronize()

    for rep in range(2):
        restore()
        say(f"[noalloc] graph replay {rep}")
        graph.replay()
        got = _snapshot(ks, vs, pos, tok, logits, hid, list(gtoks))
        assert_same(got, ref, f"replay {rep}")
    assert mk_lib.noalloc_device_error() == 0
    # an eager allocation-free loop after the capture fills the scratch itself and is still bit-exact
    restore()
    say("[noalloc] eager steps after the capture")
    toks = []
    for _ in range(3):
        mk_lib.decode_step_noalloc(w, ks, vs, pos, tokens=tok, hidden_out=hid, logits=logits, next_token=tok,
                                   flags=adv)
        toks.append(tok.clone())
    assert_same(_snapshot(ks, vs, pos, tok, logits, hid, toks), ref, "eager after capture")
    del graph


def test_noalloc_matches_workspace_step(packed2):
    import mk_lib
    cases = {
        "first": make_case(512, 300, seed=1, token=1234),
        "smaller": make_case(64, 17, seed=2, token=99),
        "layer-seam": make_case(64, 5, seed=3),
    }
    ref = {}
    for name, case in cases.items():
        ws = mk_lib.Workspace(1, case["s_max"], torch.device("cuda"))
        ref[name] = run(packed2, case, noalloc=False, ws=ws)
        assert ws.read_device_error() == 0, name
        ws.release()
    # the fresh rows were written at pos and the position advanced (sanity of the reference runs)
    for name, case in cases.items():
        assert int(ref[name]["pos"]) == case["pos"] + 1
        changed = (ref[name]["k"][0] != case["ks"][0].view(torch.int16)).any(-1).any(1).flatten()
        assert changed.nonzero().flatten().tolist() == [case["pos"]], name

    for name in ("first", "smaller", "layer-seam"):
        say(f"[noalloc] call '{name}': s_max={cases[name]['s_max']} pos={cases[name]['pos']}")
        got = run(packed2, cases[name], noalloc=True)
        assert_same(got, ref[name], name)
        if "next" in got:
            assert int(got["next"]) == int(got["logits"].view(torch.float32).argmax())

    # a step refused on the device (position == s_max): nothing written, next_token -1, no advance
    bad = make_case(64, 64, seed=4, token=7)
    say("[noalloc] refused step: pos = s_max = 64")
    got = run(packed2, bad, noalloc=True)
    assert int(got["next"]) == -1
    assert int(got["pos"]) == 64
    assert torch.all(torch.isnan(got["logits"].view(torch.float32)))
    for l in range(2):
        assert torch.equal(got["k"][l], bad["ks"][l].view(torch.int16))
        assert torch.equal(got["v"][l], bad["vs"][l].view(torch.int16))

    assert mk_lib.noalloc_device_error() == mk_lib.MK_DEVERR_POS     # sticky: kept until read
    assert mk_lib.noalloc_device_error() == 0

    say("[noalloc] call 'first' again")
    again = run(packed2, cases["first"], noalloc=True)
    assert_same(again, ref["first"], "first again")

    # a refused layer-stack step (hidden in, no next_token): only the sticky word reports it
    seam_bad = make_case(64, 64, seed=6)
    say("[noalloc] refused layer-stack step: pos = s_max = 64, no next_token")
    got = run(packed2, seam_bad, noalloc=True)
    assert int(got["pos"]) == 64
    assert mk_lib.noalloc_device_error() == mk_lib.MK_DEVERR_POS
    assert mk_lib.noalloc_device_error() == 0
    for l in range(2):
        assert torch.equal(got["k"][l], seam_bad["ks"][l].view(torch.int16))
