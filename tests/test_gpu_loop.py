"""The greedy decode loop (``mk_decode_loop``): several decode steps in one
persistent launch, the workgroups meeting at an on-device barrier between
steps, against the same steps launched one by one (``mk_decode_step``).

Each step of the loop is the single step's computation, so from the same
state (a 64-token prompt prefilled into a 256-row cache) the loop's tokens,
its last step's logits and hidden state, every K/V cache byte and the advanced
position equal those of 24 single launches bit for bit. A loop followed by
single steps continues the exchange-set and argmax-key state (equal to the
same number of single steps). The step clock is monotonic. ``model.generate``
(greedy, batch 1) runs the loop and returns the step-by-step tokens; a HIP graph
of a loop replays it exactly; the loop on generic grids and at KV positions near
4000 equals single steps; ``model.decode_loop`` gives the same result on the
stream of its prebuilt arguments and on a side stream. Refusals: batch > 1
workspace, hidden input, and positions past the cache (a device error, nothing
written).
"""

import pytest
import torch

from gpu_common import need_gpu, say

pytestmark = pytest.mark.gpu

S = 256
N = 24


@pytest.fixture(scope="module")
def model():
    need_gpu()
    from llama_with_megakernel import LlamaInferenceConfig, NeuronConfigLlamaMK, NeuronLlamaForCausalLM
    m = NeuronLlamaForCausalLM("random:0", LlamaInferenceConfig(NeuronConfigLlamaMK(seq_len=S)))
    m.compile()
    m.load()
    return m


def snapshot(m):
    torch.cuda.synchronize()
    return dict(kv=m.kv.clone(), pos=m.pos.clone(), tok=m.tokens.clone())


def restore(m, st):
    m.kv.copy_(st["kv"])
    m.pos.copy_(st["pos"])
    m.tokens.copy_(st["tok"])
    m.logits.zero_()
    m.hidden_out.zero_()
    torch.cuda.synchronize()


def singles(m, n):
    dec = m.launcher("decode")
    toks = []
    for _ in range(n):
        dec.launch()
        toks.append(m.tokens.clone())
    torch.cuda.synchronize()
    assert m.ws.read_device_error() == 0
    return torch.cat(toks).cpu()


def loop(m, n, clock=None):
    import mk_lib
    out = torch.full((n,), -5, dtype=torch.int32, device="cuda")
    mk_lib.decode_loop(m.weights, m.ws, m.k_caches, m.v_caches, m.pos, m.tokens, n, tokens_out=out,
                       step_clock=clock, logits=m.logits, next_token=m.tokens, hidden_out=m.hidden_out,
                       flags=mk_lib.MK_FLAG_ADVANCE)
    torch.cuda.synchronize()
    assert m.ws.read_device_error() == 0
    return out.cpu()


def test_loop_equals_single_steps(model):
    from mk_weights import random_token_ids
    m = model
    m.prefill(random_token_ids(64, seed=41))
    st = snapshot(m)
    ref_toks = singles(m, N)
    ref = dict(kv=m.kv.clone(), pos=m.pos.clone(), logits=m.logits.clone(), hid=m.hidden_out.clone(),
               tok=m.tokens.clone())
    restore(m, st)
    clock = torch.zeros(N + 1, dtype=torch.int64, device="cuda")
    got = loop(m, N, clock)
    say(f"[loop] tokens {got[:8].tolist()}... single steps {ref_toks[:8].tolist()}...")
    assert torch.equal(got, ref_toks)
    assert torch.equal(m.tokens, ref["tok"]) and int(m.pos.item()) == int(st["pos"].item()) + N
    assert torch.equal(m.logits.view(torch.int32), ref["logits"].view(torch.int32))
    assert torch.equal(m.hidden_out.view(torch.int16), ref["hid"].view(torch.int16))
    assert torch.equal(m.kv.view(torch.int16), ref["kv"].view(torch.int16))
    c = clock.cpu()
    assert bool((c[1:] > c[:-1]).all()), c.tolist()
    import mk_lib
    hz = mk_lib.load().mk_wall_clock_hz(0)
    d = (c[1:] - c[:-1]).double() * 1e6 / hz
    say(f"[loop] step durations (us): median {float(d.median()):.1f}, min {float(d.min()):.1f}, max {float(d.max()):.1f}")


def test_loop_then_single_steps_continue(model):
    from mk_weights import random_token_ids
    m = model
    m.prefill(random_token_ids(40, seed=43))
    st = snapshot(m)
    ref_toks = singles(m, 9)
    ref_kv = m.kv.clone()
    restore(m, st)
    got = torch.cat([loop(m, 5), singles(m, 2), loop(m, 2)])
    assert torch.equal(got, ref_toks)
    assert torch.equal(m.kv.view(torch.int16), ref_kv.view(torch.int16))


def test_loop_refusals(model):
    import mk_lib
    m = model
    with pytest.raises(mk_lib.MkError) as e:   # hidden input
        a = m.launcher("decode").args
        a_hidden = mk_lib.MkStepArgs.from_buffer_copy(a)
        a_hidden.hidden_in = m.hidden_out.data_ptr()
        a_hidden.tokens = None
        mk_lib.check(mk_lib.load().mk_decode_loop(mk_lib.ctypes.byref(m.weights), mk_lib.ctypes.byref(a_hidden),
                                                  4, None, None))
    assert e.value.code == -4
    ws8 = mk_lib.Workspace(8, S, torch.device("cuda"))
    with pytest.raises(mk_lib.MkError) as e:   # batched workspace
        mk_lib.decode_loop(m.weights, ws8, m.k_caches, m.v_caches, m.pos, m.tokens, 4)
    assert e.value.code == -4
    # positions past the cache: refused on the device, nothing written
    m.pos.fill_(S - 3)
    kv0 = m.kv.clone()
    mk_lib.decode_loop(m.weights, m.ws, m.k_caches, m.v_caches, m.pos, m.tokens, 4, flags=mk_lib.MK_FLAG_ADVANCE)
    torch.cuda.synchronize()
    assert m.ws.read_device_error() & mk_lib.MK_DEVERR_POS
    assert int(m.pos.item()) == S - 3
    assert torch.equal(m.kv.view(torch.int16), kv0.view(torch.int16))
    # and the workspace is still good for a loop afterwards
    m.pos.fill_(10)
    loop(m, 3)


def test_generate_runs_the_loop(model):
    """Greedy batch-1 ``generate`` without logits runs the steps as one
    ``mk_decode_loop`` launch; with logits it launches every step. Same tokens."""
    from mk_weights import random_token_ids
    m = model
    ids = random_token_ids(50, seed=47)
    stepwise, _ = m.generate(ids, 30, return_logits=True)
    looped = m.generate(ids, 30)
    say(f"[loop] generate: {looped[:8].tolist()}...")
    assert torch.equal(looped, stepwise)
    assert int(m.pos.item()) == 50 + 30 - 1
    with pytest.raises(ValueError):
        m.decode_loop(S)                 # past the cache: refused on the host


def test_loop_in_a_graph(model):
    """``mk_decode_loop`` is capturable (no allocation, no memset): a HIP graph of
    one 6-step loop, replayed three times from the same state with eager steps
    and synchronisations between the replays, equals the eager loop each time."""
    import mk_lib
    from mk_weights import random_token_ids
    m = model
    m.prefill(random_token_ids(30, seed=51))
    st = snapshot(m)
    ref = loop(m, 6)
    ref_kv, ref_logits = m.kv.clone(), m.logits.clone()
    restore(m, st)
    out = torch.full((6,), -5, dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        mk_lib.decode_loop(m.weights, m.ws, m.k_caches, m.v_caches, m.pos, m.tokens, 6, tokens_out=out,
                           logits=m.logits, next_token=m.tokens, hidden_out=m.hidden_out,
                           flags=mk_lib.MK_FLAG_ADVANCE)
    m.ws.register_graph(graph)
    for rep in range(3):
        restore(m, st)
        singles(m, 2)                    # eager steps between the replays
        restore(m, st)
        out.fill_(-5)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert m.ws.read_device_error() == 0
        say(f"[loop] graph replay {rep}: {out[:6].tolist()}")
        assert torch.equal(out.cpu(), ref), rep
        assert int(m.pos.item()) == int(st["pos"].item()) + 6
        assert torch.equal(m.kv.view(torch.int16), ref_kv.view(torch.int16)), rep
        assert torch.equal(m.logits.view(torch.int32), ref_logits.view(torch.int32)), rep
    del graph


def test_one_step_loop(model):
    """A loop of one step is one single step: it writes its token and both
    step-clock entries, and equals a single launch bit for bit."""
    from mk_weights import random_token_ids
    m = model
    m.prefill(random_token_ids(20, seed=53))
    st = snapshot(m)
    ref = singles(m, 1)
    ref_logits, ref_kv = m.logits.clone(), m.kv.clone()
    restore(m, st)
    clock = torch.zeros(2, dtype=torch.int64, device="cuda")
    got = loop(m, 1, clock)
    assert torch.equal(got, ref)
    assert torch.equal(m.logits.view(torch.int32), ref_logits.view(torch.int32))
    assert torch.equal(m.kv.view(torch.int16), ref_kv.view(torch.int16))
    c = clock.cpu()
    assert int(c[1]) > int(c[0]) > 0, c.tolist()


@pytest.mark.parametrize("grid", [200, 128])
def test_loop_on_a_generic_grid(model, grid):
    """The loop's generic-grid instantiation (``mk_set_grid_size``): on 200 and
    128 workgroups, 6 steps in one launch equal 6 single launches on the same
    grid bit for bit (the step barrier's sub-counter shares follow the grid)."""
    import mk_lib
    from mk_weights import random_token_ids
    m = model
    m.prefill(random_token_ids(48, seed=59))
    st = snapshot(m)
    mk_lib.set_grid_size(grid)
    try:
        assert mk_lib.grid_size() == grid
        ref = singles(m, 6)
        ref_kv = m.kv.clone()
        restore(m, st)
        got = loop(m, 6)
    finally:
        torch.cuda.synchronize()
        mk_lib.set_grid_size(0)
    say(f"[loop] grid {grid}: {got.tolist()}")
    assert torch.equal(got, ref)
    assert torch.equal(m.kv.view(torch.int16), ref_kv.view(torch.int16))


def test_loop_at_long_context():
    """At KV positions near 4000 of a 4096-row cache (attention items of several
    128-row groups, 8 splits per kv head), 10 steps in one launch equal 10
    single launches bit for bit."""
    need_gpu()
    from llama_with_megakernel import LlamaInferenceConfig, NeuronConfigLlamaMK, NeuronLlamaForCausalLM
    from mk_weights import random_token_ids
    S4 = 4096
    m = NeuronLlamaForCausalLM("random:0", LlamaInferenceConfig(NeuronConfigLlamaMK(seq_len=S4)))
    m.compile()
    m.load()
    m.prefill(random_token_ids(64, seed=61))
    g = torch.Generator(device="cuda").manual_seed(3)
    m.kv[:, :, :, :, 64:].normal_(generator=g)    # rows past the prompt: N(0,1) K/V up to the start position
    m.pos.fill_(3990)
    st = snapshot(m)
    ref = singles(m, 10)
    ref_kv = m.kv.clone()
    restore(m, st)
    got = loop(m, 10)
    assert torch.equal(got, ref)
    assert torch.equal(m.kv.view(torch.int16), ref_kv.view(torch.int16))
    assert int(m.pos.item()) == 4000


def test_model_loop_on_a_side_stream(model):
    """``model.decode_loop`` calls the prebuilt decode launcher's loop on the
    stream that launcher was built for, and ``mk_decode_loop`` with fresh
    arguments on any other current stream: same tokens and caches either way."""
    from mk_weights import random_token_ids
    m = model
    m.prefill(random_token_ids(36, seed=61))
    st = snapshot(m)
    ref = m.decode_loop(5).cpu()
    ref_kv = m.kv.clone()
    restore(m, st)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        got = m.decode_loop(5)
    side.synchronize()
    torch.cuda.synchronize()
    assert m.ws.read_device_error() == 0
    assert torch.equal(got.cpu(), ref)
    assert torch.equal(m.kv.view(torch.int16), ref_kv.view(torch.int16))
