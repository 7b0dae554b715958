"""HIP-graph replay of the decode loop (the generation loop the reference
drives step by step through NxDI, main.py:178-271) against the same steps
launched one by one.

A graph of 12 decode steps (greedy, and with the on-device sampler) is
captured once and replayed three times, each replay after an eager prefill of
the prompt on the model's stream: every replay's tokens and final logits equal
the eagerly launched steps' bit for bit (same kernels, same device state).
While the graph lives its workspace refuses to be released; once the graph is
destroyed the release goes through.
"""

import gc

import pytest
import torch

from gpu_common import need_gpu, say

pytestmark = pytest.mark.gpu

N = 12


@pytest.mark.parametrize("sampled", [False, True])
def test_graph_replays_match_eager_steps(sampled):
    need_gpu()
    import mk_lib
    from llama_with_megakernel import LlamaInferenceConfig, NeuronConfigLlamaMK, NeuronLlamaForCausalLM
    from mk_weights import random_token_ids
    cfg = LlamaInferenceConfig(NeuronConfigLlamaMK(seq_len=256, max_context_length=256))
    m = NeuronLlamaForCausalLM("random:0", cfg)
    m.compile()
    m.load()
    ids = random_token_ids(30, seed=13)
    sp = mk_lib.prepare_sampling_params(1, 20, 0.9, 0.9) if sampled else None
    toks, lg = m.generate(ids, N, return_logits=True, sampling_params=sp, seed=5)
    eager_tokens, eager_last = toks.to(torch.int32), lg[-1]
    graph = m.decode_graph(N, sampling_params=sp, seed=5)
    for rep in range(3):
        m.prefill(ids)                       # eager work on the current stream between replays
        m.logits.zero_()
        torch.cuda.current_stream().synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert m.ws.read_device_error() == 0
        got = m.graph_tokens[:, 0].cpu()       # [steps, batch]
        say(f"[graph] sampled={sampled} replay {rep}: tokens {got[:6].tolist()}... eager {eager_tokens[:6].tolist()}")
        assert torch.equal(got, eager_tokens)
        assert torch.equal(m.logits[0].cpu(), eager_last)
        assert int(m.pos.item()) == len(ids) - 1 + N
    # the graph's kernel arguments hold the workspace's exchange area: no release while it lives
    with pytest.raises(RuntimeError, match="graph"):
        m.ws.release()
    del graph
    gc.collect()
    m.ws.release()
