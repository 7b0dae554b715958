"""Batches through the drop-in model seam, checkpoints and the benchmark report, on the GPU.

* ``NeuronLlamaForCausalLM`` loaded with batch_size 8 (the batched MFMA
  kernel) generates from 8 independent prompts of different lengths (the
  reference derives the batch from its prompts, main.py:538-540): each
  sequence is prefilled into its own cache slice (chunked MK_FLAG_PREFILL
  launches per sequence) and decoded at its own position. Every generated
  step of every sequence is checked against the oracle's step from the GPU's
  cache (rows below a position are final once written) at the per-step bounds
  of the batch-1 tests (max-abs 0.15, rms 0.03), each generated token is the
  argmax of its step's logits, the oracle agrees wherever its top-2 gap is
  >= 0.1, and each sequence's cache slice holds exactly its own rows
  (0 .. n_b + T - 2) and nothing else. ``forward`` with a sub-batch updates
  only those sequences' rows.
* A safetensors checkpoint written from the seed-0 weights and read back
  through ``load_hf_checkpoint`` (the model_path of a real checkpoint) gives
  logits bit-identical to the ``random:0`` weights (2-layer model, full vocab).
* ``main.py --mode benchmark`` plain, with ``--graph`` and with ``--decode-loop`` writes a report
  with the e2e / context-encoding / token-generation sections (main.py:178-271).
"""

import json
import os

import pytest
import torch

from gpu_common import logit_stats, need_gpu, record_parity, say

pytestmark = pytest.mark.gpu

S = 256
LENS = [5, 37, 100, 64, 1, 150, 33, 90]
T = 4


@pytest.fixture(scope="module")
def batch_model():
    need_gpu()
    from llama_with_megakernel import LlamaInferenceConfig, NeuronConfigLlamaMK, NeuronLlamaForCausalLM
    from oracle.llama_ref import OracleLlama
    torch.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    cfg = LlamaInferenceConfig(NeuronConfigLlamaMK(batch_size=len(LENS), seq_len=S, max_context_length=S))
    m = NeuronLlamaForCausalLM("random:0", cfg)
    m.compile()
    m.load()
    return m, OracleLlama(m.state_dict_bf16, mode="mk")


def test_batch8_generate_matches_oracle_per_sequence(batch_model):
    from mk_weights import random_token_ids
    m, o = batch_model
    prompts = [random_token_ids(n, seed=300 + b) for b, n in enumerate(LENS)]
    m.kv.zero_()
    say(f"[mbatch] generate {T} tokens for prompts of lengths {LENS}")
    toks, logits = m.generate(prompts, T, return_logits=True)     # [B, T], [B, T, V]
    assert toks.shape == (len(LENS), T) and logits.shape == (len(LENS), T, 128256)
    worst_max = worst_rms = 0.0
    n_dec = n_ok = 0
    rec = []
    for b, ids in enumerate(prompts):
        n = len(ids)
        seq = torch.cat([ids, toks[b].long()])
        cache = [(m.kv[l, 0, b].float().cpu(), m.kv[l, 1, b].float().cpu()) for l in range(16)]
        for t in range(T):
            ref, _ = o.forward(torch.tensor([int(seq[n - 1 + t])]), n - 1 + t, [(k.clone(), v.clone())
                                                                               for k, v in cache])
            st = logit_stats(logits[b, t], ref[0])
            worst_max, worst_rms = max(worst_max, st["max_abs"]), max(worst_rms, st["rms"])
            assert st["max_abs"] <= 0.15 and st["rms"] <= 0.03, (b, t, st)
            assert int(toks[b, t]) == int(logits[b, t].argmax()), (b, t)
            top2 = ref[0].topk(2).values
            if float(top2[0] - top2[1]) >= 0.1:
                n_dec += 1
                n_ok += int(ref[0].argmax()) == int(toks[b, t])
                assert int(ref[0].argmax()) == int(toks[b, t]), (b, t)
            rec.append(dict(st, seq=b, step=t, pos=n - 1 + t))
        # the sequence's own slice: rows 0 .. n + T - 2 written, the rest untouched
        nz = (m.kv[:, :, b].view(torch.int16) != 0).any(-1)     # [L, 2, 8, S]
        rows = nz.any(0).any(0).any(0).nonzero().flatten().tolist()
        assert rows == list(range(n + T - 1)), (b, rows[:3], rows[-3:])
    say(f"[mbatch] logits worst max|d| {worst_max:.3e}, worst rms {worst_rms:.3e}; decided agreement {n_ok}/{n_dec}")
    record_parity("model_batch8", {"config": "model seam, batch 8", "prompt_lengths": LENS, "steps": T,
                                   "worst_max_abs": worst_max, "worst_rms": worst_rms, "decided_positions": n_dec,
                                   "decided_agreement": n_ok / n_dec if n_dec else None, "per_step": rec})


def test_forward_sub_batch_updates_only_its_sequences(batch_model):
    from mk_weights import random_token_ids
    m, _ = batch_model
    prompts = [random_token_ids(n, seed=400 + b) for b, n in enumerate(LENS)]
    m.prefill(prompts)
    torch.cuda.synchronize()
    before = m.kv.clone()
    pos = torch.tensor([LENS[0] - 1, LENS[1] - 1])
    ids = torch.tensor([int(prompts[0][-1]), int(prompts[1][-1])])
    logits, kv = m.forward(input_ids=ids, position_ids=pos)
    torch.cuda.synchronize()
    assert logits.shape == (2, 128256)
    assert kv[0][0] is m.k_caches[0]
    ch = (m.kv != before).any(-1)     # [L, 2, B, 8, S]
    for b in range(len(LENS)):
        rows = ch[:, :, b].any(0).any(0).any(0).nonzero().flatten().tolist()
        assert rows == ([LENS[b] - 1] if b < 2 else []), (b, rows)


def test_checkpoint_directory_matches_random_weights(tmp_path):
    need_gpu()
    from safetensors.torch import save_file
    from llama_with_megakernel import LlamaInferenceConfig, NeuronConfigLlamaMK, NeuronLlamaForCausalLM
    from mk_config import LlamaDims
    from mk_weights import random_token_ids, synthetic_state_dict
    d = LlamaDims(n_layers=2)
    sd = synthetic_state_dict(seed=0, d=d)
    save_file({"model." + k: v.contiguous() for k, v in sd.items()}, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({"model_type": "llama", "tie_word_embeddings": True}))
    ids = random_token_ids(20, seed=21)
    out = []
    for path in ("random:0", str(tmp_path)):
        cfg = LlamaInferenceConfig(NeuronConfigLlamaMK(seq_len=64, max_context_length=64), dims=d)
        m = NeuronLlamaForCausalLM(path, cfg)
        m.compile()
        m.load()
        m.prefill(ids)
        m.launcher("decode").launch()
        torch.cuda.synchronize()
        assert m.ws.read_device_error() == 0
        out.append((m.logits.cpu(), m.kv.cpu()))
        del m
    assert torch.equal(out[0][0].view(torch.int32), out[1][0].view(torch.int32))
    assert torch.equal(out[0][1].view(torch.int16), out[1][1].view(torch.int16))


@pytest.mark.timeout(300)
@pytest.mark.parametrize("graph", [False, True, "loop"])
def test_main_benchmark_report(tmp_path, graph):
    need_gpu()
    import main
    path = tmp_path / "benchmark_report.json"
    extra = {False: [], True: ["--graph"], "loop": ["--decode-loop"]}[graph]
    argv = ["--mode", "benchmark", "--enable-nki", "--prompt-len", "64", "--max-new-tokens", "32",
            "--seq-len", "128", "--num-runs", "2", "--report-path", str(path)] + extra
    assert main.main(argv) == 0
    rep = json.loads(path.read_text())
    for key in ("e2e_model", "context_encoding_model", "token_generation_model"):
        r = rep[key]
        assert 0 < r["latency_ms_p50"] <= r["latency_ms_p99"] <= r["latency_ms_p100"]
        assert r["throughput"] > 0
    tg = rep["token_generation_model"]
    say(f"[report] graph={graph}: token generation p50 {tg['latency_ms_p50']:.4f} ms, "
        f"e2e p50 {rep['e2e_model']['latency_ms_p50']:.2f} ms")
    assert tg["latency_ms_p50"] < 5.0          # one step of the 16-layer model, milliseconds
