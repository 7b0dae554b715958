"""The Python seams over libmk.so behave like the reference's entry points.

* transformer_llama_megakernel_16layers (transformer_llama.py:196-241): the
  16-layer hidden output equals the model step's hidden output bit for bit,
  the K/V caches come back as the same tensors, updated at position_ids only;
* transformer_llama_megakernel_1layer: layer l alone equals the one-layer step;
* NeuronLlamaForCausalLM.forward(input_ids, position_ids, past_key_values)
  -> (logits, past_key_values) with the caches mutated in place;
* main.py validate agrees with the stock PyTorch path (short run).
"""

import pytest
import torch

from gpu_common import need_gpu, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    need_gpu()
    from llama_with_megakernel import LlamaInferenceConfig, NeuronConfigLlamaMK, NeuronLlamaForCausalLM
    m = NeuronLlamaForCausalLM("random:0", LlamaInferenceConfig(NeuronConfigLlamaMK(seq_len=256)))
    m.compile()
    m.load()
    return m


def test_16layer_seam_matches_model_step(model):
    import transformer_llama as tl
    from mk_weights import random_token_ids
    ids = random_token_ids(50, seed=21)
    model.prefill(ids)                         # pos 49, token ids[49] pending
    kv0 = model.kv.clone()
    model.launcher("decode").launch()
    torch.cuda.synchronize()
    want = model.hidden_out.clone()
    kv_model = model.kv.clone()
    model.kv.copy_(kv0)
    P = model.packed
    X = P["embed"][int(ids[49])].view(1, 1, 2048)
    out = tl.transformer_llama_megakernel_16layers(X, P["w_qkv"], P["w_o"], P["w_gu"], P["w_down"],
                                                   *model.k_caches, *model.v_caches, P["rope"],
                                                   torch.tensor([[49]], dtype=torch.int32))
    torch.cuda.synchronize()
    Y = out[0]
    assert len(out) == 33 and all(a is b for a, b in zip(out[1:17], model.k_caches))
    assert torch.equal(Y.view(-1).view(torch.int16), want.view(-1).view(torch.int16))
    assert torch.equal(model.kv.view(torch.int16), kv_model.view(torch.int16))


def test_1layer_seam(model):
    import transformer_llama as tl
    P = model.packed
    X = torch.randn(1, 1, 2048, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).cuda()
    K = torch.randn(1, 8, 256, 64, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).cuda()
    V = torch.randn(1, 8, 256, 64, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).cuda()
    K0, V0 = K.clone(), V.clone()
    Y5, K1, V1 = tl.transformer_llama_megakernel_1layer(X, P["w_qkv"], P["w_o"], P["w_gu"], P["w_down"], K, V,
                                                        P["rope"], torch.tensor([100]), layer=5)
    torch.cuda.synchronize()
    assert K1 is K and V1 is V
    changed = (K.view(torch.int16) != K0.view(torch.int16)).any(-1)[0]    # [8, 256]
    assert changed[:, 100].all() and not changed[:, :100].any() and not changed[:, 101:].any()
    import mk_lib
    ws = mk_lib.Workspace(1, 256, torch.device("cuda"))
    out = torch.empty(1, 2048, dtype=torch.bfloat16, device="cuda")
    K2, V2 = K0.clone(), V0.clone()
    rc = mk_lib.load().mk_layer_step(mk_lib.weights_struct(P), 5, 1, 256, K2.data_ptr(), V2.data_ptr(),
                                     X.data_ptr(), torch.tensor([100], dtype=torch.int32, device="cuda").data_ptr(),
                                     out.data_ptr(), ws.buf.data_ptr(), ws.nbytes, mk_lib.current_stream_ptr())
    mk_lib.check(rc)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), Y5.view(1, 2048).view(torch.int16))
    assert torch.equal(K2.view(torch.int16), K.view(torch.int16))


def test_forward_contract(model):
    from mk_weights import random_token_ids
    ids = random_token_ids(10, seed=8)
    model.prefill(ids)
    pkv = model.past_key_values
    before = [k.clone() for k, _ in pkv]
    logits, new_kv = model.forward(input_ids=ids[9:10], position_ids=torch.tensor([[9]]), past_key_values=pkv)
    torch.cuda.synchronize()
    assert logits.shape == (1, 128256) and logits.dtype == torch.float32
    assert all(a is b for (a, _), (b, _) in zip(new_kv, pkv))
    for k0, (k1, _) in zip(before, new_kv):
        ch = (k0.view(torch.int16) != k1.view(torch.int16)).any(-1)[0]
        assert ch[:, 9].all() and not ch[:, :9].any() and not ch[:, 10:].any()


@pytest.mark.timeout(300)
def test_main_validate_short(tmp_path):
    """validate with the reference's own flags (main.py:34-105; README.md:48-51)."""
    import main
    rc = main.main(["--mode", "validate", "--enable-nki", "--prompt-len", "24", "--max-new-tokens", "48",
                    "--seq-len", "128", "--tp-degree", "1", "--torch-dtype", "bfloat16",
                    "--compiled-model-path", str(tmp_path / "nki"), "--divergence-difference-tol", "0.001",
                    "--tol-map", "{None: (1e-5, 0.05), 1000: (1e-5, 0.03), 50: (1e-5, 0.03), 5: (1e-5, 0.03)}",
                    "--num-tokens-to-check", "40", "--on-device-sampling", "--fused-qkv"])
    assert rc == 0
    assert (tmp_path / "nki" / "mk_compiled.json").exists()


@pytest.mark.timeout(300)
def test_main_generate_reference_flags(tmp_path, capsys):
    """generate with the reference's flags; --output-logits returns the
    per-step logits, whose argmax is the generated token."""
    import main
    out = main.run_generation(main.parse_args(
        ["--mode", "generate", "--enable-nki", "--prompt-ids", "5,6,7,8", "--seq-len", "64",
         "--max-new-tokens", "6", "--compiled-model-path", str(tmp_path / "g"), "--output-logits",
         "--tp-degree", "1"]))
    assert out.shape == (1, 6)
    assert "logits [6, 128256]" in capsys.readouterr().out


def test_layer_seam_token_generation(model):
    """NeuronLlamaDecoderLayerMK (llama_with_megakernel.py:65-204): layer 0
    runs the 16-layer megakernel, layers 1..15 return the stash with their own
    (K, V); the result equals the model step's hidden output bit for bit."""
    from mk_weights import random_token_ids
    ids = random_token_ids(30, seed=23)
    model.prefill(ids)                          # pos 29, token ids[29] pending
    kv0 = model.kv.clone()
    model.launcher("decode").launch()
    torch.cuda.synchronize()
    want_h, want_kv = model.hidden_out.clone(), model.kv.clone()
    model.kv.copy_(kv0)
    x = model.packed["embed"][int(ids[29])].reshape(1, 1, -1)
    pos = torch.tensor([[29]], device="cuda")
    Y, present = model.layer_stack_forward(x, pos, model.past_key_values)
    torch.cuda.synchronize()
    assert torch.equal(Y.reshape(-1), want_h.reshape(-1))
    assert torch.equal(model.kv, want_kv)
    for i, (k, v) in enumerate(present):
        assert k is model.k_caches[i] and v is model.v_caches[i]
    out0 = model.layers[0](x, position_ids=pos, past_key_value=model.past_key_values[0])
    cos, sin = out0[2], out0[3]
    assert cos.shape == sin.shape == (1, 1, 64)
    assert torch.equal(torch.cat([cos, sin], -1).reshape(-1), model.packed["rope"][29])


def test_layer_seam_context_encoding(model):
    """Context encoding through the layer seam (each layer over the prompt,
    token by token) writes the same K/V rows as the token-by-token prefill of
    the 16-layer kernel, bit for bit, and only rows 0..n-1."""
    from mk_weights import random_token_ids
    ids = random_token_ids(12, seed=29)
    model.kv.zero_()
    model.prefill(torch.cat([ids, ids[:1]]), batched=False)   # rows 0..11 written
    torch.cuda.synchronize()
    want = model.kv.clone()
    model.kv.zero_()
    x = model.packed["embed"][ids.long().cuda()].reshape(1, 12, -1)
    pos = torch.arange(12, device="cuda").reshape(1, 12)
    Y, _ = model.layer_stack_forward(x, pos, None)
    torch.cuda.synchronize()
    assert Y.shape == (1, 12, 2048)
    assert torch.equal(model.kv, want)
    assert not model.kv[:, :, :, :, 12:].any()
