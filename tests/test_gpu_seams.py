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
def test_main_validate_short():
    import main
    rc = main.main(["--mode", "validate", "--enable-nki", "--prompt-len", "24", "--max-new-tokens", "48",
                    "--seq-len", "128"])
    assert rc == 0
