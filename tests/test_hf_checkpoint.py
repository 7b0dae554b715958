"""The HF checkpoint path: ``mk_weights.load_hf_checkpoint``
reads a local safetensors checkpoint into the naming the packer consumes, the
input format on the far side of the reference's convert_hf_to_neuron_state_dict
(llama_with_megakernel.py:281-351; tied lm_head, llama.py:1404-1406).

* A transformers ``LlamaForCausalLM`` (reduced dims, tied embeddings, random
  init, built offline) saved with ``save_pretrained`` loads back to its own
  state dict (bf16), so the naming follows transformers' real format;
* sharded checkpoints and fp32 checkpoints (cast to bf16) load;
* a missing tensor, a wrong shape, or a directory without safetensors is
  refused with a clear error;
* the packed layout of a loaded checkpoint equals the packed layout of the
  state dict it was written from.
"""

import pytest
import torch


def hf_model(small_prod, tie=True):
    from transformers import LlamaConfig, LlamaForCausalLM
    d = small_prod
    cfg = LlamaConfig(vocab_size=d.vocab, hidden_size=d.hidden, intermediate_size=d.intermediate,
                      num_hidden_layers=d.n_layers, num_attention_heads=d.n_q_heads,
                      num_key_value_heads=d.n_kv_heads, head_dim=d.head_dim, rms_norm_eps=d.rms_eps,
                      rope_theta=d.rope_theta, tie_word_embeddings=tie, torch_dtype=torch.bfloat16,
                      rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                    "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})
    torch.manual_seed(0)
    m = LlamaForCausalLM(cfg).to(torch.bfloat16)
    with torch.no_grad():   # non-trivial norm gammas, so a swapped norm would show
        for n, p in m.named_parameters():
            if n.endswith("norm.weight"):
                p.copy_(1.0 + 0.1 * torch.randn_like(p, dtype=torch.float32))
    return m


def test_transformers_checkpoint_round_trip(tmp_path, small):
    from mk_weights import load_hf_checkpoint
    prod, _ = small
    m = hf_model(prod)
    m.save_pretrained(tmp_path, safe_serialization=True)
    sd = load_hf_checkpoint(str(tmp_path), prod)
    ref = {k[len("model."):]: v for k, v in m.state_dict().items() if k.startswith("model.")}
    for name, t in ref.items():
        assert sd[name].dtype == torch.bfloat16
        assert torch.equal(sd[name].view(torch.int16), t.view(torch.int16)), name
    # tied lm_head: the embedding is the output projection
    assert torch.equal(m.lm_head.weight.view(torch.int16), sd["embed_tokens.weight"].view(torch.int16))


def test_sharded_and_fp32_checkpoints(tmp_path, small):
    from safetensors.torch import save_file
    from mk_weights import load_hf_checkpoint, synthetic_state_dict
    prod, _ = small
    sd = synthetic_state_dict(seed=3, d=prod)
    names = sorted(sd)
    half = len(names) // 2
    save_file({"model." + k: sd[k].float() for k in names[:half]}, str(tmp_path / "a.safetensors"))
    save_file({"model." + k: sd[k].float() for k in names[half:]}, str(tmp_path / "b.safetensors"))
    got = load_hf_checkpoint(str(tmp_path), prod)
    for k in names:   # bf16 -> fp32 -> bf16 is exact
        assert torch.equal(got[k].view(torch.int16), sd[k].view(torch.int16)), k


def test_refusals(tmp_path, small):
    from safetensors.torch import save_file
    from mk_weights import load_hf_checkpoint, synthetic_state_dict
    prod, _ = small
    with pytest.raises(FileNotFoundError):
        load_hf_checkpoint(str(tmp_path), prod)
    sd = synthetic_state_dict(seed=1, d=prod)
    missing = {k: v for k, v in sd.items() if k != "layers.1.mlp.up_proj.weight"}
    save_file(missing, str(tmp_path / "m.safetensors"))
    with pytest.raises(KeyError, match="up_proj"):
        load_hf_checkpoint(str(tmp_path), prod)
    (tmp_path / "m.safetensors").unlink()
    bad = dict(sd)
    bad["layers.0.self_attn.k_proj.weight"] = bad["layers.0.self_attn.k_proj.weight"][:-1].contiguous()
    save_file(bad, str(tmp_path / "w.safetensors"))
    with pytest.raises(ValueError, match="k_proj"):
        load_hf_checkpoint(str(tmp_path), prod)


def test_loaded_checkpoint_packs_like_its_source(tmp_path, small):
    from safetensors.torch import save_file
    from mk_weights import load_hf_checkpoint, pack_for_megakernel, synthetic_state_dict
    prod, _ = small
    sd = synthetic_state_dict(seed=4, d=prod)
    save_file({"model." + k: v for k, v in sd.items()}, str(tmp_path / "model.safetensors"))
    a = pack_for_megakernel(sd, prod, device="cpu", rope_rows=64)
    b = pack_for_megakernel(load_hf_checkpoint(str(tmp_path), prod), prod, device="cpu", rope_rows=64)
    assert a.keys() == b.keys()
    for k in a:
        assert torch.equal(a[k].view(torch.int16) if a[k].dtype == torch.bfloat16 else a[k],
                           b[k].view(torch.int16) if b[k].dtype == torch.bfloat16 else b[k]), k


def test_untied_lm_head_is_refused(tmp_path, small):
    """The kernel's lm_head is the embedding: an untied checkpoint would give
    wrong logits, so it is refused (config flag, or a differing lm_head tensor)."""
    from safetensors.torch import save_file
    from mk_weights import load_hf_checkpoint, synthetic_state_dict
    prod, _ = small
    m = hf_model(prod, tie=False)
    m.save_pretrained(tmp_path / "untied", safe_serialization=True)
    with pytest.raises(ValueError, match="tie_word_embeddings"):
        load_hf_checkpoint(str(tmp_path / "untied"), prod)
    # no config.json: the tensors decide
    sd = synthetic_state_dict(seed=5, d=prod)
    (tmp_path / "raw").mkdir()
    other = dict(sd)
    other["lm_head.weight"] = (sd["embed_tokens.weight"].float() * 2).to(torch.bfloat16)
    save_file({("" if k == "lm_head.weight" else "model.") + k: v for k, v in other.items()},
              str(tmp_path / "raw" / "model.safetensors"))
    with pytest.raises(ValueError, match="untied"):
        load_hf_checkpoint(str(tmp_path / "raw"), prod)
    # an lm_head equal to the embedding (a tied checkpoint that stores both) loads, without it
    (tmp_path / "tied").mkdir()
    same = dict(sd)
    same["lm_head.weight"] = sd["embed_tokens.weight"].clone()
    save_file({("" if k == "lm_head.weight" else "model.") + k: v for k, v in same.items()},
              str(tmp_path / "tied" / "model.safetensors"))
    got = load_hf_checkpoint(str(tmp_path / "tied"), prod)
    assert "lm_head.weight" not in got
