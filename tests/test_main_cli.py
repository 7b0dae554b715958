"""CPU checks of main.py's prompt handling and report (no GPU calls).

* ``--prompt`` text is encoded with a tokenizer read from a local directory
  only (the reference's load_tokenizer, main.py:114-118; pad token = EOS);
  the tokenizer here is a small word-level one built offline in the test and
  saved in transformers' format, so the loading path is the real one;
* the batch is the list of prompts (main.py:538-540): repeated ``--prompt`` /
  ``--prompt-ids`` give one sequence each, kept at their own lengths; with no
  prompt, ``--batch-size`` random prompts (seeds 0, 1, ...);
* ``generate_report``'s percentiles and throughput on a known latency list.
"""

import pytest
import torch

VOCAB = {"<unk>": 0, "<s>": 1, "</s>": 2, "the": 3, "meaning": 4, "of": 5, "life": 6, "is": 7, "I": 8,
         "believe": 9}


@pytest.fixture()
def tok_dir(tmp_path):
    from tokenizers import Tokenizer, models, pre_tokenizers
    from transformers import PreTrainedTokenizerFast
    t = Tokenizer(models.WordLevel(VOCAB, unk_token="<unk>"))
    t.pre_tokenizer = pre_tokenizers.Whitespace()
    PreTrainedTokenizerFast(tokenizer_object=t, unk_token="<unk>", bos_token="<s>",
                            eos_token="</s>").save_pretrained(tmp_path / "tok")
    return tmp_path / "tok"


def test_text_prompts_through_local_tokenizer(tok_dir):
    import main
    args = main.parse_args(["--mode", "generate", "--prompt", "I believe the meaning of life is",
                            "--prompt", "the life", "--tokenizer-path", str(tok_dir)])
    prompts = main.encode_prompts(args)
    assert [p.tolist() for p in prompts] == [[8, 9, 3, 4, 5, 6, 7], [3, 6]]
    tok = main.load_tokenizer(str(tok_dir))
    assert tok.pad_token == tok.eos_token == "</s>"
    assert tok.decode([8, 9, 3, 4]) == "I believe the meaning"


def test_tokenizer_defaults_to_the_model_directory(tok_dir):
    import main
    args = main.parse_args(["--mode", "generate", "--model-path", str(tok_dir), "--prompt", "life is"])
    assert main.tokenizer_dir(args) == str(tok_dir)
    assert [p.tolist() for p in main.encode_prompts(args)] == [[6, 7]]
    args = main.parse_args(["--mode", "generate", "--prompt", "life"])   # random:0 weights, no tokenizer
    assert main.tokenizer_dir(args) is None
    with pytest.raises(SystemExit, match="tokenizer"):
        main.encode_prompts(args)


def test_prompt_ids_and_random_batches():
    import main
    from mk_weights import random_token_ids
    args = main.parse_args(["--mode", "generate", "--prompt-ids", "1,2,3", "--prompt-ids", "4,5"])
    assert [p.tolist() for p in main.encode_prompts(args)] == [[1, 2, 3], [4, 5]]
    args = main.parse_args(["--mode", "generate", "--batch-size", "3", "--prompt-len", "7"])
    ps = main.encode_prompts(args)
    assert len(ps) == 3 and all(p.numel() == 7 for p in ps)
    for b, p in enumerate(ps):
        assert torch.equal(p, random_token_ids(7, seed=b))
    assert not torch.equal(ps[0], ps[1])


def test_generate_report_fields():
    import main
    lat = [float(x) for x in range(1, 101)]       # 1..100 ms
    r = main.generate_report(lat, tokens=8)
    assert r["latency_ms_p50"] == 51.0 and r["latency_ms_p90"] == 91.0 and r["latency_ms_p99"] == 100.0
    assert r["latency_ms_p100"] == 100.0 and r["latency_ms_avg"] == 50.5
    assert abs(r["throughput"] - 8 / 0.0505) < 1e-9


# ---------------------------------------------------------------------------
# the reference's flag set (main.py:34-105)
# ---------------------------------------------------------------------------

README_COMMANDS = [   # README.md:36-51 of the reference, with the flags its megakernel needs
    "--mode generate --model-path /home/ubuntu/kchern/models/llama-3.2-1b/ --compiled-model-path /tmp/llama1b_baseline",
    "--mode generate --enable-nki --model-path /home/ubuntu/kchern/models/llama-3.2-1b/ "
    "--compiled-model-path /tmp/llama1b_nki",
    "--mode validate --enable-nki --model-path /home/ubuntu/kchern/models/llama-3.2-1b/ "
    "--compiled-model-path /tmp/llama1b_nki",
]


@pytest.mark.parametrize("cmd", README_COMMANDS)
def test_reference_readme_commands_parse(cmd):
    import main
    for extra in ([], ["--tp-degree", "1", "--seq-len", "1024"]):
        a = main.parse_args(cmd.split() + extra)
        assert a.compiled_model_path.startswith("/tmp/llama1b_")
        assert a.tp_degree == 1 and a.seq_len == 1024 and a.max_length == 1024
        assert a.torch_dtype == torch.bfloat16


def test_every_reference_flag_is_accepted():
    """One command with every flag of the reference's parser at a value this
    build can honour."""
    import main
    from mk_validate import REFERENCE_TOL_MAP
    argv = ("--mode validate --llama llama --enable-nki --base-latency 500 --base-throughput 100 "
            "--model-path random:0 --compiled-model-path /tmp/x --benchmark --divergence-difference-tol 0.002 "
            "--num-tokens-to-check 8 --prompt hi --top-k 1 --top-p 1.0 --temperature 1.0 "
            "--global-topk 256 --do-sample True --dynamic --pad-token-id 2 --torch-dtype bfloat16 --batch-size 1 "
            "--padding-side left --seq-len 1024 --n-active-tokens 1024 --n-positions 131072 "
            "--max-context-length 1024 --max-new-tokens 16 --max-length 64 --rpl-reduce-dtype float32 "
            "--output-logits --vocab-parallel --fused-qkv --sequence-parallel-enabled --flash-decoding-enabled "
            "--on-device-sampling --enable-bucketing True --bucket-n-active-tokens "
            "--context-encoding-buckets 128 512 1024 --token-generation-buckets 512 1024 --tp-degree 1 "
            "--qkv-kernel-enabled --attn-kernel-enabled --mlp-kernel-enabled --quantized-kernel-lower-bound 1200 "
            "--mlp-kernel-fuse-residual-add").split()
    argv += ["--tol-map", "{None: (1e-5, 0.05), 1000: (1e-5, 0.03), 50: (1e-5, 0.03), 5: (1e-5, 0.03)}"]
    a = main.parse_args(argv)
    assert a.tol_map_parsed == REFERENCE_TOL_MAP
    assert a.divergence_difference_tol == 0.002 and a.num_tokens_to_check == 8
    assert a.max_length == 1024                   # set from --seq-len as main.py:543 does
    assert a.context_encoding_buckets == [128, 512, 1024] and a.rpl_reduce_dtype == torch.float32


@pytest.mark.parametrize("extra, what", [
    (["--torch-dtype", "float32"], "--torch-dtype"),
    (["--tp-degree", "2"], "--tp-degree"),
    (["--quantized-mlp-kernel-enabled"], "quantized"),
    (["--rmsnorm-quantize-kernel-enabled"], "quantized"),
    (["--llama", "my_llama"], "--llama"),
    (["--n-positions", "512"], "--n-positions"),
    (["--token-generation-buckets", "4096"], "--token-generation-buckets"),
    (["--tol-map", "{1000: 0.03}"], "--tol-map"),
    (["--tol-map", "__import__('os')"], "--tol-map"),
])
def test_values_this_build_cannot_honour_are_refused(extra, what):
    import main
    with pytest.raises(SystemExit, match=what):
        main.parse_args(["--mode", "generate"] + extra)


@pytest.mark.parametrize("mode", ["evaluate_single", "evaluate_all"])
def test_contest_modes_exit_out_of_scope(mode):
    import main
    with pytest.raises(SystemExit, match="out of scope"):
        main.parse_args(["--mode", mode, "--enable-nki"])


def test_module_selection_and_defaults():
    import main
    a = main.parse_args(["--mode", "generate", "--llama", "llama_with_megakernel"])
    assert a.enable_nki                        # the module name selects the megakernel model
    a = main.parse_args(["--mode", "generate", "--do-sample", "False"])
    assert a.do_sample is False
    # --max-new-tokens defaults to filling --seq-len after the longest prompt (max_length = seq_len)
    a = main.parse_args(["--mode", "generate", "--seq-len", "1024"])
    assert main.max_new_tokens(a, [torch.zeros(384), torch.zeros(100)]) == 641
    a = main.parse_args(["--mode", "generate", "--max-new-tokens", "7"])
    assert main.max_new_tokens(a, [torch.zeros(384)]) == 7


def test_reference_default_prompt_with_a_tokenizer(tok_dir):
    """No prompt and a tokenizer: the reference's default prompt (main.py:538-539)."""
    import main
    args = main.parse_args(["--mode", "generate", "--tokenizer-path", str(tok_dir)])
    ps = main.encode_prompts(args, main.args_tokenizer(args))
    assert [p.tolist() for p in ps] == [[8, 9, 3, 4, 5, 6, 7]]


def test_tokenizer_saved_into_the_compiled_model_path(tok_dir, tmp_path):
    import main
    out = tmp_path / "compiled"
    args = main.parse_args(["--mode", "generate", "--tokenizer-path", str(tok_dir),
                            "--compiled-model-path", str(out), "--padding-side", "left"])
    tok = main.args_tokenizer(args)
    assert tok.padding_side == "left"
    assert (out / "tokenizer.json").exists() or (out / "tokenizer_config.json").exists()


def test_compiled_model_path_manifest(tmp_path, small):
    """compile(path) writes the manifest load(path) checks (the reference's
    --compiled-model-path, main.py:46, 143-150)."""
    import json
    from llama_with_megakernel import LlamaInferenceConfig, NeuronConfigLlamaMK, NeuronLlamaForCausalLM
    prod, _ = small
    cfg = LlamaInferenceConfig(NeuronConfigLlamaMK(seq_len=64, device="cpu"), dims=prod)
    m = NeuronLlamaForCausalLM("random:0", cfg)
    with pytest.raises(FileNotFoundError, match="compile"):
        m.check_manifest(str(tmp_path / "none"))
    m.compile(str(tmp_path / "c"))
    m.check_manifest(str(tmp_path / "c"))
    other = NeuronLlamaForCausalLM("random:1", cfg)
    with pytest.raises(ValueError, match="model_path"):
        other.check_manifest(str(tmp_path / "c"))
    f = tmp_path / "c" / "mk_compiled.json"
    d = json.loads(f.read_text())
    d["libmk_sha256"] = "0" * 64
    f.write_text(json.dumps(d))
    with pytest.raises(ValueError, match="libmk_sha256"):
        m.check_manifest(str(tmp_path / "c"))


@pytest.mark.parametrize("extra", [["--do-sample", "True", "--top-k", "50"], ["--graph"]])
def test_benchmark_decode_loop_needs_greedy_batch1(extra):
    """``--decode-loop`` (one mk_decode_loop launch for the token generation) is
    greedy batch 1 only; sampling or a graph is refused before any GPU work."""
    import main
    with pytest.raises(SystemExit, match="--decode-loop"):
        main.main(["--mode", "benchmark", "--enable-nki", "--decode-loop", "--prompt-len", "8",
                   "--max-new-tokens", "4", "--seq-len", "64"] + extra)
