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
