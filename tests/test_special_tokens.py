"""The special tokens of a tokenizer.json and the transcript prompt built from
them (CPU only).

WSP::SpecialTokens follows Tokenizer/SpecialTokens.h:16-44 (filled from a
tokenizer.json's added_tokens, Tokenizer/Tokenizer.cpp:102-138) and the prompt
Whisper::buildPrompt (Whisper/Whisper.cpp:202-225). The cases follow the
reference's own tokenizer tests (Tests/Tokenizer/TokenizerTests.cpp:400-420 on
its fixture, 550-580 on a real tiny.en vocabulary's special block, which is
rebuilt here from the public layout since no real tokenizer.json is present)."""

import json

import pytest

from helpers import ensure_library, load_fixture

# The 99 language codes of the multilingual Whisper vocabularies, in token order.
LANGUAGES = ("en zh de es ru ko fr ja pt tr pl ca nl ar sv it id hi fi vi he uk el ms cs ro da hu ta no th ur hr "
             "bg lt la mi ml cy sk te fa lv bn sr az sl kn et mk br eu is hy ne mn bs kk sq sw gl mr pa si km sn "
             "yo so af oc ka be tg sd gu am yi lo uz fo ht ps tk nn mt sa lb my bo tl mg as tt haw ln ha ba jw su"
             ).split()


@pytest.fixture(scope="module", autouse=True)
def library():
    ensure_library()


def write_tokenizer(path, added):
    path.write_text(json.dumps({"version": "1.0", "added_tokens": added,
                                "model": {"type": "BPE", "vocab": {"a": 0}, "merges": []}}))
    return str(path)


def tiny_en_specials():
    """The special block of an English Whisper vocabulary: <|endoftext|> 50256,
    <|startoftranscript|> 50257, the 99 languages from 50258, the task and
    control tokens, then 1501 timestamps 0.00 .. 30.00 s from 50363."""
    added = [(50256, "<|endoftext|>"), (50257, "<|startoftranscript|>")]
    added += [(50258 + i, f"<|{code}|>") for i, code in enumerate(LANGUAGES)]
    added += [(50357, "<|translate|>"), (50358, "<|transcribe|>"), (50359, "<|startoflm|>"),
              (50360, "<|startofprev|>"), (50361, "<|nocaptions|>"), (50362, "<|notimestamps|>")]
    added += [(50363 + i, f"<|{i * 0.02:.2f}|>") for i in range(1501)]
    return [{"id": i, "content": c, "special": True} for i, c in added]


def test_fixture_special_tokens(tmp_path):
    from whispereacp_amd.decoder import special_tokens_from_file
    fx = load_fixture("mini_tokenizer_specials.json")
    t = special_tokens_from_file(write_tokenizer(tmp_path / "tokenizer.json", fx["added_tokens"]))
    for key, value in fx["expected"].items():
        assert t[key] == value, key
    assert t["language_count"] == 1
    assert abs(t["timestamp_interval"] - 0.02) < 1e-6
    # names the fixture lacks stay absent
    assert t["start_of_previous"] == -1 and t["no_speech"] == -1 and t["start_of_language_model"] == -1


def test_english_vocabulary_special_block(tmp_path):
    from whispereacp_amd.decoder import special_tokens_from_file
    t = special_tokens_from_file(write_tokenizer(tmp_path / "tokenizer.json", tiny_en_specials()))
    assert (t["end_of_text"], t["start_of_transcript"], t["translate"], t["transcribe"]) == (50256, 50257, 50357,
                                                                                             50358)
    assert (t["start_of_language_model"], t["start_of_previous"], t["no_speech"], t["no_timestamps"]) == (
        50359, 50360, 50361, 50362)
    assert t["english"] == 50258 and t["language_count"] == 99
    assert t["first_timestamp"] == 50363 and t["timestamp_count"] == 1501
    assert 0.0199 < t["timestamp_interval"] < 0.0201


def test_specials_are_found_in_any_order_and_ordinary_tokens_are_ignored(tmp_path):
    from whispereacp_amd.decoder import special_tokens_from_file
    added = list(reversed(tiny_en_specials()))
    added += [{"id": 7, "content": "hello"}, {"id": 8, "content": "<|toolongname|>"},
              {"id": 9, "content": "<|EN|>"}, {"id": 10, "content": "<|1.2.3|>"}, {"id": 11, "content": "<||>"}]
    t = special_tokens_from_file(write_tokenizer(tmp_path / "tokenizer.json", added))
    assert t["first_timestamp"] == 50363 and t["timestamp_count"] == 1501 and t["language_count"] == 99
    assert 0.0199 < t["timestamp_interval"] < 0.0201


@pytest.mark.parametrize("text", ["", "[]", '{"added_tokens": 3}', '{"added_tokens": [{"content": "<|en|>"}]}',
                                  '{"added_tokens": [{"id": -1, "content": "<|en|>"}]}',
                                  '{"added_tokens": [{"id": 5}]}', '{"added_tokens": [7]}'])
def test_malformed_tokenizer_files_are_refused(tmp_path, text):
    from whispereacp_amd.decoder import ModelError, special_tokens_from_file
    path = tmp_path / "tokenizer.json"
    path.write_text(text)
    with pytest.raises(ModelError):
        special_tokens_from_file(str(path))
    with pytest.raises(ModelError):
        special_tokens_from_file(str(tmp_path / "absent.json"))


CONFIG = {"model_type": "whisper", "d_model": 384, "decoder_attention_heads": 6, "decoder_layers": 4,
          "decoder_ffn_dim": 1536, "vocab_size": 51864, "max_target_positions": 448, "max_source_positions": 1500}


def test_prompt_prefers_the_config_start_token(tmp_path):
    # Whisper::buildPrompt: config.json's decoder_start_token_id when present,
    # else the vocabulary's <|startoftranscript|>; then <|notimestamps|>.
    from whispereacp_amd.decoder import prompt_from_files
    tokenizer = write_tokenizer(tmp_path / "tokenizer.json", tiny_en_specials())
    config = tmp_path / "config.json"
    config.write_text(json.dumps(dict(CONFIG, decoder_start_token_id=50257)))
    assert prompt_from_files(str(config), tokenizer) == [50257, 50362]
    config.write_text(json.dumps(dict(CONFIG, decoder_start_token_id=50258)))
    assert prompt_from_files(str(config), tokenizer) == [50258, 50362]
    config.write_text(json.dumps(CONFIG))
    assert prompt_from_files(str(config), tokenizer) == [50257, 50362]


def test_prompt_refuses_a_vocabulary_without_its_tokens(tmp_path):
    from whispereacp_amd.decoder import ModelError, prompt_from_files
    config = tmp_path / "config.json"
    config.write_text(json.dumps(CONFIG))
    no_start = [t for t in tiny_en_specials() if t["content"] != "<|startoftranscript|>"]
    with pytest.raises(ModelError, match="startoftranscript"):
        prompt_from_files(str(config), write_tokenizer(tmp_path / "a.json", no_start))
    no_notimestamps = [t for t in tiny_en_specials() if t["content"] != "<|notimestamps|>"]
    config.write_text(json.dumps(dict(CONFIG, decoder_start_token_id=50257)))
    with pytest.raises(ModelError, match="notimestamps"):
        prompt_from_files(str(config), write_tokenizer(tmp_path / "b.json", no_notimestamps))
    # a vocabulary of the wrong size for the model
    config.write_text(json.dumps(dict(CONFIG, vocab_size=1000)))
    with pytest.raises(ModelError, match="outside the vocabulary"):
        prompt_from_files(str(config), write_tokenizer(tmp_path / "c.json", tiny_en_specials()))


def test_tokenizer_reader_under_sanitizers(tmp_path):
    # The same reader built with -fsanitize=address,undefined (tests/native):
    # well-formed and malformed tokenizer files, no sanitizer report.
    from test_safetensors import run_sanitized
    good = write_tokenizer(tmp_path / "good.json", tiny_en_specials())
    broken = []
    for i, text in enumerate(["", "{", '{"added_tokens": 3}', '{"added_tokens": [{"id": 1.5, "content": "<|a|>"}]}',
                              '{"added_tokens": [{"id": 5, "content": 7}]}', '{"added_tokens": [null]}',
                              '{"added_tokens": [{"id": 99999999999999999999, "content": "<|en|>"}]}']):
        path = tmp_path / f"broken_{i}.json"
        path.write_text(text)
        broken.append(path)
    lines = run_sanitized("tokenizer", [good] + broken)
    assert lines[0] == "tokenizer: 50256 50257 50362, 99 languages, 1501 timestamps", lines
    assert all(line.startswith("refused: ") for line in lines[1:]), lines
