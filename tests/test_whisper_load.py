"""Whisper::load on the CPU (wsp_whisper_load): the four files of a model
directory parsed without touching the GPU — the prompt, the suppression masks,
the token limit, the audio context and the refusals of Whisper/Whisper.cpp:
121-254, 415-460 and Model/PreprocessorConfig.cpp:20-136
(Tests/Model/ConfigTests.cpp:165-216, Tests/Whisper/RefusalTests.cpp)."""

import json
import os

import numpy as np
import pytest

import helpers as H
from helpers import ensure_library


@pytest.fixture(scope="module", autouse=True)
def library():
    ensure_library()


@pytest.fixture(scope="module")
def tensors():
    return H.whisper_tensors()


@pytest.fixture()
def model(tmp_path, tensors):
    return H.write_whisper(tmp_path / "model", tensors)


def loaded(directory):
    from whispereacp_amd.whisper import Whisper
    return Whisper().load(str(directory))


def edit_json(path, change):
    with open(path) as f:
        document = json.load(f)
    change(document)
    with open(path, "w") as f:
        json.dump(document, f)


def test_prompt_masks_and_limits_from_the_files(model):
    w = loaded(model)
    assert w.prompt() == [264, 268]  # decoder_start_token_id, then <|notimestamps|>
    first, later = w.masks(272)
    assert np.flatnonzero(later).tolist() == [264, 265, 266, 267, 268]
    assert np.flatnonzero(first).tolist() == [32, 263, 264, 265, 266, 267, 268]
    assert w.end_of_text() == 263
    assert w.maximum_tokens == H.WHISPER_DECODER.max_positions - 2


def test_start_token_from_the_vocabulary_and_end_of_text_from_the_specials(model):
    # Without decoder_start_token_id / eos_token_id in config.json the prompt
    # opens with <|startoftranscript|> and the run stops on <|endoftext|>.
    def drop(c):
        del c["decoder_start_token_id"], c["eos_token_id"]
    edit_json(os.path.join(model, "config.json"), drop)
    w = loaded(model)
    assert w.prompt() == [264, 268]
    assert w.end_of_text() == 263


@pytest.mark.parametrize("missing", ["config.json", "preprocessor_config.json", "tokenizer.json",
                                     "model.safetensors"])
def test_a_missing_file_is_named(model, missing):
    from whispereacp_amd.decoder import ModelError
    os.remove(os.path.join(model, missing))
    with pytest.raises(ModelError, match=missing.replace(".", r"\.")):
        loaded(model)


@pytest.mark.parametrize("change,message", [
    (lambda p: p.update(mel_filters=p["mel_filters"][:-1]), "mel_filters is not"),
    (lambda p: p["mel_filters"][3].pop(), "ragged"),
    (lambda p: p.update(mel_filters=3), "not an array"),
    (lambda p: p.update(n_fft=63), "n_fft"),
    (lambda p: p.update(hop_length=0), "non-positive"),
    (lambda p: p.pop("nb_max_frames"), "nb_max_frames"),
])
def test_a_bad_preprocessor_config_is_refused(model, change, message):
    from whispereacp_amd.decoder import ModelError
    edit_json(os.path.join(model, "preprocessor_config.json"), change)
    with pytest.raises(ModelError, match=message):
        loaded(model)


def test_a_vocabulary_without_notimestamps_is_refused(model):
    from whispereacp_amd.decoder import ModelError

    def drop(t):
        t["added_tokens"] = [a for a in t["added_tokens"] if a["content"] != "<|notimestamps|>"]
    edit_json(os.path.join(model, "tokenizer.json"), drop)
    with pytest.raises(ModelError, match="notimestamps"):
        loaded(model)


def test_a_malformed_tokenizer_is_a_model_error(model):
    from whispereacp_amd.decoder import ModelError
    with open(os.path.join(model, "tokenizer.json"), "w") as f:
        f.write('{"model": {"vocab": [], "merges": []}}')
    with pytest.raises(ModelError):
        loaded(model)


def test_suppressed_tokens_outside_the_vocabulary_are_refused(model):
    from whispereacp_amd.decoder import ModelError
    edit_json(os.path.join(model, "config.json"), lambda c: c.update(suppress_tokens=[272]))
    with pytest.raises(ModelError, match="outside the vocabulary"):
        loaded(model)


def test_token_limit_and_audio_context_refusals(model):
    from whispereacp_amd.decoder import ModelError
    w = loaded(model)
    with pytest.raises(ModelError, match="at least one token"):
        w.set_maximum_tokens(0)
    w.set_maximum_tokens(7)
    assert w.maximum_tokens == 7
    with pytest.raises(ModelError, match="audio context"):
        w.set_audio_context(101)
    with pytest.raises(ModelError, match="audio context"):
        w.set_audio_context(-1)
    w.set_audio_context(100)
    w.set_audio_context(0)


def test_audio_context_for_samples(model):
    # Whisper/Whisper.cpp:450-460: (samples + margin) over hop * 2 samples a
    # position, rounded up to 64, held between the floor and the window; the
    # window here is 100 positions, below the 448 floor, so it is the window.
    w = loaded(model)
    assert w.audio_context_for_samples(0, 0.0) == 100
    assert w.audio_context_for_samples(3200, 2.5) == 100


def test_runs_need_a_prepared_model(model):
    from whispereacp_amd.decoder import ModelError
    w = loaded(model)
    with pytest.raises(ModelError, match="prepared"):
        w.transcribe(np.zeros(10, dtype=np.float32))
    from whispereacp_amd.whisper import Whisper
    with pytest.raises(ModelError, match="loaded"):
        Whisper().prompt()
    with pytest.raises(ModelError, match="loaded"):
        Whisper().prepare(0)


def test_shapes_that_disagree_between_the_files_are_refused_at_prepare(model):
    # Whisper::requireWhisperShapes runs before any device work.
    from whispereacp_amd.decoder import ModelError
    edit_json(os.path.join(model, "preprocessor_config.json"), lambda p: p.update(nb_max_frames=180))
    w = loaded(model)
    with pytest.raises(ModelError, match="mel frames"):
        w.prepare(0)


def test_text_for_tokens_needs_no_device(model):
    from whispereacp_amd.tokenizer import Tokenizer
    w = loaded(model)
    vocabulary = Tokenizer.from_file(os.path.join(model, "tokenizer.json"))
    tokens = vocabulary.encode(" hello world")
    assert w.text_for_tokens(tokens + [263]) == " hello world"
