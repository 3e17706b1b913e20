"""Whisper end to end on the MI355X (wsp_whisper_*): samples through the mel
front end, the encoder and the greedy decoder to the transcript, against the
same chain restated on the oracle (oracle_mel_spectrogram, oracle_encode, the
KV-cached oracle decoder under the two suppression masks). The reference's
own end-to-end fixtures (Tests/Whisper/TranscribeTests.cpp) need the real
tiny.en checkpoint and jfk.wav, which are not here; these run a synthetic
model at reduced shapes (helpers.WHISPER_*) over the reference's fixture
vocabulary, and check the properties those tests assert: the transcript
composes, holds no special token, obeys the first-step mask, stops at
end-of-text or the token limit, and repeats."""

import os

import numpy as np
import pytest

import helpers as H
from helpers import ensure_library
from whispereacp_amd import synthetic as S

pytestmark = pytest.mark.gpu

SAMPLES = S.tone_and_noise(2600)  # less than the 3200-sample window: the rest is zero padding


@pytest.fixture(scope="module", autouse=True)
def library():
    ensure_library()


@pytest.fixture(scope="module")
def tensors():
    return H.whisper_tensors()


@pytest.fixture(scope="module")
def model(tmp_path_factory, tensors):
    return H.write_whisper(tmp_path_factory.mktemp("whisper"), tensors)


def prepared(directory, pack=False):
    from whispereacp_amd.whisper import Whisper
    w = Whisper().load(str(directory))
    w.set_packs_weights(pack)
    return w.prepare(0)


def oracle_run(tensors, w, samples=SAMPLES, context=0, maximum=None, end_of_text=None):
    from oracle.binding import load_oracle
    first, later = w.masks(H.WHISPER_DECODER.vocabulary_size)
    return H.oracle_transcript(load_oracle(), tensors, samples, first, later, w.prompt(),
                               w.end_of_text() if end_of_text is None else end_of_text,
                               w.maximum_tokens if maximum is None else maximum, context)


def test_transcript_matches_the_oracle_chain(model, tensors):
    w = prepared(model)
    tokens = w.transcribe(SAMPLES)
    expected, margins = oracle_run(tensors, w)
    assert min(margins) > 1e-2, "the oracle's run has a near tie; pick other inputs"
    assert tokens == expected
    # No end-of-text within the window: the run ends at the limit,
    # min(max_target_positions - prompt, max_positions - prompt + 1).
    assert len(tokens) == H.WHISPER_DECODER.max_positions - 2
    assert len(set(tokens)) >= 4
    encode_seconds, decode_seconds, steps = w.timing()
    assert steps == len(tokens) and encode_seconds > 0 and decode_seconds > 0


def test_text_is_the_tokenizer_decode_of_the_tokens(model):
    from whispereacp_amd.tokenizer import Tokenizer
    w = prepared(model)
    tokens = w.transcribe(SAMPLES)
    vocabulary = Tokenizer.from_file(os.path.join(model, "tokenizer.json"))
    assert w.text_for_tokens(tokens) == vocabulary.decode(tokens)
    assert w.transcribe_text(SAMPLES) == vocabulary.decode(tokens)


def test_no_special_token_and_the_first_step_mask_holds(model):
    w = prepared(model)
    tokens = w.transcribe(SAMPLES)
    first, later = w.masks(H.WHISPER_DECODER.vocabulary_size)
    assert first[tokens[0]] == 0
    assert all(later[t] == 0 for t in tokens)
    assert all(t not in (263, 264, 265, 266, 267, 268) for t in tokens)


def test_end_of_text_stops_the_run(tmp_path, model, tensors):
    # eos_token_id names the token the full run samples at step 6 (its first
    # occurrence), so the run must stop there with the six before it.
    w = prepared(model)
    full = w.transcribe(SAMPLES)
    stop = next(i for i in range(6, len(full)) if full[i] not in full[:i])
    directory = H.write_whisper(tmp_path / "eos", tensors, eos_token_id=full[stop])
    w2 = prepared(directory)
    assert w2.end_of_text() == full[stop]
    tokens = w2.transcribe(SAMPLES)
    assert tokens == full[:stop]
    expected, _ = oracle_run(tensors, w2)
    assert tokens == expected
    assert w2.timing()[2] == stop + 1  # the end-of-text step was read too


def test_maximum_tokens_and_a_second_run_repeat(model):
    w = prepared(model)
    full = w.transcribe(SAMPLES)
    w.set_maximum_tokens(5)
    assert w.transcribe(SAMPLES) == full[:5]
    # Past the window the window's limit applies: step j samples into slot
    # prompt + j of a max_positions + 1 slot sequence, so max_positions -
    # prompt + 1 steps, one more than the default limit's max_positions - prompt.
    w.set_maximum_tokens(100)
    longest = w.transcribe(SAMPLES)
    assert len(longest) == H.WHISPER_DECODER.max_positions - 2 + 1 and longest[:len(full)] == full
    assert w.transcribe(SAMPLES) == longest


def test_reduced_audio_context_matches_the_oracle(model, tensors):
    w = prepared(model)
    w.set_audio_context(64)
    tokens = w.transcribe(SAMPLES)
    expected, margins = oracle_run(tensors, w, context=64, maximum=20)
    assert min(margins) > 1e-2
    assert tokens[:20] == expected
    _, positions, width = w.encoded_rows()
    assert (positions, width) == (64, H.WHISPER_ENCODER.width)


def test_packed_weights_transcribe_alike(tmp_path, tensors):
    # fp16-exact float weights: ExactHalf packs every projection and the
    # logits' copy, and the products see the same values.
    exact = {n: S.StoredTensor(t.name, "F32", t.extents, t.floats().astype(np.float16).astype(np.float32).ravel())
             for n, t in tensors.items()}
    directory = H.write_whisper(tmp_path / "exact", exact)
    plain = prepared(directory, pack=False).transcribe(SAMPLES)
    packed = prepared(directory, pack=True).transcribe(SAMPLES)
    assert plain == packed
    assert len(set(plain)) >= 4


def test_bf16_encoder_projections_transcribe_as_the_oracle(tmp_path, tensors):
    # BF16 encoder projections: the C++ loader holds them as exact scaled fp16
    # (wsp_encoder_scaled_halves), each with its own scale (q and fc2 are
    # rescaled by powers of two so no two neighbours share one), and the
    # transcript follows the oracle chain over the same bf16 values.
    factors = {"self_attn.q_proj.weight": 0.25, "self_attn.k_proj.weight": 1.0, "self_attn.v_proj.weight": 0.5,
               "self_attn.out_proj.weight": 1.0, "fc1.weight": 1.0, "fc2.weight": 2.0}
    bf16 = dict(tensors)
    for layer in range(H.WHISPER_ENCODER.layers):
        for suffix, factor in factors.items():
            name = S.encoder_layer_name(layer, suffix)
            t = tensors[name]
            bf16[name] = S.StoredTensor(t.name, "BF16", t.extents, S.store(t.floats().ravel() * factor, "BF16"))
    directory = H.write_whisper(tmp_path / "bf16", bf16)
    w = prepared(directory)
    tokens = w.transcribe(SAMPLES)
    expected, margins = oracle_run(bf16, w)
    assert min(margins) > 1e-2, "the oracle's run has a near tie; pick other inputs"
    assert tokens == expected
    assert len(set(tokens)) >= 4


def test_a_frequency_major_filterbank_transcribes_alike(tmp_path, model, tensors):
    directory = H.write_whisper(tmp_path / "transposed", tensors, filters=H.whisper_filters().T)
    assert prepared(directory).transcribe(SAMPLES) == prepared(model).transcribe(SAMPLES)


def test_silence_and_an_empty_run(model):
    w = prepared(model)
    assert w.transcribe(np.zeros(0, dtype=np.float32)) == w.transcribe(np.zeros(3200, dtype=np.float32))


def test_more_than_a_window_is_refused(model):
    from whispereacp_amd.decoder import ModelError
    w = prepared(model)
    with pytest.raises(ModelError, match="one window"):
        w.transcribe(np.zeros(3201, dtype=np.float32))
