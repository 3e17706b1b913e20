"""Shared test machinery: the reference's error measure, fixture loading and a
DecoderRun harness in the shape of Tests/Decoder/Common.h:530-667 (each call
synchronises, so a test reads what it wrote before deciding what to feed)."""

from __future__ import annotations

import json
import os
import sys
from typing import List, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
GOLDEN = os.path.join(HERE, "golden")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from whispereacp_amd import synthetic as S  # noqa: E402


def worst_error(actual, expected) -> float:
    """Tests/Encoder/Common.h:731-746: max |a - e| / (1 + |e|)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - e) / (1.0 + np.abs(e))))


def max_relative_error(actual, expected) -> float:
    """max |a - e| / max |e| — the logits measure of the decode configs."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return float(np.max(np.abs(a - e)) / max(np.max(np.abs(e)), 1e-300))


def from_hex(values) -> np.ndarray:
    return np.array([float.fromhex(v) for v in values], dtype=np.float64)


def load_fixture(name: str) -> dict:
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def oracle_tensors(decoder_file, shape: S.DecoderShape) -> List[np.ndarray]:
    return [decoder_file[n].floats() for n in S.canonical_names(shape.layers)]


def ensure_library():
    """Build the library only if nothing is built yet."""
    from whispereacp_amd import _native
    if not os.path.exists(_native.LIBRARY):
        from whispereacp_amd import build
        build.build(verbose=False)
    return _native.load()


class DecoderRun:
    """One decoder, its weights and the sequence state, read back per step."""

    def __init__(self, shape: S.DecoderShape, decoder_file, packing: str = "Float", fused: bool = True):
        import torch
        from whispereacp_amd.decoder import Decoder
        self.torch = torch
        self.shape = shape
        self.decoder = Decoder(shape, decoder_file, packing)
        self.decoder.set_fused(fused)
        self._keep = []

    def begin(self, encoder: np.ndarray, cross_position_count: int = 0):
        from whispereacp_amd.decoder import to_device
        enc = to_device(np.ascontiguousarray(encoder, dtype=np.float32))
        self._keep.append(enc)
        self.decoder.begin_sequence(enc, cross_position_count)
        self.torch.cuda.synchronize()

    def step(self, tokens: Sequence[int]):
        torch = self.torch
        from whispereacp_amd.decoder import to_device
        n = len(tokens)
        ids = to_device(np.array(tokens, dtype=np.int32))
        logits = torch.empty((n, self.shape.vocabulary_size), dtype=torch.float32, device="cuda")
        self.decoder.step(ids, n, logits)
        chosen = torch.empty(n, dtype=torch.int32, device="cuda")
        self.decoder.argmax(logits, n, self.shape.vocabulary_size, None, chosen)
        torch.cuda.synchronize()
        return self.decoder.read_hidden(n), logits.cpu().numpy(), chosen.cpu().numpy().tolist()

    @property
    def position(self) -> int:
        return self.decoder.position


# ---------------------------------------------------------------------------
# greedy runs on the GPU and in the oracle, and their comparison
# ---------------------------------------------------------------------------

# The reference's worst-error measure (Tests/Encoder/Common.h:731-746) on
# logits: the oracle reads the same stored weights widened, so only fp32
# accumulation separates the two.
WORST = 1e-4


def greedy_on_gpu(decoder, shape, encoder, prompt, steps, mask=None):
    """begin_sequence, the prompt in one step, then `steps` fused
    single-token steps fed back on the device; returns the tokens (prompt
    argmax first) and every single-token step's logits row."""
    import torch
    from whispereacp_amd.decoder import to_device
    V = shape.vocabulary_size
    enc = to_device(encoder)
    slots = torch.zeros(len(prompt) + steps + 1, dtype=torch.int32, device="cuda")
    slots[:len(prompt)] = torch.tensor(prompt, dtype=torch.int32, device="cuda")
    decoder.begin_sequence(enc)
    prompt_logits = torch.empty((len(prompt), V), dtype=torch.float32, device="cuda")
    decoder.step(slots[:len(prompt)], len(prompt), prompt_logits)
    decoder.argmax(prompt_logits[-1:], 1, V, None, slots[len(prompt):len(prompt) + 1])
    rows = torch.empty((steps, V), dtype=torch.float32, device="cuda")
    base = len(prompt)
    for j in range(1, steps + 1):
        decoder.step_and_sample(slots[base + j - 1:base + j], rows[j - 1:j], mask, slots[base + j:base + j + 1])
    torch.cuda.synchronize()
    tokens = slots[base:base + steps + 1].cpu().numpy().tolist()
    return tokens, rows.cpu().numpy()


def oracle_greedy(oracle, shape, decoder_file, encoder, prompt, steps, mask=None):
    """The oracle's greedy tokens and the logits rows of its single-token steps."""
    session = oracle.session(shape, oracle_tensors(decoder_file, shape))
    session.begin(encoder)
    _, logits = session.step(prompt)
    tokens = [int(np.argmax(logits[-1]))]
    rows = []
    for _ in range(steps):
        _, logits = session.step([tokens[-1]])
        rows.append(logits[0])
        row = logits[0] if mask is None else np.where(mask != 0, -np.inf, logits[0])
        tokens.append(int(np.argmax(row)))
    return tokens, np.array(rows)


def margin(row):
    top = np.sort(row)[-2:]
    return float(top[1] - top[0])


def check_run(gpu_tokens, gpu_rows, ref_tokens, ref_rows, relative_bar, mask=None):
    for j, (a, b) in enumerate(zip(gpu_tokens, ref_tokens)):
        assert a == b, (f"token {j} differs: gpu {a}, oracle {b}; oracle top-2 margin "
                        f"{margin(ref_rows[j - 1]) if j > 0 else float('nan'):.3g}")
    for j, row in enumerate(gpu_rows):
        allowed = row if mask is None else np.where(mask != 0, -np.inf, row)
        assert gpu_tokens[j + 1] == int(np.argmax(allowed)), f"step {j}: fused argmax is not the logits' argmax"
    rel = max(max_relative_error(g, r) for g, r in zip(gpu_rows, ref_rows))
    worst = max(worst_error(g, r) for g, r in zip(gpu_rows, ref_rows))
    assert rel <= relative_bar, rel
    assert worst <= WORST, worst
    return rel, worst


# ---------------------------------------------------------------------------
# a whole Whisper directory at reduced shapes, and the oracle's transcript
# ---------------------------------------------------------------------------

# The reduced mel of Tests/Mel/MelSpectrogramTests.cpp:27-36 (3200 samples,
# 64-point frames every 16, 200 frames, 12 bands) in front of a 128-wide,
# two-head encoder (head width 64, so the flash kernel runs) and a decoder
# over the 272-token fixture vocabulary (tests/golden/mini_tokenizer.json).
WHISPER_MEL = S.reduced_mel_shape()
WHISPER_ENCODER = S.EncoderShape(12, 128, 2, 2, 256, 200)
WHISPER_DECODER = S.DecoderShape(128, 2, 2, 256, 272, 32, 100)
# The fixture vocabulary's specials: 263 <|endoftext|>, 264
# <|startoftranscript|>, 265 <|en|>, 266-267 tasks, 268 <|notimestamps|>,
# 269-271 timestamps; id 32 is "Ġ" (a bare space).
WHISPER_DECODING = dict(suppress_tokens=[264, 265, 266, 267, 268], begin_suppress_tokens=[32, 263],
                        decoder_start_token_id=264, eos_token_id=263)


def whisper_tensors():
    tensors = dict(S.synthetic_encoder_file(WHISPER_ENCODER))
    tensors.update(S.synthetic_decoder_file(WHISPER_DECODER))
    return tensors


def whisper_filters():
    return S.triangular_filters(WHISPER_MEL.mel_count, WHISPER_MEL.bin_count)


def write_whisper(path, tensors=None, filters=None, **decoding):
    """The four files of a Whisper directory at the reduced shapes."""
    with open(os.path.join(GOLDEN, "mini_tokenizer.json")) as f:
        tokenizer_json = f.read()
    config = S.whisper_config(WHISPER_ENCODER, WHISPER_DECODER, **dict(WHISPER_DECODING, **decoding))
    pre = S.preprocessor_config(WHISPER_MEL, whisper_filters() if filters is None else filters)
    return S.write_whisper_directory(str(path), config, pre, tokenizer_json,
                                     whisper_tensors() if tensors is None else tensors)


def oracle_transcript(oracle, tensors, samples, first_mask, later_mask, prompt, end_of_text, maximum_tokens,
                      context=0):
    """Whisper::transcribe restated on the oracle: samples zero-padded to the
    window, oracle_mel_spectrogram, oracle_encode over the first
    min(2 * context, frames) frames, then the greedy loop of
    Whisper::decodeTranscript (Whisper/Whisper.cpp:1361-1443) on the KV-cached
    oracle decoder. Returns the tokens and the top-2 margin of every step."""
    m, e, d = WHISPER_MEL, WHISPER_ENCODER, WHISPER_DECODER
    window = np.zeros(m.sample_count, dtype=np.float32)
    window[:len(samples)] = samples
    mel = oracle.mel_spectrogram(window, whisper_filters(), m.fft_length, m.hop_length, m.frame_count)
    frames = e.input_frames if context == 0 else min(2 * context, e.input_frames)
    run = e.with_frames(frames)
    rows = oracle.encode(run, [tensors[n].floats() for n in S.encoder_canonical_names(e.layers)],
                         np.ascontiguousarray(mel[:, :frames].astype(np.float32)))
    session = oracle.session(d, [tensors[n].floats() for n in S.canonical_names(d.layers)])
    session.begin(rows.astype(np.float32), run.positions())
    limit = min(maximum_tokens, d.max_positions - len(prompt) + 1)
    tokens, margins = [], []
    _, logits = session.step(prompt)
    row, mask = logits[-1], first_mask
    for step in range(limit):
        if step > 0:
            _, logits = session.step([tokens[-1]])
            row, mask = logits[0], later_mask
        allowed = np.where(mask != 0, -np.inf, row)
        token = int(np.argmax(allowed))
        margins.append(margin(allowed[np.isfinite(allowed)]))
        if token == end_of_text:
            break
        tokens.append(token)
    return tokens, margins
