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
