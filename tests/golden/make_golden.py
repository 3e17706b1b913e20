"""Writes the golden decoder fixtures under tests/golden/.

The expected outputs come from an independent float64 model written here with
torch library ops (``F.layer_norm``, exact ``F.gelu``, ``torch.softmax``,
``matmul``) from HuggingFace's WhisperDecoder.forward definition — not from
oracle/oracle.c — so the oracle is pinned against a second implementation
rather than against itself. Inputs are regenerated from seeds by
whispereacp_amd.synthetic; each fixture stores a SHA-256 of the stored input
bytes so a drifting generator is caught rather than silently re-based.

The encoder fixtures (encoder_*.json) come the
same way from a float64 WhisperEncoder.forward (``F.conv1d``, exact ``F.gelu``,
``F.layer_norm``, ``torch.softmax``).

Run: python tests/golden/make_golden.py          (every fixture)
     python tests/golden/make_golden.py encoder  (the encoder fixtures only)
"""

from __future__ import annotations

import dataclasses
import hashlib
import json
import math
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from whispereacp_amd import synthetic as S  # noqa: E402

EPS = float(np.float32(1e-5))  # the float epsilon, widened


def input_digest(decoder_file, encoder: np.ndarray) -> str:
    h = hashlib.sha256()
    for name in S.canonical_names(max(int(n.split(".")[3]) for n in decoder_file
                                      if n.startswith("model.decoder.layers.")) + 1):
        t = decoder_file[name]
        h.update(name.encode())
        h.update(t.dtype.encode())
        h.update(np.ascontiguousarray(t.data).tobytes())
    h.update(np.ascontiguousarray(encoder, dtype=np.float32).tobytes())
    return h.hexdigest()


def torch_decode(shape: S.DecoderShape, decoder_file, encoder: np.ndarray, tokens, cross_rows=0):
    """WhisperDecoder.forward in float64 over the whole sequence."""
    W = {n: torch.from_numpy(t.floats().astype(np.float64)) for n, t in decoder_file.items()}
    d, H = shape.width, shape.heads
    D = d // H
    T = len(tokens)
    rows = cross_rows or shape.cross_positions
    enc = torch.from_numpy(encoder.astype(np.float64))[:rows]

    h = W[S.MODEL_NAMES[0]][torch.tensor(tokens)] + W[S.MODEL_NAMES[1]][:T]

    def ln(x, prefix):
        return F.layer_norm(x, (d,), W[prefix + ".weight"], W[prefix + ".bias"], eps=EPS)

    def attention(q, k, v, causal):
        qh = q.view(q.shape[0], H, D).transpose(0, 1)
        kh = k.view(k.shape[0], H, D).transpose(0, 1)
        vh = v.view(v.shape[0], H, D).transpose(0, 1)
        scores = torch.matmul(qh, kh.transpose(1, 2)) * (1.0 / math.sqrt(D))
        if causal:
            mask = torch.ones(q.shape[0], k.shape[0], dtype=torch.bool).triu(1)
            scores = scores.masked_fill(mask, float("-inf"))
        probs = torch.softmax(scores, dim=-1)
        return torch.matmul(probs, vh).transpose(0, 1).reshape(q.shape[0], d)

    for layer in range(shape.layers):
        p = lambda s: S.layer_name(layer, s)  # noqa: E731
        n = ln(h, p("self_attn_layer_norm"))
        q = n @ W[p("self_attn.q_proj.weight")].T + W[p("self_attn.q_proj.bias")]
        k = n @ W[p("self_attn.k_proj.weight")].T
        v = n @ W[p("self_attn.v_proj.weight")].T + W[p("self_attn.v_proj.bias")]
        a = attention(q, k, v, True)
        h = h + a @ W[p("self_attn.out_proj.weight")].T + W[p("self_attn.out_proj.bias")]

        n = ln(h, p("encoder_attn_layer_norm"))
        q = n @ W[p("encoder_attn.q_proj.weight")].T + W[p("encoder_attn.q_proj.bias")]
        k = enc @ W[p("encoder_attn.k_proj.weight")].T
        v = enc @ W[p("encoder_attn.v_proj.weight")].T + W[p("encoder_attn.v_proj.bias")]
        a = attention(q, k, v, False)
        h = h + a @ W[p("encoder_attn.out_proj.weight")].T + W[p("encoder_attn.out_proj.bias")]

        n = ln(h, p("final_layer_norm"))
        f = F.gelu(n @ W[p("fc1.weight")].T + W[p("fc1.bias")], approximate="none")
        h = h + f @ W[p("fc2.weight")].T + W[p("fc2.bias")]

    hidden = ln(h, "model.decoder.layer_norm")
    logits = hidden @ W[S.MODEL_NAMES[0]].T
    return hidden.numpy(), logits.numpy()


def hexes(a: np.ndarray):
    return [float(x).hex() for x in np.asarray(a, dtype=np.float64).ravel()]


def shape_dict(shape: S.DecoderShape):
    return dict(zip(("width", "heads", "layers", "feed_forward_width", "vocabulary_size",
                     "max_positions", "cross_positions"), shape.as_tuple()))


def write(name: str, payload: dict):
    path = os.path.join(HERE, name)
    with open(path, "w") as f:
        json.dump(payload, f, indent=1)
    print("wrote", path)


def prompt_fixture(name, storage, encoder_kind, tokens, cross_rows=0):
    shape = S.small_decoder_shape()
    decoder_file = S.synthetic_decoder_file(shape, storage)
    encoder = S.synthetic_encoder_output(shape)
    if encoder_kind == "second":
        encoder = (np.float32(-0.5) * encoder + np.float32(0.25)).astype(np.float32)
    if cross_rows:
        short = S.DecoderShape(*(shape.as_tuple()[:-1] + (cross_rows,)))
        encoder = S.synthetic_encoder_output(short)
        padded = np.full((shape.cross_positions, shape.width), -1234.0, dtype=np.float32)
        padded[:cross_rows] = encoder
        encoder = padded
    hidden, logits = torch_decode(shape, decoder_file, encoder, tokens, cross_rows)
    write(name, dict(
        shape=shape_dict(shape), weights=dict(kind="reference-fixture", storage=storage),
        encoder=encoder_kind, cross_rows=cross_rows, tokens=tokens,
        input_sha256=input_digest(decoder_file, encoder),
        hidden=hexes(hidden), logits=hexes(logits)))


def logits_sample(row: np.ndarray):
    """The indices a fixture keeps of a vocabulary-long logits row: the 32
    largest (in order) and every 97th, so a 51865-wide row stays a few KB."""
    top = np.argsort(-row, kind="stable")[:32].tolist()
    return sorted(set(top) | set(range(0, row.shape[0], 97)))


def greedy_fixture(name, shape, dtype, seed, encoder_seed, prompt, steps):
    if dtype == "spread":
        decoder_file = S.synthetic_decoder_file(shape, "Float")
        encoder = S.synthetic_encoder_output(shape)
    else:
        decoder_file = S.workload_decoder_file(shape, dtype, seed)
        encoder = S.normal_encoder_output(shape.cross_positions, shape.width, encoder_seed)
    sequence = list(prompt)
    tokens, margins = [], []
    logits = None
    for _ in range(steps):
        _, logits = torch_decode(shape, decoder_file, encoder, sequence)
        row = logits[-1]
        best = int(np.argmax(row))
        second = float(np.max(np.delete(row, best)))
        tokens.append(best)
        margins.append(float(row[best]) - second)
        sequence.append(best)
    row = logits[-1]
    keep = logits_sample(row) if row.shape[0] > 4096 else list(range(row.shape[0]))
    write(name, dict(
        shape=shape_dict(shape), weights=dict(kind="workload", dtype=dtype, seed=seed),
        encoder_seed=encoder_seed, prompt=list(prompt), steps=steps,
        input_sha256=input_digest(decoder_file, encoder),
        tokens=tokens, margins=margins, last_logits_index=keep, last_logits=hexes(row[keep])))


REFERENCE_TOKENIZER_FIXTURE = "/root/reference/Tests/Tokenizer/Fixtures/MiniTokenizer.json"


def tokenizer_specials_fixture(name):
    """The added_tokens of the reference's own tokenizer test fixture
    (Tests/Tokenizer/Fixtures/MiniTokenizer.json, data its tests load), kept
    with the values its special-token test asserts
    (Tests/Tokenizer/TokenizerTests.cpp:400-420)."""
    with open(REFERENCE_TOKENIZER_FIXTURE) as f:
        source = json.load(f)
    write(name, dict(
        source="Tests/Tokenizer/Fixtures/MiniTokenizer.json (added_tokens only)",
        added_tokens=[{"id": t["id"], "content": t["content"], "special": t.get("special", True)}
                      for t in source["added_tokens"]],
        expected=dict(end_of_text=263, start_of_transcript=264, translate=266, transcribe=267, no_timestamps=268,
                      english=265, first_timestamp=269, timestamp_count=3)))


def torch_encode(shape: S.EncoderShape, encoder_file, mel: np.ndarray):
    """WhisperEncoder.forward in float64 from torch library ops (conv1d with
    padding 1, exact gelu, layer_norm, softmax), over the first
    shape.input_frames frames of ``mel``."""
    W = {n: torch.from_numpy(t.floats().astype(np.float64)) for n, t in encoder_file.items()}
    d, H = shape.width, shape.heads
    D = d // H
    x = torch.from_numpy(mel[:, :shape.input_frames].astype(np.float64))[None]
    x = F.gelu(F.conv1d(x, W["model.encoder.conv1.weight"], W["model.encoder.conv1.bias"], stride=1, padding=1))
    x = F.gelu(F.conv1d(x, W["model.encoder.conv2.weight"], W["model.encoder.conv2.bias"], stride=2, padding=1))
    h = x[0].T + W["model.encoder.embed_positions.weight"][:x.shape[2]]
    P = h.shape[0]

    def ln(v, prefix):
        return F.layer_norm(v, (d,), W[prefix + ".weight"], W[prefix + ".bias"], eps=EPS)

    for layer in range(shape.layers):
        p = lambda s: S.encoder_layer_name(layer, s)  # noqa: E731
        n = ln(h, p("self_attn_layer_norm"))
        q = (n @ W[p("self_attn.q_proj.weight")].T + W[p("self_attn.q_proj.bias")]).view(P, H, D).transpose(0, 1)
        k = (n @ W[p("self_attn.k_proj.weight")].T).view(P, H, D).transpose(0, 1)
        v = (n @ W[p("self_attn.v_proj.weight")].T + W[p("self_attn.v_proj.bias")]).view(P, H, D).transpose(0, 1)
        probs = torch.softmax(torch.matmul(q, k.transpose(1, 2)) * (1.0 / math.sqrt(D)), dim=-1)
        a = torch.matmul(probs, v).transpose(0, 1).reshape(P, d)
        h = h + a @ W[p("self_attn.out_proj.weight")].T + W[p("self_attn.out_proj.bias")]
        n = ln(h, p("final_layer_norm"))
        g = F.gelu(n @ W[p("fc1.weight")].T + W[p("fc1.bias")])
        h = h + g @ W[p("fc2.weight")].T + W[p("fc2.bias")]
    return ln(h, "model.encoder.layer_norm").numpy()


def encoder_digest(encoder_file, names, mel: np.ndarray) -> str:
    h = hashlib.sha256()
    for name in names:
        t = encoder_file[name]
        h.update(name.encode())
        h.update(t.dtype.encode())
        h.update(np.ascontiguousarray(t.data).tobytes())
    h.update(np.ascontiguousarray(mel, dtype=np.float32).tobytes())
    return h.hexdigest()


def encoder_fixture(name, shape, kind, storage_or_dtype, seed=0, positions=0):
    """The reference test-suite's small encoder (kind "reference-fixture") or
    a workload-style one; ``positions`` runs a reduced context as the
    reference's reducedContextMatchesTheShorterShape does: the expected rows
    are the shorter shape's own encode over the mel's first frames."""
    if kind == "reference-fixture":
        encoder_file = S.synthetic_encoder_file(shape, storage_or_dtype)
        mel = S.synthetic_mel(shape)
    else:
        encoder_file = S.workload_encoder_file(shape, storage_or_dtype, seed)
        mel = S.normal_mel(shape, seed + 500)
    run = shape.with_frames(shape.frames_for_positions(positions)) if positions else shape
    rows = torch_encode(run, encoder_file, mel)
    write(name, dict(
        shape=dataclasses.asdict(shape), weights=dict(kind=kind, storage=storage_or_dtype, seed=seed),
        positions=positions, input_sha256=encoder_digest(encoder_file, S.encoder_canonical_names(shape.layers), mel),
        rows=hexes(rows)))


def encoder_fixtures():
    small = S.small_encoder_shape()
    encoder_fixture("encoder_small_float.json", small, "reference-fixture", "Float")
    encoder_fixture("encoder_small_packed_half.json", small, "reference-fixture", "PackedHalf")
    encoder_fixture("encoder_small_all_half.json", small, "reference-fixture", "EveryTensorHalf")
    encoder_fixture("encoder_small_reduced.json", small, "reference-fixture", "Float", positions=3)
    # Whisper's 80 mel bins and head width 64 at a reduced width and window.
    mid = S.EncoderShape(80, 128, 2, 2, 512, 64)
    encoder_fixture("encoder_mid_f16.json", mid, "workload", "F16", seed=3000)


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "encoder":
        torch.set_default_dtype(torch.float64)
        encoder_fixtures()
        return
    if os.path.exists(REFERENCE_TOKENIZER_FIXTURE):
        tokenizer_specials_fixture("mini_tokenizer_specials.json")
    torch.set_default_dtype(torch.float64)
    prompt_fixture("small_shape_prompt_float.json", "Float", "sweep", [5, 17, 3, 11])
    prompt_fixture("small_shape_prompt_packed_half.json", "PackedHalf", "sweep", [5, 17, 3, 11])
    prompt_fixture("small_shape_prompt_all_half.json", "EveryTensorHalf", "sweep", [5, 17, 3, 11])
    prompt_fixture("small_shape_second_sequence.json", "Float", "second", [7, 2, 9])
    prompt_fixture("small_shape_reduced_cross.json", "Float", "sweep", [5, 17, 3, 11, 5],
                   cross_rows=3)
    # A full-size vocabulary and four layers: with random N(0, 0.02) weights
    # the greedy sequence of a narrow vocabulary settles on one token at once;
    # these seeds keep four to six distinct tokens over the 13.
    mid = S.DecoderShape(256, 4, 4, 1024, 51865, 32, 64)
    greedy_fixture("mid_shape_greedy_f32.json", mid, "F32", 35, 36, [1, 2, 3, 4], 12)
    greedy_fixture("mid_shape_greedy_bf16.json", mid, "BF16", 40, 41, [1, 2, 3, 4], 12)
    greedy_fixture("mid_shape_greedy_f16.json", mid, "F16", 11, 12, [1, 2, 3, 4], 12)
    greedy_fixture("mid_shape_greedy_spread.json", S.DecoderShape(64, 4, 2, 256, 97, 24, 40), "spread", 0, 0,
                   [3, 1, 4, 1], 16)
    # The tiny.en configuration the reference runs on the CPU: d 384, 6 heads,
    # 4 layers, vocab 51864, fp32 weights, 1500 encoder rows, the 4-token
    # start-of-transcript prefix and 25 greedy steps after the prompt's.
    w = S.WORKLOADS["tiny.en"]
    greedy_fixture("tiny_en_greedy.json", S.workload_shape("tiny.en"), w["dtype"], w["seed"], 7,
                   S.SOT_PREFIX[w["vocab"]], w["steps"] + 1)
    encoder_fixtures()


if __name__ == "__main__":
    main()
