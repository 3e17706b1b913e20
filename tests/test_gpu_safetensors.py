"""Decoders built from safetensors files (wsp_decoder_create_from_file,
wsp_batch_decoder_create_from_file) against decoders built from the same
tensors handed over in memory: the same bytes reach the device, so greedy
tokens and every logits row are bit-equal. The files are written by the
`safetensors` package (F16, BF16 and F32 storage) with a HuggingFace
config.json beside them (Decoder/DecoderWeights.cpp:97-178 loads the same
names; Model/SafeTensors.cpp maps the file)."""

import json

import numpy as np
import pytest

from helpers import ensure_library, greedy_on_gpu
from whispereacp_amd import synthetic as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def library():
    ensure_library()


def save(decoder_file, path):
    import torch
    from safetensors.torch import save_file
    tensors = {}
    for name, t in decoder_file.items():
        data = np.ascontiguousarray(t.data).reshape(t.extents)
        if t.dtype == "F32":
            tensors[name] = torch.from_numpy(data.astype(np.float32))
        elif t.dtype == "F16":
            tensors[name] = torch.from_numpy(data.astype(np.float16))
        else:
            tensors[name] = torch.from_numpy(data.astype(np.uint16).view(np.int16)).view(torch.bfloat16)
    save_file(tensors, str(path), metadata={"format": "pt"})


def write_config(shape, path):
    path.write_text(json.dumps({
        "model_type": "whisper", "d_model": shape.width, "decoder_attention_heads": shape.heads,
        "decoder_layers": shape.layers, "decoder_ffn_dim": shape.feed_forward_width,
        "vocab_size": shape.vocabulary_size, "max_target_positions": shape.max_positions,
        "max_source_positions": shape.cross_positions}))


@pytest.mark.parametrize("dtype,packing", [("F16", "ExactHalf"), ("BF16", "ExactHalf"), ("F32", "Float"),
                                           ("F32", "ExactHalf")])
def test_decoder_from_file_decodes_like_the_tensor_table(tmp_path, dtype, packing):
    from whispereacp_amd.decoder import Decoder, shape_from_config
    shape = S.DecoderShape(256, 4, 2, 1024, 4099, 448, 300)
    f = S.workload_decoder_file(shape, dtype, 41)
    if dtype == "F32":
        # fp16-exact values, so ExactHalf packs them (the reference's rule)
        for t in f.values():
            t.data[...] = t.data.astype(np.float16).astype(np.float32)
    save(f, tmp_path / "model.safetensors")
    write_config(shape, tmp_path / "config.json")
    loaded_shape = shape_from_config(str(tmp_path / "config.json"))
    assert loaded_shape == shape
    enc = S.normal_encoder_output(300, shape.width, 9)
    prompt = [1, 2, 3, 4]
    from_file = Decoder(loaded_shape, packing=packing, path=str(tmp_path / "model.safetensors"))
    a_tokens, a_rows = greedy_on_gpu(from_file, shape, enc, prompt, 12)
    in_memory = Decoder(shape, f, packing=packing)
    b_tokens, b_rows = greedy_on_gpu(in_memory, shape, enc, prompt, 12)
    assert a_tokens == b_tokens
    assert np.array_equal(a_rows, b_rows)
    if packing == "ExactHalf":
        assert from_file.uses_fused == in_memory.uses_fused


def test_batch_from_file_decodes_like_the_tensor_table(tmp_path):
    import torch
    from whispereacp_amd.decoder import BatchedDecoder, to_device
    shape = S.DecoderShape(256, 4, 2, 1024, 4099, 448, 100)
    f = S.workload_decoder_file(shape, "BF16", 43)
    save(f, tmp_path / "model.safetensors")
    enc = to_device(np.stack([S.normal_encoder_output(100, shape.width, 20 + s) for s in range(3)]))
    outs = []
    for dec in (BatchedDecoder(shape, None, streams=3, path=str(tmp_path / "model.safetensors")),
                BatchedDecoder(shape, f, streams=3)):
        dec.begin(enc)
        slots = torch.zeros((9, 3), dtype=torch.int32, device="cuda")
        logits = torch.empty((8, 3, shape.vocabulary_size), dtype=torch.float32, device="cuda")
        dec.step(torch.tensor([[5, 6, 7, 8]] * 3, dtype=torch.int32, device="cuda"), 4,
                 torch.empty((12, shape.vocabulary_size), dtype=torch.float32, device="cuda"), None, slots[0])
        for j in range(8):
            dec.step(slots[j], 1, logits[j], None, slots[j + 1])
        torch.cuda.synchronize()
        outs.append((slots.cpu().numpy(), logits.cpu().numpy()))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])


def test_a_file_missing_a_tensor_is_a_model_error_naming_it(tmp_path):
    from whispereacp_amd.decoder import Decoder, ModelError
    shape = S.DecoderShape(128, 2, 1, 512, 1000, 16, 16)
    f = S.workload_decoder_file(shape, "F16", 44)
    del f["model.decoder.layers.0.fc2.bias"]
    save(f, tmp_path / "model.safetensors")
    with pytest.raises(ModelError, match="fc2.bias"):
        Decoder(shape, packing="ExactHalf", path=str(tmp_path / "model.safetensors"))


def test_greedy_from_a_checkpoint_directory_follows_the_config(tmp_path, oracle):
    # The product loop end to end from files: shape, suppression masks, start
    # and end-of-text ids from config.json, weights from model.safetensors, the
    # prompt [decoder_start_token_id, <|notimestamps|>] from config.json and
    # tokenizer.json (Whisper::buildPrompt) — against the oracle's greedy loop
    # under the same masks (first step: suppress_tokens and
    # begin_suppress_tokens; later: suppress_tokens) and the same stop.
    from helpers import oracle_tensors
    from whispereacp_amd.decoder import (Decoder, decoding_from_config, prompt_from_files, shape_from_config,
                                         to_device)
    shape = S.DecoderShape(256, 4, 2, 1024, 4099, 64, 120)
    f = S.workload_decoder_file(shape, "F16", 47)
    enc = S.normal_encoder_output(120, shape.width, 13)
    save(f, tmp_path / "model.safetensors")
    (tmp_path / "tokenizer.json").write_text(json.dumps({"added_tokens": [
        {"id": 4001, "content": "<|endoftext|>"}, {"id": 4000, "content": "<|startoftranscript|>"},
        {"id": 4002, "content": "<|en|>"}, {"id": 4050, "content": "<|notimestamps|>"},
        {"id": 4051, "content": "<|0.00|>"}, {"id": 4052, "content": "<|0.02|>"}]}))
    prompt = [4000, 4050]

    def oracle_run(first_ids, later_ids, end=None, limit=30):
        session = oracle.session(shape, oracle_tensors(f, shape))
        session.begin(enc)
        _, logits = session.step(prompt)
        first, later = np.zeros(shape.vocabulary_size), np.zeros(shape.vocabulary_size)
        first[first_ids + later_ids] = 1
        later[later_ids] = 1
        out = [int(np.argmax(np.where(first != 0, -np.inf, logits[-1])))]
        while len(out) < limit and out[-1] != end:
            _, logits = session.step([out[-1]])
            out.append(int(np.argmax(np.where(later != 0, -np.inf, logits[0]))))
        return out

    free = oracle_run([], [], limit=4)
    suppress, begin_suppress = [free[2]], [free[0]]
    masked = oracle_run(begin_suppress, suppress)
    end = masked[5]                               # an id the masked run meets
    expected = masked[:masked.index(end)]
    config = {"model_type": "whisper", "d_model": 256, "decoder_attention_heads": 4, "decoder_layers": 2,
              "decoder_ffn_dim": 1024, "vocab_size": 4099, "max_target_positions": 64, "max_source_positions": 120,
              "suppress_tokens": suppress, "begin_suppress_tokens": begin_suppress, "decoder_start_token_id": 4000,
              "eos_token_id": end}
    (tmp_path / "config.json").write_text(json.dumps(config))

    loaded = shape_from_config(str(tmp_path / "config.json"))
    first, later, start, eot = decoding_from_config(str(tmp_path / "config.json"), loaded.vocabulary_size)
    assert (start, eot) == (4000, end)
    assert prompt_from_files(str(tmp_path / "config.json"), str(tmp_path / "tokenizer.json")) == prompt
    decoder = Decoder(loaded, packing="ExactHalf", path=str(tmp_path / "model.safetensors"))
    tokens, _ = decoder.greedy(to_device(enc), prompt_from_files(str(tmp_path / "config.json"),
                                                                 str(tmp_path / "tokenizer.json")), 30,
                               end_of_text=eot, first_mask=to_device(first), later_mask=to_device(later))
    assert tokens == expected
    assert tokens[0] != free[0] and free[2] not in tokens
