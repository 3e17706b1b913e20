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
