"""The safetensors reader and the config.json decoder shape (CPU only).

The cases follow the reference's own loader tests (Tests/Model/SafeTensorsTests.cpp:
57-434): the widening values are the ones IEEE 754 binary16 and bfloat16
define for those bit patterns, every malformed header is refused when the file
is opened, and a mapped file parses to the tensors its bytes hold. Files
written by the `safetensors` package itself (an independent writer) read back
value for value."""

import json
import os
import struct

import numpy as np
import pytest

from helpers import ensure_library


@pytest.fixture(scope="module", autouse=True)
def library():
    ensure_library()


def assemble(header: str, blob: bytes = b"", length=None) -> bytes:
    h = header.encode()
    return struct.pack("<Q", len(h) if length is None else length) + h + blob


def open_bytes(data: bytes):
    from whispereacp_amd.decoder import SafeTensorsFile
    return SafeTensorsFile(data=data)


def refused(data: bytes):
    from whispereacp_amd.decoder import ModelError
    with pytest.raises(ModelError):
        open_bytes(data)


def f32(*values) -> bytes:
    return np.array(values, dtype="<f4").tobytes()


def u16(*values) -> bytes:
    return np.array(values, dtype="<u2").tobytes()


SINGLE = '{"weight":{"dtype":"F32","shape":[2,3],"data_offsets":[0,24]}}'


def test_single_tensor():
    f = open_bytes(assemble(SINGLE, f32(1, 2, 3, 4, 5, 6)))
    assert f.tensors() == [("weight", "F32", (2, 3), 24)]
    assert f.read_floats("weight", 6).tolist() == [1, 2, 3, 4, 5, 6]


def test_read_needs_room_for_every_value():
    from whispereacp_amd.decoder import ModelError
    f = open_bytes(assemble(SINGLE, f32(1, 2, 3, 4, 5, 6)))
    with pytest.raises(ModelError):
        f.read_floats("weight", 5)


def test_multiple_tensors_are_named_in_order_and_metadata_is_kept():
    header = ('{"__metadata__":{"format":"pt"},"b":{"dtype":"F32","shape":[2],"data_offsets":[8,16]},'
              '"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}')
    f = open_bytes(assemble(header, f32(1, 2, 3, 4)))
    assert [t[0] for t in f.tensors()] == ["a", "b"]
    assert f.metadata("format") == "pt"
    assert f.metadata("nope") is None
    assert f.read_floats("a", 2)[0] == 1 and f.read_floats("b", 2)[0] == 3


def test_empty_tensor_is_legal():
    f = open_bytes(assemble('{"empty":{"dtype":"F32","shape":[0,4],"data_offsets":[0,0]}}'))
    assert f.tensors() == [("empty", "F32", (0, 4), 0)]
    assert f.read_floats("empty", 0).size == 0


def test_half_widens_to_the_ieee_values():
    bits = u16(0x0000, 0x8000, 0x3C00, 0xC000, 0x3555, 0x0001, 0x03FF, 0x7BFF)
    v = open_bytes(assemble('{"w":{"dtype":"F16","shape":[8],"data_offsets":[0,16]}}', bits)).read_floats("w", 8)
    assert v[0] == 0 and v[1] == 0 and np.signbit(v[1])
    assert v[2] == 1 and v[3] == -2
    assert v[4] == np.float32(0.333251953125)
    assert v[5] == np.float32(2.0 ** -24) and v[6] == np.float32(1023 * 2.0 ** -24)
    assert v[7] == 65504


def test_half_infinities_and_nan():
    v = open_bytes(assemble('{"w":{"dtype":"F16","shape":[3],"data_offsets":[0,6]}}',
                            u16(0x7C00, 0xFC00, 0x7E00))).read_floats("w", 3)
    assert np.isposinf(v[0]) and np.isneginf(v[1]) and np.isnan(v[2])


def test_bfloat_widens_to_float():
    v = open_bytes(assemble('{"w":{"dtype":"BF16","shape":[5],"data_offsets":[0,10]}}',
                            u16(0x0000, 0x3F80, 0xC000, 0x4049, 0x7F80))).read_floats("w", 5)
    assert v[:3].tolist() == [0, 1, -2]
    assert v[3] == np.float32(3.140625) and np.isposinf(v[4])


def test_double_narrows_to_float():
    v = open_bytes(assemble('{"w":{"dtype":"F64","shape":[2],"data_offsets":[0,16]}}',
                            np.array([0.5, -0.25], "<f8").tobytes())).read_floats("w", 2)
    assert v.tolist() == [0.5, -0.25]


def test_integer_tensors_are_not_floats():
    from whispereacp_amd.decoder import ModelError
    f = open_bytes(assemble('{"w":{"dtype":"I32","shape":[2],"data_offsets":[0,8]}}',
                            np.array([1, 2], "<i4").tobytes()))
    assert f.tensors() == [("w", "I32", (2,), 8)]
    with pytest.raises(ModelError):
        f.read_floats("w", 2)


def test_unknown_tensor_lookup():
    from whispereacp_amd.decoder import ModelError
    with pytest.raises(ModelError):
        open_bytes(assemble(SINGLE, f32(1, 2, 3, 4, 5, 6))).read_floats("nope", 6)


MALFORMED = [
    b"\0" * 7,                                                      # shorter than the length prefix
    assemble("{}", length=3),                                        # header length past the end
    assemble("{}", length=2 ** 64 - 1),
    assemble("{not json"), assemble("[1,2,3]"), assemble(""),        # not a JSON object
    assemble('{"w":42}'),                                            # entry not an object
    assemble('{"w":{"shape":[1],"data_offsets":[0,4]}}', f32(1)),    # missing fields
    assemble('{"w":{"dtype":"F32","data_offsets":[0,4]}}', f32(1)),
    assemble('{"w":{"dtype":"F32","shape":[1]}}', f32(1)),
    assemble('{"w":{"dtype":"F8_E4M3","shape":[1],"data_offsets":[0,1]}}', b"\0"),  # unknown dtype
    assemble('{"w":{"dtype":32,"shape":[1],"data_offsets":[0,4]}}', f32(1)),
    assemble('{"w":{"dtype":"F32","shape":[1],"data_offsets":[4]}}', f32(1, 2)),     # malformed offsets
    assemble('{"w":{"dtype":"F32","shape":[1],"data_offsets":[8,4]}}', f32(1, 2)),
    assemble('{"w":{"dtype":"F32","shape":[1],"data_offsets":[-4,0]}}', f32(1, 2)),
    assemble('{"w":{"dtype":"F32","shape":[1],"data_offsets":[0,1.5]}}', f32(1, 2)),
    assemble('{"w":{"dtype":"F32","shape":[4],"data_offsets":[0,16]}}', f32(1, 2)),  # range leaves the blob
    assemble('{"w":{"dtype":"F32","shape":[3],"data_offsets":[0,8]}}', f32(1, 2)),   # shape disagrees
    assemble('{"w":{"dtype":"F16","shape":[2],"data_offsets":[0,8]}}', f32(1, 2)),
    assemble('{"w":{"dtype":"F32","shape":[-1],"data_offsets":[0,0]}}'),             # negative dimension
    assemble('{"w":{"dtype":"F32","shape":"2","data_offsets":[0,0]}}'),
    assemble('{"__metadata__":{"format":7}}'),                                       # metadata not strings
    assemble('{"__metadata__":7}'),
    assemble('{"w":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}} x', f32(1)),     # trailing text
]


@pytest.mark.parametrize("data", MALFORMED, ids=lambda d: str(len(d)))
def test_malformed_headers_are_refused_when_opened(data):
    refused(data)


def test_missing_file_and_directory_are_errors(tmp_path):
    from whispereacp_amd.decoder import ModelError, SafeTensorsFile
    with pytest.raises(ModelError):
        SafeTensorsFile(path=str(tmp_path / "no" / "model.safetensors"))
    with pytest.raises(ModelError):
        SafeTensorsFile(path=str(tmp_path))


def test_mapped_file_matches_its_bytes(tmp_path):
    from whispereacp_amd.decoder import SafeTensorsFile
    header = ('{"__metadata__":{"format":"pt"},"bias":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},'
              '"weight":{"dtype":"F16","shape":[4],"data_offsets":[8,16]}}')
    data = assemble(header, f32(0.25, -0.5) + u16(0x3C00, 0xC000, 0x0000, 0x4000))
    path = tmp_path / "mixed.safetensors"
    path.write_bytes(data)
    mapped, owned = SafeTensorsFile(path=str(path)), open_bytes(data)
    assert mapped.tensors() == owned.tensors()
    assert mapped.metadata("format") == "pt"
    for name, _, shape, _ in owned.tensors():
        n = int(np.prod(shape))
        assert np.array_equal(mapped.read_floats(name, n), owned.read_floats(name, n))


def test_files_from_the_safetensors_package_read_back(tmp_path):
    safetensors_numpy = pytest.importorskip("safetensors.numpy")
    rng = np.random.default_rng(3)
    tensors = {
        "model.decoder.layers.0.fc1.weight": rng.standard_normal((8, 4)).astype(np.float32),
        "half": rng.standard_normal(7).astype(np.float16),
        "double": rng.standard_normal((2, 2)),
        "ints": np.arange(5, dtype=np.int64),
    }
    path = tmp_path / "written.safetensors"
    safetensors_numpy.save_file(tensors, str(path), metadata={"format": "np"})
    from whispereacp_amd.decoder import ModelError, SafeTensorsFile
    f = SafeTensorsFile(path=str(path))
    listed = {name: (dtype, shape) for name, dtype, shape, _ in f.tensors()}
    assert listed == {"double": ("F64", (2, 2)), "half": ("F16", (7,)), "ints": ("I64", (5,)),
                      "model.decoder.layers.0.fc1.weight": ("F32", (8, 4))}
    assert f.metadata("format") == "np"
    assert np.array_equal(f.read_floats("model.decoder.layers.0.fc1.weight", 32),
                          tensors["model.decoder.layers.0.fc1.weight"].ravel())
    assert np.array_equal(f.read_floats("half", 7), tensors["half"].astype(np.float32))
    assert np.array_equal(f.read_floats("double", 4), tensors["double"].ravel().astype(np.float32))
    with pytest.raises(ModelError):
        f.read_floats("ints", 5)


SMALL_CONFIG = {"model_type": "whisper", "d_model": 768, "decoder_attention_heads": 12, "decoder_layers": 12,
                "decoder_ffn_dim": 3072, "vocab_size": 51865, "max_target_positions": 448,
                "max_source_positions": 1500, "encoder_layers": 12, "num_mel_bins": 80}


def test_shape_from_config(tmp_path):
    from whispereacp_amd.decoder import shape_from_config
    path = tmp_path / "config.json"
    path.write_text(json.dumps(SMALL_CONFIG))
    s = shape_from_config(str(path))
    assert (s.width, s.heads, s.layers, s.feed_forward_width, s.vocabulary_size, s.max_positions,
            s.cross_positions) == (768, 12, 12, 3072, 51865, 448, 1500)
    assert shape_from_config(str(path), 300).cross_positions == 300


@pytest.mark.parametrize("change", [{"d_model": None}, {"model_type": "bert"}, {"decoder_attention_heads": 7},
                                    {"decoder_layers": 0}, {"vocab_size": 1.5}])
def test_config_errors_are_model_errors(tmp_path, change):
    from whispereacp_amd.decoder import ModelError, shape_from_config
    config = dict(SMALL_CONFIG)
    for k, v in change.items():
        if v is None:
            del config[k]
        else:
            config[k] = v
    path = tmp_path / "config.json"
    path.write_text(json.dumps(config))
    with pytest.raises(ModelError):
        shape_from_config(str(path))
    with pytest.raises(ModelError):
        shape_from_config(os.path.join(str(tmp_path), "absent.json"))


def test_suppression_masks_and_prompt_ids_from_config(tmp_path):
    # Whisper::buildSuppressionMasks: later steps suppress suppress_tokens, the
    # first step those and begin_suppress_tokens (Whisper/Whisper.cpp:227-254).
    from whispereacp_amd.decoder import decoding_from_config
    config = dict(SMALL_CONFIG, suppress_tokens=[1, 2, 50256], begin_suppress_tokens=[220, 50256],
                  decoder_start_token_id=50258, eos_token_id=50257)
    path = tmp_path / "config.json"
    path.write_text(json.dumps(config))
    first, later, start, end = decoding_from_config(str(path), 51865)
    assert np.flatnonzero(later).tolist() == [1, 2, 50256]
    assert np.flatnonzero(first).tolist() == [1, 2, 220, 50256]
    assert set(np.unique(first)) <= {0.0, 1.0}
    assert (start, end) == (50258, 50257)


def test_config_without_decoding_fields_suppresses_nothing(tmp_path):
    from whispereacp_amd.decoder import decoding_from_config
    path = tmp_path / "config.json"
    path.write_text(json.dumps(SMALL_CONFIG))
    first, later, start, end = decoding_from_config(str(path), 51865)
    assert not first.any() and not later.any() and (start, end) == (-1, -1)


@pytest.mark.parametrize("change", [{"suppress_tokens": [51865]}, {"begin_suppress_tokens": [-1]},
                                    {"suppress_tokens": "1"}, {"eos_token_id": 1.5}])
def test_config_tokens_outside_the_vocabulary_are_refused(tmp_path, change):
    from whispereacp_amd.decoder import ModelError, decoding_from_config
    path = tmp_path / "config.json"
    path.write_text(json.dumps(dict(SMALL_CONFIG, **change)))
    with pytest.raises(ModelError):
        decoding_from_config(str(path), 51865)


# --- the same readers under AddressSanitizer and UndefinedBehaviorSanitizer ---

def sanitized_reader():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "_build", "safetensors_check")
    if not os.path.exists(path):
        import subprocess
        subprocess.run(["make", "-s", "_build/safetensors_check"], cwd=os.path.dirname(os.path.dirname(path)),
                       check=True)
    return path


def run_sanitized(mode, paths):
    import subprocess
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=86",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=87")
    result = subprocess.run([sanitized_reader(), mode] + [str(p) for p in paths], capture_output=True, text=True,
                            env=env, timeout=120)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "runtime error" not in result.stderr and "AddressSanitizer" not in result.stderr, result.stderr
    lines = result.stdout.splitlines()
    assert len(lines) == len(paths), result.stdout
    return lines


def test_malformed_headers_are_refused_under_sanitizers(tmp_path):
    # host/SafeTensors.cpp (its own JSON reader over a mapped file) built with
    # -fsanitize=address,undefined: every malformed header of the cases above
    # is refused with a ModelError and no sanitizer report, and well-formed
    # files (empty tensors, metadata, every widened dtype) read in full.
    bad = []
    for i, data in enumerate(MALFORMED):
        path = tmp_path / f"bad_{i}.safetensors"
        path.write_bytes(data)
        bad.append(path)
    lines = run_sanitized("open", bad)
    assert all(line.startswith("refused: ") for line in lines), lines
    good = {
        "single": assemble(SINGLE, f32(1, 2, 3, 4, 5, 6)),
        "empty": assemble('{"empty":{"dtype":"F32","shape":[0,4],"data_offsets":[0,0]}}'),
        "metadata": assemble('{"__metadata__":{"format":"pt"},"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}',
                             f32(1, 2)),
        "widened": assemble('{"h":{"dtype":"F16","shape":[2],"data_offsets":[0,4]},'
                            '"b":{"dtype":"BF16","shape":[2],"data_offsets":[4,8]},'
                            '"d":{"dtype":"F64","shape":[1],"data_offsets":[8,16]}}',
                            u16(0x3C00, 0x7C00) + u16(0x3F80, 0xC000) + np.array([0.5], "<f8").tobytes()),
    }
    paths = []
    for name, data in good.items():
        path = tmp_path / f"{name}.safetensors"
        path.write_bytes(data)
        paths.append(path)
    lines = run_sanitized("open", paths + [tmp_path / "absent.safetensors"])
    assert [line.split(",")[0] for line in lines[:4]] == ["read: 1 tensors", "read: 1 tensors", "read: 1 tensors",
                                                          "read: 3 tensors"], lines
    assert lines[4].startswith("refused: ")


def test_config_readers_under_sanitizers(tmp_path):
    good = tmp_path / "config.json"
    good.write_text(json.dumps(dict(SMALL_CONFIG, suppress_tokens=[1, 2], begin_suppress_tokens=[3])))
    broken = []
    for i, text in enumerate(["", "{", "[]", '{"d_model": "wide"}', json.dumps(dict(SMALL_CONFIG, d_model=-1)),
                              json.dumps(dict(SMALL_CONFIG, suppress_tokens=[10 ** 9]))]):
        path = tmp_path / f"broken_{i}.json"
        path.write_text(text)
        broken.append(path)
    lines = run_sanitized("config", [good] + broken)
    assert lines[0].startswith("config: 768 12 12 3072 51865 448 1500"), lines
    assert all(line.startswith("refused: ") for line in lines[1:]), lines
