"""The C ABI on the CPU: the library loads, exports every entry point the
headers declare, and refuses bad arguments before touching a device."""

import ctypes
import os
import re

import pytest

from helpers import ROOT, ensure_library

HEADERS = [os.path.join(ROOT, "include", "wsp_hip.h"), os.path.join(ROOT, "include", "wsp_decoder.h")]


def declared_functions():
    names = []
    for path in HEADERS:
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[a-z_]+\*?\s+\*?(wsp_[a-z_]+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_headers_declare_the_entry_points():
    names = declared_functions()
    for required in ("wsp_hip_ctx_create", "wsp_hip_linear", "wsp_hip_layernorm", "wsp_hip_embed",
                     "wsp_hip_attention", "wsp_hip_argmax", "wsp_hip_project_cross_kv", "wsp_hip_decoder_step",
                     "wsp_decoder_create", "wsp_decoder_step", "wsp_decoder_greedy"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ensure_library()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_signatures_cover_every_declared_symbol():
    from whispereacp_amd import _native
    assert set(declared_functions()) == set(_native.SIGNATURES)


def test_context_refuses_bad_arguments_without_a_device():
    from whispereacp_amd import _native as N
    lib = ensure_library()
    handle = ctypes.c_void_p()
    assert lib.wsp_hip_ctx_create(None, 0, None, ctypes.byref(handle)) == N.WSP_ERR_ARGUMENT
    bad = N.wsp_decoder_shape(10, 3, 1, 16, 24, 16, 6)  # width not divisible by heads
    assert lib.wsp_hip_ctx_create(ctypes.byref(bad), 0, None, ctypes.byref(handle)) == N.WSP_ERR_SHAPE
    zero = N.wsp_decoder_shape(8, 2, 0, 16, 24, 16, 6)
    assert lib.wsp_hip_ctx_create(ctypes.byref(zero), 0, None, ctypes.byref(handle)) == N.WSP_ERR_SHAPE
    assert lib.wsp_hip_linear(None, None, 1, 1, None, 0, None, None, 1, 0) == N.WSP_ERR_ARGUMENT
    assert lib.wsp_hip_argmax(None, None, 1, 1, None, None) == N.WSP_ERR_ARGUMENT
    assert lib.wsp_hip_decoder_step(None, None, None, 0, 1, None, None, None, None) == N.WSP_ERR_ARGUMENT
    assert lib.wsp_hip_step_report(None, None, None) == N.WSP_ERR_ARGUMENT
    assert lib.wsp_hip_step_report_next(None, None) == N.WSP_ERR_ARGUMENT
    assert lib.wsp_hip_last_error(None) == b"no context"


def test_static_attention_refuses_before_touching_a_device():
    # Arguments and the fixed partials capacity are checked before any device
    # call, with the reason in the caller's buffer.
    from whispereacp_amd import _native as N
    lib = ensure_library()
    error = ctypes.create_string_buffer(256)
    p = ctypes.c_void_p(16)
    assert lib.wsp_hip_attention_static(None, 1, p, p, 1, 64, 1, 1, 1.0, p, None, error, 256) == N.WSP_ERR_ARGUMENT
    assert lib.wsp_hip_attention_static(p, 1, p, p, 1, 128, 1, 1, 1.0, p, None, error, 256) == N.WSP_ERR_LOGIC
    assert lib.wsp_hip_attention_static(p, 5, p, p, 4, 64, 1, 1, 1.0, p, None, error, 256) == N.WSP_ERR_SHAPE
    # 20 heads x 4096 queries over 4096 keys: four chunks of partials, 21.6M floats
    status = lib.wsp_hip_attention_static(p, 4096, p, p, 4096, 1280, 20, 0, 1.0, p, None, error, 256)
    assert status == N.WSP_ERR_CAPACITY
    assert b"without allocation" in error.value


def test_decoder_refuses_a_bad_shape_as_a_model_error():
    from whispereacp_amd import _native as N
    from whispereacp_amd.decoder import Decoder, ModelError
    from whispereacp_amd import synthetic as S
    ensure_library()
    with pytest.raises(ModelError):
        Decoder(S.DecoderShape(10, 3, 1, 16, 24, 16, 6), {})
    assert N.load().wsp_decoder_create(None, None, 0, 0, 0, None, None) == N.WSP_ERR_ARGUMENT


def test_loader_names_a_missing_or_misshapen_table_before_any_upload():
    # embed_tokens is checked before anything reaches the device, so these run
    # on the CPU (Tests/Decoder/DecoderWeightsTests.cpp:149-254).
    from whispereacp_amd.decoder import Decoder, ModelError
    from whispereacp_amd import synthetic as S
    ensure_library()
    shape = S.small_decoder_shape()
    good = S.synthetic_decoder_file(shape, "Float")
    missing = dict(good)
    del missing["model.decoder.embed_tokens.weight"]
    with pytest.raises(ModelError, match="embed_tokens"):
        Decoder(shape, missing)
    short = dict(good)
    t = good["model.decoder.embed_tokens.weight"]
    short["model.decoder.embed_tokens.weight"] = S.StoredTensor(t.name, t.dtype, (shape.vocabulary_size - 1,
                                                                                 shape.width),
                                                                 t.data[: (shape.vocabulary_size - 1) * shape.width])
    with pytest.raises(ModelError, match="embed_tokens"):
        Decoder(shape, short)
    odd = dict(good)
    odd["model.decoder.embed_tokens.weight"] = S.StoredTensor(t.name, "I8", t.extents, t.data)
    with pytest.raises(ModelError, match="I8"):
        Decoder(shape, odd)


def test_batch_refuses_bad_arguments_without_a_device():
    from whispereacp_amd import _native as N
    lib = ensure_library()
    handle = ctypes.c_void_p()
    shape = N.wsp_decoder_shape(1024, 16, 24, 4096, 51865, 448, 1500)
    assert lib.wsp_batch_create(None, 16, 1, N.WSP_F16, 0, None, ctypes.byref(handle)) == N.WSP_ERR_ARGUMENT
    assert lib.wsp_batch_create(ctypes.byref(shape), 0, 1, N.WSP_F16, 0, None, ctypes.byref(handle)) == N.WSP_ERR_ARGUMENT
    # fp32 projections have no matrix-core form here
    assert lib.wsp_batch_create(ctypes.byref(shape), 16, 1, N.WSP_F32, 0, None, ctypes.byref(handle)) == N.WSP_ERR_LOGIC
    # more than 128 rows per step
    assert lib.wsp_batch_create(ctypes.byref(shape), 33, 4, N.WSP_F16, 0, None, ctypes.byref(handle)) == N.WSP_ERR_CAPACITY
    wide = N.wsp_decoder_shape(1024, 8, 24, 4096, 51865, 448, 1500)  # heads 128 wide
    assert lib.wsp_batch_create(ctypes.byref(wide), 16, 1, N.WSP_F16, 0, None, ctypes.byref(handle)) == N.WSP_ERR_SHAPE
    assert not handle.value
    assert lib.wsp_batch_step(None, None, None, 1, None, None, None, None) == N.WSP_ERR_ARGUMENT
    assert lib.wsp_batch_begin(None, None, N.WSP_F16, None, 0) == N.WSP_ERR_ARGUMENT
    assert lib.wsp_batch_last_error(None) == b"null batch"
    assert lib.wsp_batch_position(None) == -1


def net_refusals():
    path = os.path.join(ROOT, "tests", "native", "_build", "net_refusals")
    if not os.path.exists(path):
        import subprocess
        ensure_library()
        subprocess.run(["make", "-s", "_build/net_refusals"], cwd=os.path.join(ROOT, "tests", "native"), check=True)
    return path


def test_net_refusals_without_a_device():
    # WSP::HipNet refuses with std::logic_error what it can refuse before
    # anything is prepared: a recording, a cache or an op before prepare(), the
    # encoder-only ops, a shape past four extents.
    import subprocess
    result = subprocess.run([net_refusals(), "host"], capture_output=True, text=True, timeout=60)
    assert result.returncode == 0, result.stdout + result.stderr
    assert result.stdout.count("ok ") == 7, result.stdout


def test_batch_split_sizing_and_refusals_on_the_host():
    # The batched step's split products refuse a launch whose partials or
    # counters would overflow the buffers reserved at create; the sizing rule
    # and the refusal are host code (csrc/batch_plan.h), checked here on the
    # CPU under ASan/UBSan: every planned launch fits, one column group, row
    # tile or split more does not.
    import subprocess
    path = os.path.join(ROOT, "tests", "native", "_build", "batch_plan_check")
    subprocess.run(["make", "-s", "_build/batch_plan_check"], cwd=os.path.join(ROOT, "tests", "native"), check=True)
    result = subprocess.run([path], capture_output=True, text=True, timeout=60)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "FAIL" not in result.stdout and result.stdout.count("ok ") == 32, result.stdout


def test_headers_compile_as_c99(tmp_path):
    # The C ABI is meant for C callers (cgo, ctypes, plain C): both headers
    # must stand alone as C99, with no C++ in their C view.
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    source = tmp_path / "check.c"
    source.write_text('#include "wsp_hip.h"\n#include "wsp_decoder.h"\n'
                      "int main(void) { wsp_whisper* w = 0; wsp_decoder* d = 0; (void) w; (void) d; return 0; }\n")
    subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", "-I", os.path.join(ROOT, "include"),
                    "-fsyntax-only", str(source)], check=True)
