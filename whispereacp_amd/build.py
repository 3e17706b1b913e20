"""Compiles the gfx950 library (HIP kernels, C ABI and the C++ decoder layer)
into whispereacp_amd/_build/libwhispereacp_hip.so with hipcc.

Every HIP translation unit is built with packed FP32 arithmetic switched off
(``-target-feature -packed-fp32-ops``) and for gfx950 only.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from typing import List

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBRARY = os.path.join(BUILD, "libwhispereacp_hip.so")
ARCH = "gfx950"

DEVICE_SOURCES = ["ops.hip", "capi.hip", "cross_kv.hip", "fused_step.hip", "step_kernel.hip", "batch.hip",
                  "mfma_product.hip", "split_product.hip", "attention_static.hip", "encoder.hip", "mel.hip"]
HOST_SOURCES = ["host/Gpu.cpp", "host/Net.cpp", "host/Half.cpp", "host/HipNet.cpp", "host/DecoderWeights.cpp",
                "host/Decoder.cpp", "host/DecoderRecording.cpp", "host/Argmax.cpp", "host/GreedyDecoder.cpp", "host/BatchedDecoder.cpp",
                "host/SafeTensors.cpp", "host/Tokenizer.cpp", "host/Encoder.cpp", "host/Whisper.cpp",
                "host/decoder_capi.cpp"]

COMMON = ["-std=c++20", "-fPIC", "-Wall", "-Wno-unused-result", "-I" + os.path.join(HERE, "..", "include")]
DEVICE_FLAGS = ["-O3", "--offload-arch=" + ARCH, "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HOST_FLAGS = ["-O2", "-D__HIP_PLATFORM_AMD__", "-I" + os.path.join(ROCM, "include")]
# Per-source device flags: the pre-split products keep their matrix-core
# accumulators in VGPRs (in AGPRs the compiler shuffles them between steps).
SOURCE_FLAGS = {"split_product.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the gfx950 library cannot be built")
    return path


def _object_path(source: str) -> str:
    return os.path.join(BUILD, "obj", source.replace("/", "_") + ".o")


def _compile(source: str, device: bool) -> str:
    out = _object_path(source)
    flags = DEVICE_FLAGS + SOURCE_FLAGS.get(source, []) if device else HOST_FLAGS
    cmd = [hipcc()] + COMMON + flags + ["-c", os.path.join(CSRC, source), "-o", out]
    if not device:
        cmd[1:1] = ["-x", "c++"]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"compiling {source} failed:\n{result.stderr[-6000:]}")
    return out


def build(verbose: bool = True) -> str:
    """Compile every source and link the shared library; returns its path."""
    os.makedirs(os.path.join(BUILD, "obj"), exist_ok=True)
    jobs = [(s, True) for s in DEVICE_SOURCES] + [(s, False) for s in HOST_SOURCES]
    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    objects: List[str] = []
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        futures = {pool.submit(_compile, s, d): s for s, d in jobs}
        for f in concurrent.futures.as_completed(futures):
            objects.append(f.result())
            if verbose:
                print(f"  compiled {futures[f]}", flush=True)
    tmp = LIBRARY + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", tmp] + sorted(objects)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking failed:\n{result.stderr[-6000:]}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"  linked {LIBRARY}", flush=True)
    return LIBRARY


# The timeline variant: the persistent step built with WSP_STEP_TIMELINE, which
# stamps the real-time clock at every phase boundary of every workgroup. Only
# the two translation units that see the macro are recompiled; the rest are the
# main build's objects.
TIMELINE_SOURCES = ["step_kernel.hip", "fused_step.hip"]
TIMELINE_BUILD = os.path.join(BUILD, "timeline")
TIMELINE_LIBRARY = os.path.join(TIMELINE_BUILD, "libwhispereacp_hip.so")


def build_timeline(verbose: bool = True) -> str:
    """The timeline variant of the library (after build()); returns its path."""
    if not all(os.path.exists(_object_path(s)) for s in DEVICE_SOURCES + HOST_SOURCES):
        build(verbose)
    os.makedirs(TIMELINE_BUILD, exist_ok=True)
    objects = []
    for source in DEVICE_SOURCES + HOST_SOURCES:
        if source not in TIMELINE_SOURCES:
            objects.append(_object_path(source))
            continue
        out = os.path.join(TIMELINE_BUILD, source.replace("/", "_") + ".o")
        cmd = [hipcc()] + COMMON + DEVICE_FLAGS + ["-DWSP_STEP_TIMELINE", "-c", os.path.join(CSRC, source), "-o", out]
        result = subprocess.run(cmd, capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError(f"compiling {source} (timeline) failed:\n{result.stderr[-6000:]}")
        objects.append(out)
        if verbose:
            print(f"  compiled {source} (timeline)", flush=True)
    tmp = TIMELINE_LIBRARY + ".tmp"
    result = subprocess.run([hipcc(), "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", tmp] + sorted(objects),
                            capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking the timeline variant failed:\n{result.stderr[-6000:]}")
    os.replace(tmp, TIMELINE_LIBRARY)
    if verbose:
        print(f"  linked {TIMELINE_LIBRARY}", flush=True)
    return TIMELINE_LIBRARY


if __name__ == "__main__":
    try:
        build()
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
