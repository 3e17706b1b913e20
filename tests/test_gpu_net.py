"""WSP::HipNet's misuse refusals on a prepared net (device 0). HipNet records a
program and places its values when the recording ends: an op with no recording
open, a pass on another stream, a second begin(), a handle kept past its
recording, more values live at one instruction than scratch buffers, a full
value table, a tensor of another net, a value with nowhere to live, a cache
appended past its capacity and output() of a view each end in
std::logic_error; a proper recording passes, and a chain of five LayerNorms
whose handles all stay held runs in two buffers and matches the host. The cases
are C++ (tests/native/net_refusals.cpp), run in a process of their own."""

import os
import subprocess

import pytest

from helpers import ROOT, ensure_library

pytestmark = pytest.mark.gpu


def test_net_refusals_on_a_prepared_net():
    ensure_library()
    path = os.path.join(ROOT, "tests", "native", "_build", "net_refusals")
    if not os.path.exists(path):
        subprocess.run(["make", "-s", "_build/net_refusals"], cwd=os.path.join(ROOT, "tests", "native"), check=True)
    result = subprocess.run([path, "device"], capture_output=True, text=True, timeout=120)
    print(result.stdout)
    assert result.returncode == 0, result.stdout + result.stderr
    assert result.stdout.count("ok ") == 12, result.stdout
