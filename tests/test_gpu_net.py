"""WSP::HipNet's misuse refusals on a prepared net (device 0), in the manner of
the reference's KernelNet (Net/KernelNet.cpp:228-244, 274-288, 313-335): an op
recorded outside begin()/end(), a pass on another stream, a value outliving its
recording, every scratch buffer of a capacity held, more live values than
records, a tensor of another net, a value with no buffer of its capacity left
unplaced, and a cache appended past its capacity each end in std::logic_error
with the reference's message; the same recording used properly passes. The
cases are C++ (tests/native/net_refusals.cpp), run in a process of their own."""

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
    assert result.stdout.count("ok ") == 9, result.stdout
