"""GPU-vs-CPU twin tests of the C++ host layer (the reference's
tests/cuda_*_test.rs restated in tests/cpp/twin_tests.cpp). The binary runs
once per session; each case is reported as its own pytest item."""
import os
import re
import subprocess

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "twin_tests")
SRC = os.path.join(HERE, "cpp", "twin_tests.cpp")


def case_names():
    text = open(SRC).read()
    block = text[text.index("const Case kCases[]"):]
    return re.findall(r'\{"(\w+)",', block)


@pytest.fixture(scope="module")
def twin_results():
    if not os.path.exists(BIN):
        pytest.fail(f"twin-test binary missing: {BIN} (run __graft_entry__.build())")
    print(f"running {BIN}", flush=True)
    proc = subprocess.run([BIN], capture_output=True, text=True, timeout=600)
    results = {}
    for line in proc.stdout.splitlines():
        m = re.match(r"(PASS|FAIL) (\w+)(?::\s*(.*))?$", line)
        if m:
            results[m.group(2)] = (m.group(1), m.group(3) or "")
    if not results:
        pytest.fail(f"twin_tests produced no results (status {proc.returncode}):\n"
                    f"{proc.stdout[-2000:]}\n{proc.stderr[-2000:]}")
    return results, proc


@pytest.mark.parametrize("name", case_names())
def test_twin(twin_results, name):
    results, proc = twin_results
    assert name in results, f"{name} did not report (crash?):\n{proc.stdout[-1500:]}\n{proc.stderr[-1500:]}"
    status, msg = results[name]
    assert status == "PASS", msg
