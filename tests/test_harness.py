"""The C++ harness (tests/harness/harness_hip.cpp): a plain host program that
calls libtcrv_hip and libtcrv_hip_route through their C headers and the
exported fixture functions (generated from tests/harness/emitc_fixtures.manifest
by tianchen-rv_amd/tcrv_hip_export) by their names -- the reference's add proof
(examples/qemu/harness_add.cpp:13-33) through the exported add, every other
exported fixture function, the route selection matrix, and routed
contractions, each checked bit for bit against the oracle.  Started as a child
process."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
HARNESS = os.path.join(HERE, "harness", "harness_hip")


def test_harness_is_built():
    assert os.path.exists(HARNESS), "run __graft_entry__.build()"


@pytest.mark.gpu
def test_harness_runs_on_the_gpu():
    r = subprocess.run([HARNESS], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.splitlines()
    assert "add proof ok: 1031 elements checked (exported add)" in lines
    exported = [ln for ln in lines if ln.startswith("exported ")]
    assert len(exported) == 12 and all("bit-identical to the oracle" in ln for ln in exported)
    assert sum(1 for ln in lines if ln.startswith("route ")) == 12
    assert sum(1 for ln in lines if "bit-identical to the oracle" in ln) == 17
    assert lines[-1] == "harness ok"
