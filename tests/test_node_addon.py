"""The Node.js N-API binding (node/tlm_addon.cc): built with node-gyp against
the system Node headers, then node/test_addon.js checks on the CPU that every
entry point is bound, the host-side helpers return what the C ABI computes,
and failing calls throw an Error carrying tlm_last_error() and its TLM_ERR_*
code; node/runner.js (the DecoderHIPRunner of the Node host) builds the same
synthetic tensors as the Python host.  Then node/test_runner_mock.js runs the
addon and runner.js over a stand-in library with the same C ABI
(node/test_mock_tlm.c, a formula decoder built here with gcc): the Promise
reads run off the JS thread and reject with the worker thread's error, and
generate() follows generateAsync (prompt cache, greedy, device top-k and host
sampling, stop tokens, onToken).  Skipped where Node.js or its headers are
absent."""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
NODE_DIR = ROOT / "node"
HEADERS = Path("/usr/include/nodejs")


def _tools():
    node, gyp = shutil.which("node"), shutil.which("node-gyp")
    if not node or not gyp or not (HEADERS / "src" / "node_api.h").exists():
        pytest.skip("Node.js, node-gyp or the Node headers are not installed")
    return node, gyp


def test_addon_builds_and_binds_the_c_abi():
    node, gyp = _tools()
    lib = ROOT / "three-llm_amd" / "libtlm.so"
    if not lib.exists():
        pytest.skip("libtlm.so is not built")
    env = dict(os.environ, TLM_LIB=str(lib))
    b = subprocess.run([gyp, "rebuild", f"--nodedir={HEADERS}"], cwd=NODE_DIR, env=env, capture_output=True,
                       text=True, timeout=300)
    assert b.returncode == 0, b.stdout[-2000:] + b.stderr[-2000:]
    addon = NODE_DIR / "build" / "Release" / "tlm_addon.node"
    assert addon.exists()
    r = subprocess.run([node, str(NODE_DIR / "test_addon.js"), str(addon)], env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "1..11" in r.stdout


def test_runner_over_a_stand_in_library(tmp_path):
    node, _ = _tools()
    addon = NODE_DIR / "build" / "Release" / "tlm_addon.node"
    if not addon.exists():
        pytest.skip("the addon is not built (test_addon_builds_and_binds_the_c_abi builds it)")
    mock = tmp_path / "libtlm_mock.so"
    b = subprocess.run(["gcc", "-shared", "-fPIC", "-O2", "-Wall", "-Werror", "-I", str(ROOT / "include"), "-o",
                        str(mock), str(NODE_DIR / "test_mock_tlm.c"), "-lpthread"], capture_output=True, text=True)
    assert b.returncode == 0, b.stderr[-2000:]
    env = dict(os.environ, TLM_LIB=str(mock))
    r = subprocess.run([node, str(NODE_DIR / "test_runner_mock.js"), str(addon)], env=env, capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "1..8" in r.stdout
