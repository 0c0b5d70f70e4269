"""The Node.js host on the GPU: node/test_runner_gpu.js drives node/runner.js's
DecoderHIPRunner through the N-API addon over libtlm.so, on the synthetic tiny
decoder and the 24-layer Qwen2.5-0.5B-shaped decoder, against the oracle's
expectations in tests/golden/node_runner.json: logits after the prompt within
max-abs 2e-2 / rel 1e-2, the greedy stream of generate() equal to the oracle's
(up to a near-tie), the device-fed loop equal to the host loop with one graph
launch per decode token, and the device's top-8 candidates equal to the 8 best
logits, which generate() then samples from.  The reads are Promises settled
from the addon's thread pool.  Skipped where Node.js or the built addon is
absent (test_node_addon.py builds it)."""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parents[1]


def test_node_runner_against_the_oracle():
    node = shutil.which("node")
    addon = ROOT / "node" / "build" / "Release" / "tlm_addon.node"
    if not node or not addon.exists():
        pytest.skip("Node.js or the built addon is absent")
    env = dict(os.environ, TLM_LIB=str(ROOT / "three-llm_amd" / "libtlm.so"))
    r = subprocess.run([node, str(ROOT / "node" / "test_runner_gpu.js"), str(addon)], env=env, capture_output=True,
                       text=True, timeout=240)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert "1..8" in r.stdout
