"""The N-API addon + Node HipContext (the TypeScript host's drop-in) on the
GPU: fluidaudio-web_amd/node/selftest.js checks each op against inline JS
references and the fused encoder's packed-vs-standalone equality."""
import os
import shutil
import subprocess

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE_DIR = os.path.join(ROOT, "fluidaudio-web_amd", "node")


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_node_selftest():
    if not os.path.exists(os.path.join(NODE_DIR, "fa_hip.node")):
        pytest.skip("N-API addon not built (no node headers at build time)")
    r = subprocess.run(["node", os.path.join(NODE_DIR, "selftest.js")], capture_output=True, text=True, timeout=110)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
