"""gpu_cli input handling that happens before any device is touched (no GPU needed)."""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "beam_search_collab_amd", "bin", "gpu_cli")


def run_cli(text):
    p = subprocess.run([CLI], input=text, capture_output=True, text=True, timeout=60)
    return p.returncode, p.stdout, p.stderr


@pytest.mark.skipif(not os.path.exists(CLI), reason="gpu_cli not built")
def test_cli_rejects_bad_input():
    rc, _, err = run_cli("{not json")
    assert rc == 1 and "JSON parse error" in err
    rc, _, err = run_cli(json.dumps({"search": {"mode": "base"}}))
    assert rc == 1 and 'Missing "data" key' in err
    rc, _, err = run_cli(json.dumps({"data": {}, "search": {"mode": "sophia_beam"}}))
    assert rc == 1 and "sophia" in err
    rc, _, err = run_cli(json.dumps({"data": {"graph": "/nonexistent/graph.bin", "base": "b", "query": "q",
                                              "gt": "g"}, "search": {"mode": "base"}}))
    assert rc == 1 and err.strip()
