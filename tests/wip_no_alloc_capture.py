"""karpo_attn_fwd_noalloc under HIP graph capture, through the C ABI, in a process of its own."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu


def test_noalloc_first_call_inside_a_graph_capture(gpu):
    """The entry point's first call on the device made inside a capture (a fresh process, tests/noalloc_capture.py):
    the call succeeds, every replay with rewritten bounds equals the workspace entry point's eager call bit for bit
    and writes every row, and eager calls after the first leave the device's free memory unchanged."""
    child = Path(__file__).resolve().parent / "noalloc_capture.py"
    done = subprocess.run([sys.executable, "-u", str(child)], capture_output=True, text=True, timeout=180)
    print(done.stdout[-3000:], done.stderr[-3000:], flush=True)
    assert done.returncode == 0, done.stderr[-3000:]
    result = json.loads(done.stdout.strip().splitlines()[-1])
    assert result["status_in_capture"] == 0, result
    assert len(result["replays"]) == 5
    for r in result["replays"]:
        assert r["equal"] and not r["nan"], r
    assert result["eager_status"] == [0, 0, 0]
    assert len(set(result["free_bytes"])) == 1, result["free_bytes"]
