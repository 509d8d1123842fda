"""bench.py's command line on the CPU: it measures one GPU, and a request for
more exits with a message, before touching a device."""

from __future__ import annotations

import os
import subprocess
import sys

BENCH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "bench.py")


def test_more_than_one_gpu_is_refused_with_a_message():
    for gpus in ("2", "8"):
        result = subprocess.run([sys.executable, BENCH, "--gpus", gpus, "--steps", "5"],
                                capture_output=True, text=True, timeout=120)
        assert result.returncode == 2, result.stderr
        assert "measures one GPU" in result.stderr
        assert result.stdout == ""
