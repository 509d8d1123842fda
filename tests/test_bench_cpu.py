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


def _bench_module():
    import importlib.util

    spec = importlib.util.spec_from_file_location("bench_under_test", BENCH)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def test_output_checks_accept_the_oracle_and_catch_planted_mistakes():
    """The checks bench.py runs around its timed steps, driven with host
    tensors holding the oracle's own outputs (accepted) and then with one
    planted mistake per kernel (each refused)."""
    import types

    import numpy as np
    import pytest
    import torch

    bench = _bench_module()
    oracle, inputs = bench.seeded_inputs()
    expected = bench.expected_step(oracle, inputs)

    def pools():
        t = lambda a: torch.from_numpy(np.array(a, dtype=np.float32).reshape(-1))
        return types.SimpleNamespace(
            patches=[t(expected["patches"])], tokens=[t(expected["tokens"])],
            ln_y=[t(expected["ln_y"])], logits=[t(expected["probabilities"])],
            gamma=t(inputs["gamma"]), px_sets=1, ln_sets=1, tok_sets=1, sm_sets=1)

    report = bench.check_first_step(types.SimpleNamespace(cuda=types.SimpleNamespace(
        synchronize=lambda: None)), pools(), expected)
    assert report["gather"] == "bit-exact" and report["layer_norm_max_abs"] == 0.0
    fake_torch = types.SimpleNamespace(cuda=types.SimpleNamespace(synchronize=lambda: None),
                                       equal=torch.equal, from_numpy=torch.from_numpy,
                                       int32=torch.int32)
    assert "checked after timing" in bench.check_after_timing(fake_torch, pools(), expected)

    def planted(field, index, value):
        p = pools()
        getattr(p, field)[0][index] = float(value)
        return p

    cases = [("patches", 12345, np.nextafter(np.float32(expected["patches"].reshape(-1)[12345]),
                                             np.float32(9))),
             ("tokens", 5, 1.0), ("ln_y", 77, expected["ln_y"].reshape(-1)[77] + 2.0e-5),
             ("logits", 3, expected["probabilities"].reshape(-1)[3] + 2.0e-5)]
    for field, index, value in cases:
        with pytest.raises(bench.CheckFailed):
            bench.check_first_step(fake_torch, planted(field, index, value), expected)
    for field, index, value in (("patches", 9, 0.5), ("tokens", 0, 0.5), ("ln_y", 1, 9.0),
                                ("logits", 0, 1.5)):
        with pytest.raises(bench.CheckFailed):
            bench.check_after_timing(fake_torch, planted(field, index, value), expected)
