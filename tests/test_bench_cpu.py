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
    assert "checked after timing" in bench.check_after_timing(fake_torch, pools(), expected, 1)

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
            bench.check_after_timing(fake_torch, planted(field, index, value), expected, 1)


class _CpuTorch:
    """torch on the CPU with a no-op device synchronize, for bench.py's
    harness functions."""

    def __init__(self):
        import types

        import torch

        self._torch = torch
        self.cuda = types.SimpleNamespace(synchronize=lambda: None)

    def __getattr__(self, name):
        return getattr(self._torch, name)


class _CpuKernels:
    """Stand-ins for the five launches on CPU tensors: each writes only the
    buffer it is handed (the oracle's output, or torch's softmax in place), so
    a set that no launch reached keeps its reset contents. @p skip names a
    (kernel, buffer) pair the stand-in leaves untouched."""

    def __init__(self, expected, skip=None):
        import torch

        self.ln_y = torch.from_numpy(expected["ln_y"].reshape(-1).copy())
        self.patches = torch.from_numpy(expected["patches"].reshape(-1).copy())
        self.skip = skip
        self.calls = {}

    def _skipped(self, name, buffer):
        self.calls[name] = self.calls.get(name, 0) + 1
        return self.skip is not None and self.skip[0] == name and \
            self.skip[1].data_ptr() == buffer.data_ptr()

    def layer_norm(self, x, gamma, beta, y, rows, cols, eps):
        if not self._skipped("layer_norm", y):
            y.copy_(self.ln_y)

    def softmax(self, x, y, rows, cols):
        import torch

        if not self._skipped("softmax", y):
            y.copy_(torch.softmax(x.view(rows, cols), dim=1).view(-1))

    def extract_patches(self, images, patches, batch, channels, height, width, patch):
        if not self._skipped("extract_patches", patches):
            patches.copy_(self.patches)

    def broadcast(self, tokens, cls, count, stride, batch):
        if not self._skipped("broadcast", tokens):
            tokens.view(batch, stride)[:, :count].copy_(cls)

    def add_broadcast(self, tokens, pos, count, batch):
        if not self._skipped("add_broadcast", tokens):
            tokens.view(batch, count).add_(pos)


def _graph_like_timer(body):
    """The timed graph's launches: one untimed replay, then the timed one."""
    body()
    body()
    return 1.0


def test_checked_steps_at_the_real_pool_sizes():
    """bench.py's sequence around the timed region (first-step check, warm-up,
    reset of the written sets, timed steps, after-timing check) with the real
    pools on the CPU: 18 gather, 70 LayerNorm, 69 token and 23 softmax sets.
    It passes at the driver's --steps 20 --warmup 5 and at the default
    --steps 200 --warmup 20, and fails when one written set is skipped by a
    launch or holds a wrong value afterwards."""
    import pytest

    bench = _bench_module()
    torch = _CpuTorch()
    oracle, inputs = bench.seeded_inputs()
    expected = bench.expected_step(oracle, inputs)
    pools = bench.Pools(torch, "cpu", inputs)
    assert (pools.px_sets, pools.ln_sets, pools.tok_sets, pools.sm_sets) == (18, 70, 69, 23)

    for steps, warmup in ((20, 5), (200, 20)):
        kernels = _CpuKernels(expected)
        ms, checks = bench.checked_steps(torch, pools, pools.launchers(kernels), expected,
                                         steps, warmup, _graph_like_timer)
        assert ms == 1.0
        assert kernels.calls["layer_norm"] == 1 + warmup + 2 * steps
        assert checks["gather"] == "bit-exact"
        written = min(steps, 18), min(steps, 70), min(steps, 69), min(steps, 23)
        assert checks["after_timing"].startswith(
            f"{written[0]} gather, {written[1]} LayerNorm, {written[2]} token, {written[3]} softmax")

    # A launch that misses one set inside the written range leaves its reset
    # contents there (NaN, zeros, or the raw logits): refused.
    for name, buffers in (("layer_norm", pools.ln_y), ("extract_patches", pools.patches),
                          ("broadcast", pools.tokens), ("softmax", pools.logits)):
        with pytest.raises(bench.CheckFailed):
            bench.checked_steps(torch, pools, pools.launchers(_CpuKernels(expected, (name, buffers[7]))),
                                expected, 20, 5, _graph_like_timer)

    # A wrong value in a written set after timing: refused.
    kernels = _CpuKernels(expected)
    bench.checked_steps(torch, pools, pools.launchers(kernels), expected, 20, 5, _graph_like_timer)
    pools.ln_y[19][5] += 1.0e-4
    with pytest.raises(bench.CheckFailed):
        bench.check_after_timing(torch, pools, expected, 20)
    pools.ln_y[19][5] -= 1.0e-4
    pools.patches[17][100] = 0.25
    with pytest.raises(bench.CheckFailed):
        bench.check_after_timing(torch, pools, expected, 20)


def test_steps_below_one_are_refused():
    result = subprocess.run([sys.executable, BENCH, "--steps", "0"], capture_output=True,
                            text=True, timeout=120)
    assert result.returncode == 2 and "--steps must be at least 1" in result.stderr
