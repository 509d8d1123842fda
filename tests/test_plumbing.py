"""Runs the C++ plumbing tests (tests/cpp/plumbing_test.cpp).

The `host` group needs no GPU: TensorView, launcher argument validation and
exception mapping, HipError, weight files, VitConfig, arena sizing, PPM
loading and preprocessing's argument checks. The `device` group needs one:
DeviceBuffer, HostBuffer (pinned), Stream, DeviceArena, VisionTransformer (fp32
and bf16, from float32 and bf16 weight files) and preprocessing through the
C++ API. They follow the reference's tests/tensor_test.cu,
device_buffer_test.cu, host_buffer_test.cu, stream_test.cu,
device_arena_test.cu, weights_test.cu, vit_test.cu and image_test.cu.
"""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

from conftest import ROOT

BINARY = Path(ROOT) / "tests" / "cpp" / "bin" / "plumbing_test"


def plumbing_binary() -> Path:
    if not BINARY.exists():
        # Built by __graft_entry__.build(); only a missing binary is built here.
        subprocess.run(["make", "-s", "-C", str(BINARY.parents[1])], check=True)
    return BINARY


def run_group(group: str, cwd: Path) -> None:
    result = subprocess.run([str(plumbing_binary()), group], cwd=cwd, capture_output=True,
                            text=True, timeout=120)
    print(result.stdout, result.stderr)
    failed = [line for line in result.stdout.splitlines() if ": FAIL" in line]
    assert result.returncode == 0 and not failed, "\n".join(failed) or result.stderr


def test_plumbing_host(tmp_path):
    run_group("host", tmp_path)


@pytest.mark.gpu
def test_plumbing_device(tmp_path):
    run_group("device", tmp_path)
