"""The cu-vit program end to end on the GPU (the reference's src/main.cpp):
a ViT-Tiny/16 weight file with seeded N(0, 0.02) weights, a PPM, and the
reported top classes checked against the oracle's preprocess + forward pass at
the model tolerance of tests/vit_test.cu:128-130 (rtol = atol = 1e-4), plus
the --raw, --benchmark, --batch and --precision paths and the run-time errors.
"""

from __future__ import annotations

import os
import re
import subprocess

import numpy as np
import pytest

from image_support import random_pixels, write_ppm
from vit_support import random_weights, tiny_config, write_weights

pytestmark = pytest.mark.gpu

ROW = re.compile(r"^  +(\d+)  +(-?\d+\.\d{4})  +(\d+\.\d{2})%$")


@pytest.fixture(scope="module")
def setup(cuvit, oracle, tmp_path_factory):
    folder = tmp_path_factory.mktemp("cli")
    config = tiny_config(cuvit)
    tensors = random_weights(cuvit, oracle, config, 2024, small=False)
    weights = str(folder / "vit_tiny.cvw")
    write_weights(cuvit, tensors, weights)
    pixels = random_pixels(77, 240, 320)
    image = str(folder / "image.ppm")
    write_ppm(image, 320, 240, pixels, comment=" cu-vit test image")
    tensor = oracle.preprocess(pixels, config.image_size)
    raw = str(folder / "image.bin")
    tensor.astype(np.float32).tofile(raw)
    arrays = [t for _, t in tensors]
    return {
        "folder": folder, "config": config, "weights": weights, "image": image, "raw": raw,
        "logits": oracle.vit_forward(config, arrays, tensor.reshape(-1)),
        "logits_bf16": oracle.vit_forward(config, arrays, tensor.reshape(-1), bf16=True),
    }


def run(cuvit, *arguments):
    print("cu-vit", *arguments, flush=True)
    return subprocess.run([cuvit.cli_path(), *arguments], capture_output=True, text=True,
                          timeout=120)


def top_rows(stdout: str):
    lines = stdout.splitlines()
    start = lines.index(next(line for line in lines if line.startswith("Top ")))
    rows = []
    for line in lines[start + 1:]:
        match = ROW.match(line)
        if not match:
            break
        rows.append((int(match.group(1)), float(match.group(2)), float(match.group(3))))
    return lines[start], rows


def softmax_percent(logits: np.ndarray) -> np.ndarray:
    shifted = np.exp(logits.astype(np.float64) - logits.max())
    return 100.0 * shifted / shifted.sum()


def test_image_classification_matches_the_oracle(cuvit, setup):
    result = run(cuvit, "--weights", setup["weights"], "--image", setup["image"], "--top", "5")
    assert result.returncode == 0, result.stderr
    lines = result.stdout.splitlines()
    assert lines[0] == "Cu-Vit"
    assert lines[1].startswith("GPU: ") and "gfx950" in lines[1]
    assert re.match(r"^Weights: 152 tensors, \d+\.\d{2} MiB; activations \d+\.\d{2} MiB$", lines[2])
    assert lines[3] == f"Input:   {setup['image']} (320x240)"
    title, rows = top_rows(result.stdout)
    assert title == "Top 5:" and len(rows) == 5

    expected = setup["logits"]
    percent = softmax_percent(expected)
    order = np.argsort(-expected)
    for rank, (label, logit, probability) in enumerate(rows):
        # Printed to 4 decimals: the model tolerance plus half a unit of print.
        assert abs(logit - expected[label]) <= 1e-4 + 1e-4 * abs(expected[label]) + 5e-5, label
        assert abs(probability - percent[label]) <= 0.01, label
        # The label at each rank is the oracle's, up to ties within tolerance.
        assert expected[label] >= expected[order[rank]] - 3e-4
    assert [r[1] for r in rows] == sorted((r[1] for r in rows), reverse=True)


def test_raw_tensor_gives_the_same_report(cuvit, setup):
    """The oracle's preprocessed tensor through --raw: bit-identical input to
    the kernel's, so the same logits and the same report."""
    from_image = run(cuvit, "--weights", setup["weights"], "--image", setup["image"], "--top", "10")
    from_raw = run(cuvit, "--weights", setup["weights"], "--raw", setup["raw"], "--top", "10")
    assert from_image.returncode == 0 and from_raw.returncode == 0, from_raw.stderr
    assert f"Input:   {setup['raw']} (preprocessed tensor)" in from_raw.stdout
    assert top_rows(from_image.stdout) == top_rows(from_raw.stdout)
    assert top_rows(from_raw.stdout)[0] == "Top 10:"


def test_benchmark_line(cuvit, setup):
    result = run(cuvit, "--weights", setup["weights"], "--image", setup["image"],
                 "--benchmark", "20", "--batch", "8", "--top", "1")
    assert result.returncode == 0, result.stderr
    match = re.search(r"^Batch 8: (\d+\.\d{3}) ms per pass, (\d+\.\d{3}) ms per image "
                      r"\((\d+\.\d) images/s over 20 iterations\)$", result.stdout, re.M)
    assert match, result.stdout
    ms, per_image, rate = (float(g) for g in match.groups())
    assert ms > 0 and abs(per_image - ms / 8) < 2e-3 and abs(rate - 8000.0 / ms) / rate < 0.01
    # The report before the benchmark is of batch slot 0 alone.
    label, logit, _ = top_rows(result.stdout)[1][0]
    assert label == int(np.argmax(setup["logits"]))


def test_bf16_precision(cuvit, setup):
    result = run(cuvit, "--weights", setup["weights"], "--image", setup["image"],
                 "--precision", "bf16", "--top", "5")
    assert result.returncode == 0, result.stderr
    expected = setup["logits_bf16"]
    top = set(np.argsort(-expected)[:8].tolist())
    for label, logit, _ in top_rows(result.stdout)[1]:
        assert label in top
        assert abs(logit - expected[label]) < 0.05


@pytest.mark.parametrize("case", ["missing_weights", "short_raw", "not_ppm", "zero_batch"])
def test_run_time_errors(cuvit, setup, case):
    folder = setup["folder"]
    if case == "missing_weights":
        arguments = ("--weights", str(folder / "absent.cvw"), "--image", setup["image"])
        message = None
    elif case == "short_raw":
        short = str(folder / "short.bin")
        np.zeros(100, np.float32).tofile(short)
        arguments = ("--weights", setup["weights"], "--raw", short)
        message = f"Tensor is shorter than the model's input: {short}"
    elif case == "not_ppm":
        text = str(folder / "text.ppm")
        with open(text, "w") as handle:
            handle.write("P3\n1 1\n255\n0 0 0\n")
        arguments = ("--weights", setup["weights"], "--image", text)
        message = f"Only binary PPM (P6) images are supported: {text}"
    else:
        arguments = ("--weights", setup["weights"], "--image", setup["image"], "--batch", "0")
        message = "--batch must be at least one"
    result = run(cuvit, *arguments)
    assert result.returncode == 1
    assert result.stderr.startswith("cu-vit failed: ")
    if message is not None:
        assert result.stderr == f"cu-vit failed: {message}\n"
    assert os.path.exists(cuvit.cli_path())
