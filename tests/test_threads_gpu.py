"""Launches from several host threads at once. The reference's launchers are
stateless and re-entrant, enqueue-only on the stream they are given
(include/cuvit/kernels.hpp:9-154): any host thread may call them with its
own stream. Here four threads, each with its own stream and buffers, run
LayerNorm, softmax and the patch gather 20 times concurrently; every result
must equal, bit for bit, the same launches made from one thread.
"""

from __future__ import annotations

import threading

import numpy as np
import pytest
import torch

from conftest import to_device, to_host

pytestmark = pytest.mark.gpu

THREADS = 4
ROWS, COLUMNS = 591, 197        # softmax: one ViT-Tiny head batch of 3 images
LN_ROWS, LN_COLUMNS = 394, 192  # LayerNorm: two ViT-Tiny images
IMAGES = 2                      # gather: [2, 3, 224, 224]


def make_inputs(oracle, seed, device):
    generator = oracle.generator(seed)
    return {
        "logits": to_device(generator.normal(ROWS * COLUMNS), device),
        "x": to_device(generator.normal(LN_ROWS * LN_COLUMNS), device),
        "gamma": to_device(generator.normal(LN_COLUMNS, 1.0, 0.02), device),
        "beta": to_device(generator.normal(LN_COLUMNS, 0.0, 0.02), device),
        "images": to_device(generator.normal(IMAGES * 3 * 224 * 224), device),
    }


def launch(cuvit, inputs, outputs, stream):
    cuvit.softmax(inputs["logits"], outputs["probabilities"], ROWS, COLUMNS, stream=stream)
    cuvit.layer_norm(inputs["x"], inputs["gamma"], inputs["beta"], outputs["normalized"],
                     LN_ROWS, LN_COLUMNS, stream=stream)
    cuvit.extract_patches(inputs["images"], outputs["patches"], IMAGES, 3, 224, 224, 16,
                          stream=stream)


def empty_outputs(device):
    return {
        "probabilities": torch.full((ROWS * COLUMNS,), float("nan"), device=device),
        "normalized": torch.full((LN_ROWS * LN_COLUMNS,), float("nan"), device=device),
        "patches": torch.full((IMAGES * 3 * 224 * 224,), float("nan"), device=device),
    }


def test_concurrent_launches_from_host_threads(cuvit, oracle, device):
    inputs = [make_inputs(oracle, 8100 + i, device) for i in range(THREADS)]
    print(f"{THREADS} threads: softmax [{ROWS},{COLUMNS}], layer norm [{LN_ROWS},{LN_COLUMNS}], "
          f"gather of {IMAGES} images", flush=True)

    # The same launches from this thread, one after another, on the default stream.
    expected = []
    for i in range(THREADS):
        outputs = empty_outputs(device)
        launch(cuvit, inputs[i], outputs, None)
        expected.append(outputs)
    torch.cuda.synchronize()

    streams = [torch.cuda.Stream() for _ in range(THREADS)]
    actual = [empty_outputs(device) for _ in range(THREADS)]
    torch.cuda.synchronize()
    barrier = threading.Barrier(THREADS)
    failures = []

    def run(i):
        try:
            barrier.wait()
            for _ in range(20):
                launch(cuvit, inputs[i], actual[i], streams[i])
            streams[i].synchronize()
        except Exception as error:  # reported below, on the main thread
            failures.append(f"thread {i}: {error!r}")

    threads = [threading.Thread(target=run, args=(i,)) for i in range(THREADS)]
    for thread in threads:
        thread.start()
    for thread in threads:
        thread.join()
    torch.cuda.synchronize()
    assert not failures, failures
    for i in range(THREADS):
        for name in ("probabilities", "normalized", "patches"):
            got = to_host(actual[i][name]).view(np.uint32)
            want = to_host(expected[i][name]).view(np.uint32)
            assert np.array_equal(got, want), f"thread {i}: {name} differs from the one-thread launch"
