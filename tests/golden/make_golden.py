"""Writes the committed fixtures in this folder. Run from the repository root
after building oracle/ (including oracle/_ref, which needs the reference tree):

    python tests/golden/make_golden.py

generator_streams.json
    The first 64 float32 values (as bit patterns) of every seeded stream the
    measured configurations and the ported reference tests draw, from the
    DataGenerator restatement (std::mt19937_64 + libstdc++ distributions,
    tests/test_utils.hpp:233-263). The reference's own generator cannot be
    compiled here (test_utils.hpp includes the CUDA runtime), so these pin the
    restatement across hosts and toolchains rather than against the reference.

reference_vectors.npz
    Inputs and outputs of the reference's own CPU code (oracle/_ref: its
    tests/reference/linear_algebra.hpp compiled in place): LayerNorm and softmax
    rows at widths 192, 197 and 768, the GELU landmarks of
    tests/elementwise_test.cu:38-39, and one small GEMM.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

from oracle import Oracle, Reference  # noqa: E402

STREAMS = [
    # (label, seed, kind, a, b): normal(mean a, std b) or uniform(low a, high b)
    ("C1 layer norm input x[197,192]", 101, "normal", 0.0, 1.0),
    ("C2 softmax logits", 202, "normal", 0.0, 1.0),
    ("C3 images U(-1,1)", 303, "uniform", -1.0, 1.0),
    ("C4 weights N(0,0.02)", 404, "normal", 0.0, 0.02),
    ("C4 images U(-1,1)", 404, "uniform", -1.0, 1.0),
    ("C5 inputs N(0,1)", 505, "normal", 0.0, 1.0),
    ("elementwise_test GELU", 31, "normal", 0.0, 3.0),
    ("elementwise_test add", 9, "normal", 0.0, 1.0),
    ("elementwise_test LN 197x192", 197 * 101 + 192, "normal", 0.0, 1.0),
    ("elementwise_test LN offset", 7, "normal", 1000.0, 1.0),
    ("elementwise_test softmax 197x197", 197 * 17 + 197, "normal", 0.0, 4.0),
    ("vit_test image seed 1", 1, "normal", 0.0, 1.0),
    ("numerics_test uniform", 99, "uniform", -2.0, 3.0),
]


def main() -> None:
    oracle = Oracle()
    streams = []
    for label, seed, kind, a, b in STREAMS:
        g = oracle.generator(seed)
        values = g.normal(64, a, b) if kind == "normal" else g.uniform(64, a, b)
        streams.append({"label": label, "seed": seed, "kind": kind, "a": a, "b": b,
                        "bits": values.view(np.uint32).tolist()})
    with open(os.path.join(HERE, "generator_streams.json"), "w") as out:
        json.dump(streams, out, indent=1)

    reference = Reference()
    vectors = {}
    for width in (192, 197, 768):
        g = oracle.generator(7000 + width)
        x = g.normal(4 * width).reshape(4, width)
        gamma = g.normal(width, 1.0, 0.2)
        beta = g.normal(width, 0.0, 0.2)
        vectors[f"ln_x_{width}"] = x
        vectors[f"ln_gamma_{width}"] = gamma
        vectors[f"ln_beta_{width}"] = beta
        vectors[f"ln_y_{width}"] = reference.layer_norm(x, gamma, beta, 1e-6)
        logits = g.normal(3 * width, 0.0, 4.0).reshape(3, width)
        vectors[f"sm_x_{width}"] = logits
        vectors[f"sm_y_{width}"] = reference.softmax(logits)
    landmarks = np.array([-30, -8, -2.7, -2, -1, -0.5, 0, 0.5, 1, 2, 2.7, 8, 30], np.float32)
    vectors["gelu_x"] = landmarks
    vectors["gelu_y"] = reference.gelu(landmarks)
    g = oracle.generator(7777)
    a, b, bias = g.normal(9 * 21), g.normal(13 * 21), g.normal(13)
    vectors["gemm_a"], vectors["gemm_b"], vectors["gemm_bias"] = a, b, bias
    vectors["gemm_c"] = reference.gemm_transposed(a, b, bias, 9, 13, 21)
    np.savez(os.path.join(HERE, "reference_vectors.npz"), **vectors)


if __name__ == "__main__":
    main()
