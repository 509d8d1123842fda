"""Seeded inputs of the benchmark configurations. TEST INFRASTRUCTURE ONLY.

The configurations the layer-kernel path is measured and judged on, drawn with
the reference tests' DataGenerator (tests/test_utils.hpp:233-263, restated in
oracle.cpp) so that the GPU run and the CPU oracle see the same values. One
generator per configuration, drawn in the order listed:

  C1  seed 101  x[rows, 192] ~ N(0, 1), gamma[192] ~ N(1, 0.02),
                beta[192] ~ N(0, 0.02); epsilon 1e-6. rows = 197 (batch 1)
                or 6304 (batch 32).
  C2  seed 202  logits[32 * 3 * 197, 197] = N(0, 1) * (8 / sqrt(64)).
  C3  seed 303  images[32, 3, 224, 224] ~ U(-1, 1), pos[197, 192] ~ N(0, 0.02),
                cls[192] ~ N(0, 0.02); the token buffer starts at zero.
  C5  seed 505  every value drawn in fp32 and rounded to bf16 (nearest even),
                except gamma, beta and the bias, which stay fp32:
                LayerNorm x[12608, 768] ~ N(0, 1), gamma ~ N(1, 0.02),
                beta ~ N(0, 0.02); softmax logits[151296, 197] ~ N(0, 1);
                FC1 A[12608, 768] ~ N(0, 1), W[3072, 768] ~ N(0, 0.02),
                bias[3072] ~ N(0, 0.02); images[64, 3, 224, 224] ~ N(0, 1).

Used by tests/ (parity at these exact inputs) and by bench.py's checking and
CPU-baseline leg (the timed GPU step runs on these values and one step's
outputs are compared with the oracle's before timing).

in_row_chunks runs an oracle function over row ranges on several host threads:
the oracle's entry points are ctypes calls, which release the interpreter lock,
so a full-size comparison (a 12608 x 3072 x 768 GEMM) takes seconds instead of
minutes.
"""

from __future__ import annotations

import math
import os
from concurrent.futures import ThreadPoolExecutor
from typing import Callable, Dict

import numpy as np

EMBED, TOKENS = 192, 197
BATCH = 32
SOFTMAX_ROWS = BATCH * 3 * TOKENS
IMAGE, CHANNELS, PATCH = 224, 3, 16


def layer_norm_c1(oracle, rows: int = TOKENS) -> Dict[str, np.ndarray]:
    g = oracle.generator(101)
    return {"x": g.normal(rows * EMBED).reshape(rows, EMBED),
            "gamma": g.normal(EMBED, 1.0, 0.02), "beta": g.normal(EMBED, 0.0, 0.02),
            "epsilon": 1.0e-6}


def softmax_c2(oracle) -> np.ndarray:
    scale = np.float32(8.0 / math.sqrt(64.0))  # exactly 1
    return (oracle.generator(202).normal(SOFTMAX_ROWS * TOKENS) * scale).reshape(
        SOFTMAX_ROWS, TOKENS)


def tokens_c3(oracle, batch: int = BATCH) -> Dict[str, np.ndarray]:
    g = oracle.generator(303)
    return {"images": g.uniform(batch * CHANNELS * IMAGE * IMAGE, -1.0, 1.0),
            "pos": g.normal(TOKENS * EMBED, 0.0, 0.02), "cls": g.normal(EMBED, 0.0, 0.02)}


def vit_base_c5(oracle) -> Dict[str, np.ndarray]:
    """bf16 values as their bit patterns (uint16, key + "_bits") and as the
    fp32 values they stand for (the oracle's inputs)."""
    from oracle import bf16_to_float

    rows, embed, hidden, heads, batch = 64 * TOKENS, 768, 3072, 12, 64
    g = oracle.generator(505)
    out: Dict[str, np.ndarray] = {}

    def bf16(name, values):
        bits = oracle.round_bf16(values)
        out[name + "_bits"] = bits
        out[name] = bf16_to_float(bits)

    bf16("ln_x", g.normal(rows * embed))
    out["ln_gamma"] = g.normal(embed, 1.0, 0.02)
    out["ln_beta"] = g.normal(embed, 0.0, 0.02)
    bf16("logits", g.normal(batch * heads * TOKENS * TOKENS))
    bf16("fc1_a", g.normal(rows * embed))
    bf16("fc1_w", g.normal(hidden * embed, 0.0, 0.02))
    out["fc1_bias"] = g.normal(hidden, 0.0, 0.02)
    bf16("images", g.normal(batch * CHANNELS * IMAGE * IMAGE))
    return out


def workers() -> int:
    """Host threads for the chunked oracle: the CPUs this process may use, at
    most 16 (one GPU's share of a host)."""
    try:
        available = len(os.sched_getaffinity(0))
    except AttributeError:
        available = os.cpu_count() or 1
    return max(1, min(16, available))


def in_row_chunks(fn: Callable[[int, int], np.ndarray], rows: int, chunk: int) -> np.ndarray:
    """fn(start, stop) for consecutive row ranges of at most @p chunk rows,
    run on worker threads; the results are stacked in row order."""
    ranges = [(s, min(rows, s + chunk)) for s in range(0, rows, chunk)]
    with ThreadPoolExecutor(max_workers=workers()) as pool:
        parts = list(pool.map(lambda r: fn(*r), ranges))
    return np.concatenate(parts, axis=0)
