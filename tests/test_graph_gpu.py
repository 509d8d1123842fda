"""Stream-ordered HIP graph capture of the library's launches.

No launcher allocates, synchronizes or issues a memset, so a whole forward
pass (and any launch sequence) can be captured into a HIP graph and replayed.
Each graph is replayed several times with eager work and synchronizations
between the replays, and every replay is checked bitwise against the eager
result of the same launches.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from conftest import to_device, to_host
from numerics import require_exact
from vit_support import random_image, random_weights, small_config, tiny_config, write_weights

pytestmark = pytest.mark.gpu


def capture(body):
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            body()
    torch.cuda.synchronize()
    return graph


@pytest.mark.parametrize("precision,tiny", [(0, False), (1, False), (0, True), (1, True)])
def test_model_forward_replays_match_eager(cuvit, oracle, device, tmp_path, precision, tiny):
    config = tiny_config(cuvit) if tiny else small_config(cuvit)
    batch = 2 if tiny else 3
    tensors = random_weights(cuvit, oracle, config, 4040, small=not tiny)
    path = os.path.join(tmp_path, "graph.cvw")
    write_weights(cuvit, tensors, path)
    model = cuvit.VisionTransformer(config, cuvit.WeightFile(path), batch, precision)
    images = to_device(np.concatenate([random_image(oracle, config, 80 + i) for i in range(batch)]),
                       device)
    eager = torch.empty(batch * config.classes, device=device)
    model.forward(images, eager, batch)
    expected = to_host(eager)

    logits = torch.full_like(eager, float("nan"))
    graph = capture(lambda: model.forward(images, logits, batch))
    noise = torch.randn(1 << 20, device=device)
    for replay in range(3):
        logits.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        require_exact(to_host(logits), expected, f"replay {replay} differs from the eager forward")
        # eager work between replays, through the same model and buffers
        other = torch.empty_like(eager)
        model.forward(images, other, batch)
        noise.mul_(1.5)
        torch.cuda.synchronize()


def test_launch_sequence_replays_match_eager(cuvit, oracle, device):
    """LayerNorm, in-place softmax, the gather, broadcast and positional add,
    the GEMM with GELU and with accumulate, and fused attention in one graph."""
    g = oracle.generator(4141)
    rows, embed, tokens, batch, heads = 394, 192, 197, 2, 3
    x = to_device(g.normal(rows * embed), device)
    gamma = to_device(g.normal(embed, 1.0, 0.02), device)
    beta = to_device(g.normal(embed, 0.0, 0.02), device)
    logits_in = to_device(g.normal(batch * heads * tokens * tokens), device)
    images = to_device(g.uniform(batch * 3 * 224 * 224), device)
    pos = to_device(g.normal(tokens * embed, 0.0, 0.02), device)
    cls = to_device(g.normal(embed, 0.0, 0.02), device)
    w = to_device(g.normal(768 * embed, 0.0, 0.05), device)
    bias = to_device(g.normal(768, 0.0, 0.02), device)
    qkv = to_device(g.normal(batch * tokens * 3 * embed), device)

    def run(out):
        cuvit.layer_norm(x, gamma, beta, out["ln"], rows, embed, 1e-6)
        out["sm"].copy_(logits_in)
        cuvit.softmax(out["sm"], out["sm"], batch * heads * tokens, tokens)
        cuvit.extract_patches(images, out["px"], batch, 3, 224, 224, 16)
        out["tok"].zero_()
        cuvit.broadcast(out["tok"], cls, embed, tokens * embed, batch)
        cuvit.add_broadcast(out["tok"], pos, tokens * embed, batch)
        p = cuvit.gemm_problem(rows, 768, embed, cuvit.TRANSPOSED)
        p.epilogue.gelu = 1
        cuvit.gemm(out["ln"], w, bias, out["fc1"], p)
        q = cuvit.gemm_problem(rows, embed, 768, cuvit.NO_TRANSPOSE)
        q.epilogue.accumulate = 1
        out["acc"].copy_(x)
        cuvit.gemm(out["fc1"], w, None, out["acc"], q)
        cuvit.attention(qkv, out["ctx"], batch, heads, tokens, 64)

    def buffers():
        return {"ln": torch.empty(rows * embed, device=device),
                "sm": torch.empty(batch * heads * tokens * tokens, device=device),
                "px": torch.empty(batch * 196 * 768, device=device),
                "tok": torch.empty(batch * tokens * embed, device=device),
                "fc1": torch.empty(rows * 768, device=device),
                "acc": torch.empty(rows * embed, device=device),
                "ctx": torch.empty(batch * tokens * embed, device=device)}

    eager = buffers()
    run(eager)
    expected = {k: to_host(v) for k, v in eager.items()}
    replayed = buffers()
    graph = capture(lambda: run(replayed))
    for replay in range(3):
        for v in replayed.values():
            v.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for k, v in replayed.items():
            require_exact(to_host(v), expected[k], f"replay {replay}: {k} differs from eager")
        run(buffers())  # eager launches between replays
        torch.cuda.synchronize()
