"""The C-ABI boundary on the CPU: the library loads, exports every entry point
include/cuvit/capi.h declares, mirrors the reference's struct layout, and
validates arguments in the reference's order and wording before any HIP call
(src/kernels/normalization.cu:224-350, src/kernels/gemm.cu:199-231). None of
these calls reaches a kernel, so they run without a GPU.
"""

from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cuvit", "capi.h")
FAKE = 0x1000  # a non-null address that is never dereferenced: validation stops first


def declared_functions():
    text = Path(HEADER).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cuvit_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_gemm_problem_layout_matches_the_reference(cuvit):
    """cuvit_gemm_problem mirrors cuvit::GemmProblem field for field."""
    assert ctypes.sizeof(cuvit.GemmProblem) == 104
    assert cuvit.GemmProblem.batch.offset == 32
    assert cuvit.GemmProblem.epilogue.offset == 96
    p = cuvit.gemm_problem(3, 4, 5, cuvit.TRANSPOSED)
    assert (p.m, p.n, p.k, p.layout, p.alpha, p.lda, p.ldb, p.ldc) == (3, 4, 5, 1, 1.0, 0, 0, 0)
    assert (p.batch.count, p.batch.inner, p.epilogue.accumulate, p.epilogue.gelu) == (1, 0, 0, 0)


def test_zero_extents_return_before_any_check(lib):
    """normalization.cu:226-228: empty launches succeed even with null operands."""
    assert lib.cuvit_layer_norm_f32(None, None, None, None, 0, 4, 1e-6, None) == 0
    assert lib.cuvit_layer_norm_f32(None, None, None, None, 4, 0, 1e-6, None) == 0
    assert lib.cuvit_softmax_f32(None, None, 0, 4, None) == 0
    assert lib.cuvit_gelu_f32(None, None, 0, None) == 0
    assert lib.cuvit_add_f32(None, None, 0, None) == 0
    assert lib.cuvit_add_broadcast_f32(None, None, 0, 3, None) == 0
    assert lib.cuvit_add_broadcast_f32(None, None, 3, 0, None) == 0
    assert lib.cuvit_broadcast_f32(None, None, 0, 0, 3, None) == 0
    assert lib.cuvit_extract_patches_f32(None, None, 0, -1, -1, -1, -1, None) == 0
    assert lib.cuvit_layer_norm_bf16(None, None, None, None, 0, 4, 1e-6, None) == 0
    assert lib.cuvit_softmax_bf16(None, None, 4, 0, None) == 0
    assert lib.cuvit_attention_f32(None, None, 0, 3, 197, 64, None) == 0
    assert lib.cuvit_attention_f32(None, None, 2, 3, 0, 64, None) == 0
    assert lib.cuvit_broadcast_bf16(None, None, 0, 0, 3, None) == 0
    assert lib.cuvit_attention_bf16(None, None, 0, 12, 197, 64, None) == 0
    assert lib.cuvit_convert_f32_to_bf16(None, None, 0, None) == 0
    assert lib.cuvit_convert_bf16_to_f32(None, None, 0, None) == 0


@pytest.mark.parametrize("call,message", [
    (lambda l: l.cuvit_layer_norm_f32(FAKE, FAKE, FAKE, FAKE, -1, 4, 1e-6, None),
     "Layer norm dimensions cannot be negative"),
    (lambda l: l.cuvit_layer_norm_f32(FAKE, None, FAKE, FAKE, 2, 4, 1e-6, None),
     "Layer norm operands cannot be null"),
    (lambda l: l.cuvit_softmax_f32(FAKE, FAKE, 3, -2, None), "Softmax dimensions cannot be negative"),
    (lambda l: l.cuvit_softmax_f32(None, FAKE, 3, 2, None), "Softmax operands cannot be null"),
    (lambda l: l.cuvit_gelu_f32(FAKE, FAKE, -5, None), "GELU element count cannot be negative"),
    (lambda l: l.cuvit_gelu_f32(None, FAKE, 4, None), "GELU operands cannot be null"),
    (lambda l: l.cuvit_add_f32(FAKE, FAKE, -1, None), "Residual add element count cannot be negative"),
    (lambda l: l.cuvit_add_f32(FAKE, None, 8, None), "Residual add operands cannot be null"),
    (lambda l: l.cuvit_add_broadcast_f32(FAKE, FAKE, -1, 2, None),
     "Broadcast add extents cannot be negative"),
    (lambda l: l.cuvit_add_broadcast_f32(None, FAKE, 4, 2, None),
     "Broadcast add operands cannot be null"),
    (lambda l: l.cuvit_broadcast_f32(FAKE, FAKE, 8, 4, 2, None), "Broadcast extents are inconsistent"),
    (lambda l: l.cuvit_broadcast_f32(FAKE, FAKE, 4, 8, -2, None), "Broadcast extents are inconsistent"),
    (lambda l: l.cuvit_broadcast_f32(FAKE, None, 4, 8, 2, None), "Broadcast operands cannot be null"),
    (lambda l: l.cuvit_extract_patches_f32(FAKE, FAKE, 1, 0, 16, 16, 4, None),
     "Patch extraction dimensions must be positive"),
    (lambda l: l.cuvit_extract_patches_f32(FAKE, FAKE, -1, 3, 16, 16, 4, None),
     "Patch extraction dimensions must be positive"),
    (lambda l: l.cuvit_extract_patches_f32(FAKE, FAKE, 1, 3, 18, 16, 4, None),
     "Patch extraction needs the image to divide into whole patches"),
    (lambda l: l.cuvit_extract_patches_f32(None, FAKE, 1, 3, 16, 16, 4, None),
     "Patch extraction operands cannot be null"),
    (lambda l: l.cuvit_extract_patches_bf16(FAKE, None, 2, 3, 224, 224, 16, None),
     "Patch extraction operands cannot be null"),
    (lambda l: l.cuvit_gelu_bf16(FAKE, None, 3, None), "GELU operands cannot be null"),
    (lambda l: l.cuvit_attention_f32(FAKE, FAKE, 2, -3, 197, 64, None),
     "Attention extents cannot be negative"),
    (lambda l: l.cuvit_attention_f32(None, FAKE, 2, 3, 197, 64, None),
     "Attention operands cannot be null"),
    (lambda l: l.cuvit_attention_f32(FAKE, FAKE, 2, 3, 197, 32, None),
     "Fused attention supports head_dim 64 and at most 256 tokens"),
    (lambda l: l.cuvit_attention_f32(FAKE, FAKE, 2, 3, 257, 64, None),
     "Fused attention supports head_dim 64 and at most 256 tokens"),
    (lambda l: l.cuvit_attention_f32(FAKE + 4, FAKE, 2, 3, 197, 64, None),
     "Fused attention needs 16-byte aligned operands"),
    (lambda l: l.cuvit_attention_bf16(FAKE, FAKE, 2, 3, 197, 32, None),
     "Fused attention supports head_dim 64 and at most 256 tokens"),
    (lambda l: l.cuvit_attention_bf16(FAKE, None, 2, 3, 197, 64, None),
     "Attention operands cannot be null"),
    (lambda l: l.cuvit_attention_bf16(FAKE + 8, FAKE, 2, 3, 197, 64, None),
     "Fused attention needs 16-byte aligned operands"),
    (lambda l: l.cuvit_broadcast_bf16(FAKE, FAKE, 8, 4, 2, None), "Broadcast extents are inconsistent"),
    (lambda l: l.cuvit_broadcast_bf16(None, FAKE, 4, 8, 2, None), "Broadcast operands cannot be null"),
    (lambda l: l.cuvit_convert_f32_to_bf16(FAKE, FAKE, -1, None), "GELU element count cannot be negative"),
    (lambda l: l.cuvit_convert_f32_to_bf16(FAKE, None, 4, None), "GELU operands cannot be null"),
    (lambda l: l.cuvit_convert_bf16_to_f32(None, FAKE, 4, None), "GELU operands cannot be null"),
])
def test_invalid_arguments(cuvit, lib, call, message):
    status = call(lib)
    assert status == cuvit.ERROR_INVALID_ARGUMENT
    assert lib.cuvit_last_error().decode() == message


def test_oversized_launches_are_length_errors(cuvit, lib):
    """normalization.cu:214-220: more than 2^31 - 1 blocks of 256 threads."""
    huge = (1 << 31) * 256
    for status in (lib.cuvit_gelu_f32(FAKE, FAKE, huge, None),
                   lib.cuvit_add_f32(FAKE, FAKE, huge, None),
                   lib.cuvit_add_broadcast_f32(FAKE, FAKE, 1 << 30, 1 << 20, None),
                   lib.cuvit_broadcast_f32(FAKE, FAKE, 1 << 30, 1 << 30, 1 << 20, None),
                   lib.cuvit_broadcast_bf16(FAKE, FAKE, 1 << 30, 1 << 30, 1 << 20, None),
                   lib.cuvit_convert_f32_to_bf16(FAKE, FAKE, huge, None),
                   lib.cuvit_extract_patches_f32(FAKE, FAKE, 1 << 20, 3, 1 << 14, 1 << 14, 16, None)):
        assert status == cuvit.ERROR_LENGTH
        assert "grid limit" in lib.cuvit_last_error().decode()


def test_attention_shape_limits(cuvit, lib):
    assert cuvit.attention_supported(197, 64) and cuvit.attention_supported(256, 64)
    assert cuvit.attention_supported(1, 64)
    assert not cuvit.attention_supported(257, 64) and not cuvit.attention_supported(197, 96)
    assert lib.cuvit_attention_f32(FAKE, FAKE, 256, 256, 197, 64, None) == cuvit.ERROR_LENGTH
    assert "65535" in lib.cuvit_last_error().decode()
    # an image's QKV rows past the kernels' 32-bit offsets: 256 tokens of
    # 3 x 10923 heads x 64 fp32 values are 65,552 bytes more than 0x7FFFFFF0
    # (10922 heads would fit); bf16 halves the bytes
    assert lib.cuvit_attention_f32(FAKE, FAKE, 1, 10923, 256, 64, None) == cuvit.ERROR_LENGTH
    assert "2^31 - 16 bytes" in lib.cuvit_last_error().decode()
    assert lib.cuvit_attention_bf16(FAKE, FAKE, 1, 21846, 256, 64, None) == cuvit.ERROR_LENGTH
    assert "2^31 - 16 bytes" in lib.cuvit_last_error().decode()


def gemm_status(cuvit, lib, a=FAKE, b=FAKE, c=FAKE, **fields):
    p = cuvit.gemm_problem(fields.pop("m", 4), fields.pop("n", 4), fields.pop("k", 4),
                           fields.pop("layout", cuvit.NO_TRANSPOSE))
    for key, value in fields.items():
        if key in ("count", "inner"):
            setattr(p.batch, key, value)
        else:
            setattr(p, key, value)
    return lib.cuvit_gemm_f32(a, b, None, c, ctypes.byref(p), None)


def test_gemm_validation_order(cuvit, lib):
    """gemm.cu:205-231, in order."""
    assert gemm_status(cuvit, lib, a=None, b=None, c=None, m=0) == 0
    assert gemm_status(cuvit, lib, a=None, b=None, c=None, n=0) == 0
    assert gemm_status(cuvit, lib, a=None, b=None, c=None, count=0) == 0
    cases = [
        (dict(m=-1), "GEMM dimensions cannot be negative"),
        (dict(k=-1), "GEMM dimensions cannot be negative"),
        (dict(count=-3), "GEMM dimensions cannot be negative"),
        (dict(count=6, inner=4), "A split GEMM batch must divide into whole inner groups"),
        (dict(a=None), "GEMM operands cannot be null"),
        (dict(c=None, count=6, inner=3), "GEMM operands cannot be null"),
        (dict(lda=3), "A GEMM leading dimension is smaller than its row"),
        (dict(ldc=3), "A GEMM leading dimension is smaller than its row"),
        (dict(ldb=3, layout=1), "A GEMM leading dimension is smaller than its row"),
        (dict(ldb=3, layout=0, n=5, k=2), "A GEMM leading dimension is smaller than its row"),
        (dict(layout=7), "GEMM layout is not a GemmLayout value"),
    ]
    for fields, message in cases:
        assert gemm_status(cuvit, lib, **fields) == cuvit.ERROR_INVALID_ARGUMENT, fields
        assert lib.cuvit_last_error().decode() == message, fields
    # the split check precedes the null check (gemm.cu:211-216)
    assert gemm_status(cuvit, lib, a=None, count=6, inner=4) == cuvit.ERROR_INVALID_ARGUMENT
    assert "split" in lib.cuvit_last_error().decode()


def test_python_errors_carry_the_status(cuvit):
    with pytest.raises(cuvit.InvalidArgument) as info:
        cuvit.softmax(None, FAKE, 2, 2)
    assert isinstance(info.value, ValueError)
    assert "null" in str(info.value)
    with pytest.raises(cuvit.LengthError):
        cuvit.gelu(FAKE, FAKE, (1 << 31) * 256)


def test_config_validation(cuvit):
    """vit_test.cu:324-345 and VitConfig::validate (vit.cu:36-47)."""
    config = cuvit.default_config()
    assert (config.image_size, config.patch_size, config.channels, config.embed_dim,
            config.depth, config.heads, config.mlp_hidden, config.classes) == \
        (224, 16, 3, 192, 12, 3, 768, 1000)
    assert abs(config.layer_norm_epsilon - 1e-6) < 1e-12
    cuvit.validate_config(config)
    config.embed_dim = 25
    config.heads = 4
    with pytest.raises(cuvit.InvalidArgument, match="divide across the heads"):
        cuvit.validate_config(config)
    config = cuvit.default_config()
    config.image_size = 30
    with pytest.raises(cuvit.InvalidArgument, match="whole patches"):
        cuvit.validate_config(config)
    config = cuvit.default_config()
    config.depth = 0
    with pytest.raises(cuvit.InvalidArgument, match="positive"):
        cuvit.validate_config(config)


def test_expected_tensor_names(cuvit):
    """vit.cu:49-63: 4 + 12 * depth + 4 timm names; ViT-Tiny has 152."""
    names = cuvit.expected_tensor_names(cuvit.default_config())
    assert len(names) == 152
    assert names[0][0] == "cls_token" and names[-1][0] == "head.bias"
    assert sum(int(__import__("numpy").prod(s)) for _, s in names) == 5717416


def test_model_precision_is_validated_before_any_allocation(cuvit, lib, tmp_path):
    """cuvit_vit_create_ex rejects an unknown precision before it touches the device."""
    writer = cuvit.WeightWriter()
    writer.add("cls_token", __import__("numpy").zeros((1, 1, 4), "float32"))
    path = str(tmp_path / "one.cvw")
    writer.write(path)
    weights = cuvit.WeightFile(path)
    config = cuvit.default_config()
    handle = ctypes.c_void_p()
    status = lib.cuvit_vit_create_ex(ctypes.byref(config), weights.handle, 1, 7, ctypes.byref(handle))
    assert status == cuvit.ERROR_INVALID_ARGUMENT
    assert lib.cuvit_last_error().decode() == "precision is not a cuvit_precision value"
    assert not handle.value
    assert lib.cuvit_vit_precision(None) == -1
    assert (cuvit.PRECISION_F32, cuvit.PRECISION_BF16) == (0, 1)


def test_last_error_belongs_to_the_calling_thread(cuvit):
    """Launchers may be called from any host thread (kernels.hpp: stateless,
    re-entrant), so the message a failing call leaves behind is its own
    thread's. Four threads each fail in their own way 500 times, concurrently;
    ctypes releases the interpreter lock around both the failing call and the
    message read, so a shared message would show up here as another thread's."""
    import threading

    cases = [
        (lambda: cuvit.layer_norm(FAKE, FAKE, FAKE, FAKE, -1, 4),
         "Layer norm dimensions cannot be negative"),
        (lambda: cuvit.softmax(None, None, 2, 3), "Softmax operands cannot be null"),
        (lambda: cuvit.gelu(FAKE, FAKE, -5), "GELU element count cannot be negative"),
        (lambda: cuvit.extract_patches(FAKE, FAKE, 1, 3, 10, 10, 4),
         "Patch extraction needs the image to divide into whole patches"),
    ]
    barrier = threading.Barrier(len(cases))
    failures = []

    def run(call, expected):
        barrier.wait()
        for _ in range(500):
            try:
                call()
            except cuvit.InvalidArgument as error:
                if expected not in str(error):
                    failures.append(f"expected {expected!r}, got {error}")
                    return
            else:
                failures.append(f"no error for {expected!r}")
                return

    threads = [threading.Thread(target=run, args=case) for case in cases]
    for thread in threads:
        thread.start()
    for thread in threads:
        thread.join()
    assert not failures, failures[:3]


def test_host_tensors_are_refused_before_any_launch(cuvit):
    """A torch tensor in host memory never reaches a kernel as a device address:
    the binding names the operand and raises InvalidArgument. Zero and negative
    extents still go to the library's own checks first."""
    import torch

    x = torch.zeros(4 * 8)
    g = torch.ones(8)
    with pytest.raises(cuvit.InvalidArgument, match="x is not a GPU tensor"):
        cuvit.layer_norm(x, g, g, FAKE, 4, 8)
    with pytest.raises(cuvit.InvalidArgument, match="out is not a GPU tensor"):
        cuvit.softmax(FAKE, x, 4, 8)
    with pytest.raises(cuvit.InvalidArgument, match="images is not a GPU tensor"):
        cuvit.extract_patches(torch.zeros(3 * 16 * 16), FAKE, 1, 3, 16, 16, 8)
    with pytest.raises(cuvit.InvalidArgument, match="A is not a GPU tensor"):
        cuvit.gemm(torch.zeros(12), FAKE, None, FAKE, cuvit.gemm_problem(3, 4, 4))
    with pytest.raises(cuvit.InvalidArgument, match="pixels is not a GPU tensor"):
        cuvit.preprocess(torch.zeros(4 * 4 * 3, dtype=torch.uint8), FAKE, 1, 4, 4,
                         cuvit.Preprocessing(size=4))
    # The library's order still holds where an extent is zero or negative.
    cuvit.layer_norm(x, g, g, x, 0, 8)
    with pytest.raises(cuvit.InvalidArgument, match="cannot be negative"):
        cuvit.gelu(x, x, -5)


def test_gemm_operand_spans_follow_the_batch_layout(cuvit):
    """The elements a GEMM touches per operand, which the binding requires each
    tensor to hold: the last batch entry's offset plus its last row."""
    from cuvit_amd import _offset_range

    assert _offset_range(1, 0, 100, 0) == (0, 0)
    assert _offset_range(4, 0, 100, 0) == (0, 300)
    assert _offset_range(6, 3, 10, 1000) == (0, 1000 + 20)    # 2 outer groups of 3
    assert _offset_range(6, 6, 10, 1000) == (0, 50)           # one group: flat
    assert _offset_range(4, 0, -5, 0) == (-15, 0)
