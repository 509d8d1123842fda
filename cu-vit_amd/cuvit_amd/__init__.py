"""Python binding of libcuvit_amd.so, the MI355X (gfx950) layer-kernel library.

The library's interface is the C ABI in include/cuvit/capi.h; this module binds
it with ctypes so tests and the benchmark can drive the HIP kernels on device
tensors that PyTorch allocates. PyTorch provides device memory and the stream
handle only; every computation runs in the library's own HIP kernels. There is
no fallback: if the library is not built, loading raises.

Launcher functions mirror the reference's kernels.hpp (names, argument order,
error behaviour): an invalid argument raises InvalidArgument (a ValueError, the
counterpart of std::invalid_argument), an oversized launch raises LengthError,
and a failed launch raises HipError.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

__all__ = [
    "CuvitError", "InvalidArgument", "LengthError", "HipError", "OutOfRange",
    "GemmProblem", "VitConfig", "library", "library_path", "check", "stream_handle",
    "gemm", "layer_norm", "softmax", "gelu", "extract_patches", "extract_patches_f32_to_bf16",
    "add", "add_broadcast",
    "broadcast", "convert_to_bf16", "convert_to_f32", "attention", "attention_supported",
    "gemm_problem", "WeightWriter", "WeightFile", "VisionTransformer",
    "NO_TRANSPOSE", "TRANSPOSED", "PRECISION_F32", "PRECISION_BF16",
    "Preprocessing", "RgbImage", "load_ppm", "preprocess", "preprocess_image", "cli_path",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
_DEFAULT_LIB = os.path.join(os.path.dirname(_HERE), "lib", "libcuvit_amd.so")

NO_TRANSPOSE = 0
TRANSPOSED = 1

PRECISION_F32 = 0
PRECISION_BF16 = 1

OK = 0
ERROR_INVALID_ARGUMENT = 1
ERROR_LENGTH = 2
ERROR_HIP = 3
ERROR_RUNTIME = 4
ERROR_OUT_OF_RANGE = 5


class CuvitError(RuntimeError):
    """Base of the errors a C-ABI status turns into."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class InvalidArgument(CuvitError, ValueError):
    """CUVIT_ERROR_INVALID_ARGUMENT (std::invalid_argument in the reference)."""


class LengthError(CuvitError):
    """CUVIT_ERROR_LENGTH (std::length_error)."""


class HipError(CuvitError):
    """CUVIT_ERROR_HIP (CudaError in the reference); .hip_code is the hipError_t."""

    def __init__(self, status: int, message: str, hip_code: int):
        super().__init__(status, message)
        self.hip_code = hip_code


class OutOfRange(CuvitError, IndexError):
    """CUVIT_ERROR_OUT_OF_RANGE (std::out_of_range)."""


class GemmBatch(ctypes.Structure):
    _fields_ = [
        ("count", ctypes.c_int),
        ("stride_a", ctypes.c_int64),
        ("stride_b", ctypes.c_int64),
        ("stride_c", ctypes.c_int64),
        ("inner", ctypes.c_int),
        ("outer_stride_a", ctypes.c_int64),
        ("outer_stride_b", ctypes.c_int64),
        ("outer_stride_c", ctypes.c_int64),
    ]


class GemmEpilogue(ctypes.Structure):
    _fields_ = [("accumulate", ctypes.c_uint8), ("gelu", ctypes.c_uint8)]


class GemmProblem(ctypes.Structure):
    """cuvit_gemm_problem / cuvit::GemmProblem (reference kernels.hpp:74-85)."""

    _fields_ = [
        ("m", ctypes.c_int),
        ("n", ctypes.c_int),
        ("k", ctypes.c_int),
        ("layout", ctypes.c_int32),
        ("alpha", ctypes.c_float),
        ("lda", ctypes.c_int),
        ("ldb", ctypes.c_int),
        ("ldc", ctypes.c_int),
        ("batch", GemmBatch),
        ("epilogue", GemmEpilogue),
    ]


class VitConfig(ctypes.Structure):
    """cuvit_vit_config / cuvit::VitConfig (reference vit.hpp:15-35)."""

    _fields_ = [
        ("image_size", ctypes.c_int),
        ("patch_size", ctypes.c_int),
        ("channels", ctypes.c_int),
        ("embed_dim", ctypes.c_int),
        ("depth", ctypes.c_int),
        ("heads", ctypes.c_int),
        ("mlp_hidden", ctypes.c_int),
        ("classes", ctypes.c_int),
        ("layer_norm_epsilon", ctypes.c_float),
    ]

    def patches_per_side(self) -> int:
        return self.image_size // self.patch_size

    def patch_count(self) -> int:
        return self.patches_per_side() ** 2

    def token_count(self) -> int:
        return self.patch_count() + 1

    def head_dim(self) -> int:
        return self.embed_dim // self.heads

    def patch_elements(self) -> int:
        return self.channels * self.patch_size * self.patch_size


class Preprocessing(ctypes.Structure):
    """cuvit_preprocessing / cuvit::Preprocessing (reference image.hpp:30-38),
    with the reference's defaults: size 224, crop fraction 0.9, mean and
    stddev 0.5 per channel."""

    _fields_ = [
        ("size", ctypes.c_int),
        ("crop_fraction", ctypes.c_float),
        ("mean", ctypes.c_float * 3),
        ("stddev", ctypes.c_float * 3),
    ]

    def __init__(self, size: int = 224, crop_fraction: float = 0.9,
                 mean=(0.5, 0.5, 0.5), stddev=(0.5, 0.5, 0.5)):
        super().__init__(size, crop_fraction, (ctypes.c_float * 3)(*mean),
                         (ctypes.c_float * 3)(*stddev))


_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_SIGNATURES = {
    "cuvit_last_error": (ctypes.c_char_p, []),
    "cuvit_last_hip_error": (_I, []),
    "cuvit_version": (_I, []),
    "cuvit_gemm_problem_init": (None, [ctypes.POINTER(GemmProblem), _I, _I, _I, _I]),
    "cuvit_gemm_f32": (_I, [_P, _P, _P, _P, ctypes.POINTER(GemmProblem), _P]),
    "cuvit_gemm_bf16": (_I, [_P, _P, _P, _P, ctypes.POINTER(GemmProblem), _P]),
    "cuvit_layer_norm_f32": (_I, [_P, _P, _P, _P, _I, _I, _F, _P]),
    "cuvit_layer_norm_bf16": (_I, [_P, _P, _P, _P, _I, _I, _F, _P]),
    "cuvit_gelu_f32": (_I, [_P, _P, _L, _P]),
    "cuvit_gelu_bf16": (_I, [_P, _P, _L, _P]),
    "cuvit_softmax_f32": (_I, [_P, _P, _I, _I, _P]),
    "cuvit_softmax_bf16": (_I, [_P, _P, _I, _I, _P]),
    "cuvit_extract_patches_f32": (_I, [_P, _P, _I, _I, _I, _I, _I, _P]),
    "cuvit_extract_patches_bf16": (_I, [_P, _P, _I, _I, _I, _I, _I, _P]),
    "cuvit_extract_patches_f32_to_bf16": (_I, [_P, _P, _I, _I, _I, _I, _I, _P]),
    "cuvit_add_f32": (_I, [_P, _P, _L, _P]),
    "cuvit_add_broadcast_f32": (_I, [_P, _P, _L, _I, _P]),
    "cuvit_broadcast_f32": (_I, [_P, _P, _L, _L, _I, _P]),
    "cuvit_broadcast_bf16": (_I, [_P, _P, _L, _L, _I, _P]),
    "cuvit_convert_f32_to_bf16": (_I, [_P, _P, _L, _P]),
    "cuvit_convert_bf16_to_f32": (_I, [_P, _P, _L, _P]),
    "cuvit_attention_supported": (_I, [_I, _I]),
    "cuvit_attention_f32": (_I, [_P, _P, _I, _I, _I, _I, _P]),
    "cuvit_attention_bf16": (_I, [_P, _P, _I, _I, _I, _I, _P]),
    "cuvit_weight_writer_create": (_I, [ctypes.POINTER(_P)]),
    "cuvit_weight_writer_add": (_I, [_P, ctypes.c_char_p, _I, ctypes.POINTER(_L), _P]),
    "cuvit_weight_writer_add_bf16": (_I, [_P, ctypes.c_char_p, _I, ctypes.POINTER(_L), _P]),
    "cuvit_weight_writer_write": (_I, [_P, ctypes.c_char_p]),
    "cuvit_weight_writer_destroy": (None, [_P]),
    "cuvit_weight_file_load": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "cuvit_weight_file_size": (_L, [_P]),
    "cuvit_weight_file_contains": (_I, [_P, ctypes.c_char_p]),
    "cuvit_weight_file_float_data": (_I, [_P, ctypes.c_char_p, _I, ctypes.POINTER(_L), ctypes.POINTER(_P)]),
    "cuvit_weight_file_bf16_data": (_I, [_P, ctypes.c_char_p, _I, ctypes.POINTER(_L), ctypes.POINTER(_P)]),
    "cuvit_weight_file_version": (_I, [_P]),
    "cuvit_weight_file_type": (_I, [_P, ctypes.c_char_p]),
    "cuvit_weight_file_entry_name": (ctypes.c_char_p, [_P, _L]),
    "cuvit_weight_file_payload_bytes": (ctypes.c_uint64, [_P]),
    "cuvit_weight_file_destroy": (None, [_P]),
    "cuvit_vit_config_default": (None, [ctypes.POINTER(VitConfig)]),
    "cuvit_vit_config_validate": (_I, [ctypes.POINTER(VitConfig)]),
    "cuvit_vit_create": (_I, [ctypes.POINTER(VitConfig), _P, _I, ctypes.POINTER(_P)]),
    "cuvit_vit_create_ex": (_I, [ctypes.POINTER(VitConfig), _P, _I, _I, ctypes.POINTER(_P)]),
    "cuvit_vit_precision": (_I, [_P]),
    "cuvit_vit_forward": (_I, [_P, _P, _P, _I, _P]),
    "cuvit_vit_weight_bytes": (ctypes.c_uint64, [_P]),
    "cuvit_vit_activation_bytes": (ctypes.c_uint64, [_P]),
    "cuvit_vit_destroy": (None, [_P]),
    "cuvit_image_load_ppm": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "cuvit_image_width": (_I, [_P]),
    "cuvit_image_height": (_I, [_P]),
    "cuvit_image_pixels": (_P, [_P]),
    "cuvit_image_destroy": (None, [_P]),
    "cuvit_preprocessing_default": (None, [ctypes.POINTER(Preprocessing)]),
    "cuvit_preprocess_u8": (_I, [_P, _I, _I, _I, ctypes.POINTER(Preprocessing), _P, _P]),
}

_lib: Optional[ctypes.CDLL] = None


def library_path() -> str:
    return os.environ.get("CUVIT_AMD_LIBRARY", _DEFAULT_LIB)


def library() -> ctypes.CDLL:
    """The loaded libcuvit_amd.so. Raises if it has not been built."""
    global _lib
    if _lib is None:
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"libcuvit_amd.so not found at {path}: build it first "
                "(python -c 'import __graft_entry__ as g; g.build()' or make -C cu-vit_amd)")
        lib = ctypes.CDLL(path)
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def check(status: int) -> None:
    """Raises the exception matching a C-ABI status."""
    if status == OK:
        return
    lib = library()
    message = (lib.cuvit_last_error() or b"").decode()
    if status == ERROR_INVALID_ARGUMENT:
        raise InvalidArgument(status, message)
    if status == ERROR_LENGTH:
        raise LengthError(status, message)
    if status == ERROR_HIP:
        raise HipError(status, message, lib.cuvit_last_hip_error())
    if status == ERROR_OUT_OF_RANGE:
        raise OutOfRange(status, message)
    raise CuvitError(status, message)


def _ptr(x) -> Optional[int]:
    """Device address of a torch tensor, an int address, or None (NULL)."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _operand(x, name: str, dtype: str, elements: int) -> Optional[int]:
    """The address of operand @p x after checking that the kernel may touch
    @p elements of it: a torch tensor must live on the GPU, hold @p dtype
    ("float32", "bfloat16" or "uint8"), be contiguous and have at least that
    many elements; anything else would be a device access outside the
    tensor or a host address read by the GPU. Raw int addresses and None go
    through unchecked, as in the C API (None becomes NULL, which the library
    rejects with its own message)."""
    if x is None or isinstance(x, int):
        return x
    if x.device.type != "cuda":
        raise InvalidArgument(ERROR_INVALID_ARGUMENT, f"{name} is not a GPU tensor ({x.device})")
    if str(x.dtype) != "torch." + dtype:
        raise InvalidArgument(ERROR_INVALID_ARGUMENT,
                              f"{name} holds {x.dtype}; this launch needs torch.{dtype}")
    if not x.is_contiguous():
        raise InvalidArgument(ERROR_INVALID_ARGUMENT, f"{name} is not contiguous")
    if x.numel() < elements:
        raise InvalidArgument(ERROR_INVALID_ARGUMENT,
                              f"{name} holds {x.numel()} elements; the launch touches {elements}")
    return x.data_ptr()


def _positive(*extents) -> bool:
    """True when every extent is positive: only then are the operand checks
    applied, so that zero and negative extents reach the library's own
    checks in the reference's order (a zero extent returns first, even with
    null pointers; a negative one is InvalidArgument)."""
    return all(int(e) > 0 for e in extents)


def _storage(bf16: bool) -> str:
    return "bfloat16" if bf16 else "float32"


def _offset_range(count: int, inner: int, stride: int, outer_stride: int):
    """Smallest and largest element offset of a batch entry's operand
    (split batches: entry i sits at (i / inner) * outer_stride + (i % inner)
    * stride; flat ones at i * stride)."""
    if 0 < inner < count:
        outer_span = (count // inner - 1) * outer_stride
        inner_span = (inner - 1) * stride
        return (min(0, outer_span) + min(0, inner_span), max(0, outer_span) + max(0, inner_span))
    span = (count - 1) * stride
    return min(0, span), max(0, span)


def _gemm_operands(a, b, bias, c, problem: "GemmProblem", bf16: bool):
    p = problem
    if not _positive(p.m, p.n, p.batch.count) or p.k < 0:
        return _ptr(a), _ptr(b), _ptr(bias), _ptr(c)
    transposed = p.layout == TRANSPOSED
    lda = p.lda or p.k
    ldb = p.ldb or (p.k if transposed else p.n)
    ldc = p.ldc or p.n
    if lda < p.k or ldc < p.n or ldb < (p.k if transposed else p.n):
        return _ptr(a), _ptr(b), _ptr(bias), _ptr(c)  # the library names the bad ld
    count, inner = p.batch.count, p.batch.inner

    def span(rows: int, ld: int, cols: int, stride: int, outer_stride: int, name: str) -> int:
        if rows <= 0 or cols <= 0:
            return 0
        low, high = _offset_range(count, inner, stride, outer_stride)
        if low < 0:
            raise InvalidArgument(ERROR_INVALID_ARGUMENT,
                                  f"{name}: a batch entry starts before the tensor")
        return high + (rows - 1) * ld + cols

    t = _storage(bf16)
    a_rows, a_cols = p.m, p.k
    b_rows, b_cols = (p.n, p.k) if transposed else (p.k, p.n)
    return (_operand(a, "A", t, span(a_rows, lda, a_cols, p.batch.stride_a,
                                     p.batch.outer_stride_a, "A")),
            _operand(b, "B", t, span(b_rows, ldb, b_cols, p.batch.stride_b,
                                     p.batch.outer_stride_b, "B")),
            _operand(bias, "bias", "float32", p.n),
            _operand(c, "C", t, span(p.m, ldc, p.n, p.batch.stride_c, p.batch.outer_stride_c, "C")))


def stream_handle(stream=None) -> Optional[int]:
    """hipStream_t of a torch stream (default: torch's current stream)."""
    import torch

    if stream is None:
        if not torch.cuda.is_available():
            return None  # host-only use: argument validation never reaches a stream
        stream = torch.cuda.current_stream()
    return stream.cuda_stream or None


def _bf16(x) -> bool:
    if x is None or isinstance(x, int):
        return False
    import torch

    return x.dtype == torch.bfloat16


def gemm_problem(m: int, n: int, k: int, layout: int = NO_TRANSPOSE) -> GemmProblem:
    """The reference's gemm_problem() (kernels.hpp:89-96)."""
    problem = GemmProblem()
    library().cuvit_gemm_problem_init(ctypes.byref(problem), m, n, k, layout)
    return problem


def gemm(a, b, bias, c, problem: GemmProblem, stream=None, bf16: Optional[bool] = None) -> None:
    bf16 = bf16 if bf16 is not None else _bf16(a)
    fn = library().cuvit_gemm_bf16 if bf16 else library().cuvit_gemm_f32
    pa, pb, pbias, pc = _gemm_operands(a, b, bias, c, problem, bf16)
    check(fn(pa, pb, pbias, pc, ctypes.byref(problem), stream_handle(stream)))


def layer_norm(x, gamma, beta, out, rows: int, columns: int, epsilon: float = 1.0e-6,
               stream=None, bf16: Optional[bool] = None) -> None:
    bf16 = bf16 if bf16 is not None else _bf16(x)
    fn = library().cuvit_layer_norm_bf16 if bf16 else library().cuvit_layer_norm_f32
    if _positive(rows, columns):
        t, n = _storage(bf16), rows * columns
        x, out = _operand(x, "x", t, n), _operand(out, "out", t, n)
        gamma = _operand(gamma, "gamma", "float32", columns)
        beta = _operand(beta, "beta", "float32", columns)
    check(fn(_ptr(x), _ptr(gamma), _ptr(beta), _ptr(out), rows, columns, epsilon,
             stream_handle(stream)))


def softmax(x, out, rows: int, columns: int, stream=None, bf16: Optional[bool] = None) -> None:
    bf16 = bf16 if bf16 is not None else _bf16(x)
    fn = library().cuvit_softmax_bf16 if bf16 else library().cuvit_softmax_f32
    if _positive(rows, columns):
        t, n = _storage(bf16), rows * columns
        x, out = _operand(x, "x", t, n), _operand(out, "out", t, n)
    check(fn(_ptr(x), _ptr(out), rows, columns, stream_handle(stream)))


def gelu(x, out, count: int, stream=None, bf16: Optional[bool] = None) -> None:
    bf16 = bf16 if bf16 is not None else _bf16(x)
    fn = library().cuvit_gelu_bf16 if bf16 else library().cuvit_gelu_f32
    if _positive(count):
        x, out = _operand(x, "x", _storage(bf16), count), _operand(out, "out", _storage(bf16), count)
    check(fn(_ptr(x), _ptr(out), count, stream_handle(stream)))


def extract_patches(images, patches, batch: int, channels: int, height: int, width: int,
                    patch: int, stream=None, bf16: Optional[bool] = None) -> None:
    bf16 = bf16 if bf16 is not None else _bf16(images)
    fn = library().cuvit_extract_patches_bf16 if bf16 else library().cuvit_extract_patches_f32
    if _positive(batch, channels, height, width, patch):
        n = batch * channels * height * width
        images = _operand(images, "images", _storage(bf16), n)
        patches = _operand(patches, "patches", _storage(bf16), n)
    check(fn(_ptr(images), _ptr(patches), batch, channels, height, width, patch,
             stream_handle(stream)))


def extract_patches_f32_to_bf16(images, patches, batch: int, channels: int, height: int,
                                width: int, patch: int, stream=None) -> None:
    """fp32 images into bf16 patch rows in one pass (bitwise the conversion
    then the bf16 gather)."""
    if _positive(batch, channels, height, width, patch):
        n = batch * channels * height * width
        images = _operand(images, "images", "float32", n)
        patches = _operand(patches, "patches", _storage(True), n)
    check(library().cuvit_extract_patches_f32_to_bf16(_ptr(images), _ptr(patches), batch, channels,
                                                      height, width, patch, stream_handle(stream)))


def add(accumulator, addend, count: int, stream=None) -> None:
    if _positive(count):
        accumulator = _operand(accumulator, "accumulator", "float32", count)
        addend = _operand(addend, "addend", "float32", count)
    check(library().cuvit_add_f32(_ptr(accumulator), _ptr(addend), count, stream_handle(stream)))


def add_broadcast(accumulator, addend, count: int, batch: int, stream=None) -> None:
    if _positive(count, batch):
        accumulator = _operand(accumulator, "accumulator", "float32", count * batch)
        addend = _operand(addend, "addend", "float32", count)
    check(library().cuvit_add_broadcast_f32(_ptr(accumulator), _ptr(addend), count, batch,
                                            stream_handle(stream)))


def broadcast(destination, source, count: int, destination_stride: int, batch: int,
              stream=None, bf16: Optional[bool] = None) -> None:
    bf16 = bf16 if bf16 is not None else _bf16(destination)
    fn = library().cuvit_broadcast_bf16 if bf16 else library().cuvit_broadcast_f32
    if _positive(count, batch) and destination_stride >= count:
        destination = _operand(destination, "destination", _storage(bf16),
                               (batch - 1) * destination_stride + count)
        source = _operand(source, "source", _storage(bf16), count)
    check(fn(_ptr(destination), _ptr(source), count, destination_stride, batch,
             stream_handle(stream)))


def convert_to_bf16(x, out, count: int, stream=None) -> None:
    """fp32 -> bf16, round to nearest-even (an extension)."""
    if _positive(count):
        x, out = _operand(x, "x", "float32", count), _operand(out, "out", "bfloat16", count)
    check(library().cuvit_convert_f32_to_bf16(_ptr(x), _ptr(out), count, stream_handle(stream)))


def convert_to_f32(x, out, count: int, stream=None) -> None:
    """bf16 -> fp32, exact (an extension)."""
    if _positive(count):
        x, out = _operand(x, "x", "bfloat16", count), _operand(out, "out", "float32", count)
    check(library().cuvit_convert_bf16_to_f32(_ptr(x), _ptr(out), count, stream_handle(stream)))


def attention_supported(tokens: int, head_dim: int) -> bool:
    """True when the fused attention kernel covers (tokens, head_dim)."""
    return bool(library().cuvit_attention_supported(tokens, head_dim))


def attention(qkv, context, images: int, heads: int, tokens: int, head_dim: int,
              stream=None) -> None:
    """Fused softmax(Q.K^T / sqrt(head_dim)).V from the packed
    [images, tokens, 3, heads, head_dim] projection into
    [images, tokens, heads, head_dim]; an extension replacing the reference's
    three attention launches (vit.cu:205-245) with bitwise the same result."""
    bf16 = _bf16(qkv)
    fn = library().cuvit_attention_bf16 if bf16 else library().cuvit_attention_f32
    if _positive(images, heads, tokens, head_dim):
        n = images * tokens * heads * head_dim
        qkv = _operand(qkv, "qkv", _storage(bf16), 3 * n)
        context = _operand(context, "context", _storage(bf16), n)
    check(fn(_ptr(qkv), _ptr(context), images, heads, tokens, head_dim, stream_handle(stream)))


class WeightWriter:
    """WeightFileWriter (reference weights.hpp:78-92) over the C ABI."""

    def __init__(self):
        handle = ctypes.c_void_p()
        check(library().cuvit_weight_writer_create(ctypes.byref(handle)))
        self._handle = handle

    def add(self, name: str, array) -> None:
        import numpy as np

        data = np.ascontiguousarray(array, dtype=np.float32)
        extents = (ctypes.c_int64 * max(data.ndim, 1))(*data.shape)
        check(library().cuvit_weight_writer_add(self._handle, name.encode(), data.ndim, extents,
                                                data.ctypes.data))

    def add_bf16(self, name: str, bits) -> None:
        """A bfloat16 tensor from its bit patterns (uint16); the file becomes version 2."""
        import numpy as np

        data = np.ascontiguousarray(bits, dtype=np.uint16)
        extents = (ctypes.c_int64 * max(data.ndim, 1))(*data.shape)
        check(library().cuvit_weight_writer_add_bf16(self._handle, name.encode(), data.ndim,
                                                     extents, data.ctypes.data))

    def write(self, path: str) -> None:
        check(library().cuvit_weight_writer_write(self._handle, os.fsencode(path)))

    def close(self) -> None:
        if getattr(self, "_handle", None):
            library().cuvit_weight_writer_destroy(self._handle)
            self._handle = None

    def __del__(self):
        self.close()


class WeightFile:
    """WeightFile (reference weights.hpp:45-74) over the C ABI."""

    def __init__(self, path: str):
        handle = ctypes.c_void_p()
        check(library().cuvit_weight_file_load(os.fsencode(path), ctypes.byref(handle)))
        self._handle = handle

    @property
    def handle(self):
        return self._handle

    def __len__(self) -> int:
        return library().cuvit_weight_file_size(self._handle)

    def contains(self, name: str) -> bool:
        return bool(library().cuvit_weight_file_contains(self._handle, name.encode()))

    def names(self):
        lib = library()
        return [lib.cuvit_weight_file_entry_name(self._handle, i).decode() for i in range(len(self))]

    def payload_bytes(self) -> int:
        return library().cuvit_weight_file_payload_bytes(self._handle)

    def float_data(self, name: str, shape):
        import numpy as np

        extents = (ctypes.c_int64 * max(len(shape), 1))(*shape)
        pointer = ctypes.c_void_p()
        check(library().cuvit_weight_file_float_data(self._handle, name.encode(), len(shape),
                                                     extents, ctypes.byref(pointer)))
        count = int(np.prod(shape)) if len(shape) else 1
        buffer = (ctypes.c_float * count).from_address(pointer.value) if count else []
        return np.array(np.frombuffer(buffer, dtype=np.float32, count=count)).reshape(shape)

    def bf16_data(self, name: str, shape):
        """The bfloat16 payload's bit patterns (uint16)."""
        import numpy as np

        extents = (ctypes.c_int64 * max(len(shape), 1))(*shape)
        pointer = ctypes.c_void_p()
        check(library().cuvit_weight_file_bf16_data(self._handle, name.encode(), len(shape),
                                                    extents, ctypes.byref(pointer)))
        count = int(np.prod(shape)) if len(shape) else 1
        buffer = (ctypes.c_uint16 * count).from_address(pointer.value) if count else []
        return np.array(np.frombuffer(buffer, dtype=np.uint16, count=count)).reshape(shape)

    @property
    def version(self) -> int:
        return library().cuvit_weight_file_version(self._handle)

    def dtype(self, name: str) -> int:
        """1 for float32, 2 for bfloat16, 0 when absent."""
        return library().cuvit_weight_file_type(self._handle, name.encode())

    def close(self) -> None:
        if getattr(self, "_handle", None):
            library().cuvit_weight_file_destroy(self._handle)
            self._handle = None

    def __del__(self):
        self.close()


def default_config() -> VitConfig:
    config = VitConfig()
    library().cuvit_vit_config_default(ctypes.byref(config))
    return config


def validate_config(config: VitConfig) -> None:
    check(library().cuvit_vit_config_validate(ctypes.byref(config)))


class VisionTransformer:
    """VisionTransformer (reference vit.hpp:53-120) over the C ABI."""

    def __init__(self, config: VitConfig, weights: WeightFile, max_batch: int = 1,
                 precision: int = 0):
        """precision: PRECISION_F32 (the reference's) or PRECISION_BF16 (an extension)."""
        handle = ctypes.c_void_p()
        check(library().cuvit_vit_create_ex(ctypes.byref(config), weights.handle, max_batch,
                                            precision, ctypes.byref(handle)))
        self._handle = handle
        self.config = config
        self.max_batch = max_batch

    @property
    def precision(self) -> int:
        return library().cuvit_vit_precision(self._handle)

    def forward(self, images, logits, batch: int, stream=None) -> None:
        c = self.config
        if _positive(batch):
            images = _operand(images, "images", "float32",
                              batch * c.channels * c.image_size * c.image_size)
            logits = _operand(logits, "logits", "float32", batch * c.classes)
        check(library().cuvit_vit_forward(self._handle, _ptr(images), _ptr(logits), batch,
                                          stream_handle(stream)))

    def weight_bytes(self) -> int:
        return library().cuvit_vit_weight_bytes(self._handle)

    def activation_bytes(self) -> int:
        return library().cuvit_vit_activation_bytes(self._handle)

    def close(self) -> None:
        if getattr(self, "_handle", None):
            library().cuvit_vit_destroy(self._handle)
            self._handle = None

    def __del__(self):
        self.close()


def expected_tensor_names(config: VitConfig):
    """VisionTransformer::expected_tensor_names (reference vit.cu:49-63), with shapes."""
    e, t, h = config.embed_dim, config.token_count(), config.mlp_hidden
    names = [("cls_token", (1, 1, e)), ("pos_embed", (1, t, e)),
             ("patch_embed.proj.weight", (e, config.channels, config.patch_size, config.patch_size)),
             ("patch_embed.proj.bias", (e,))]
    for i in range(config.depth):
        p = f"blocks.{i}."
        names += [(p + "norm1.weight", (e,)), (p + "norm1.bias", (e,)),
                  (p + "attn.qkv.weight", (3 * e, e)), (p + "attn.qkv.bias", (3 * e,)),
                  (p + "attn.proj.weight", (e, e)), (p + "attn.proj.bias", (e,)),
                  (p + "norm2.weight", (e,)), (p + "norm2.bias", (e,)),
                  (p + "mlp.fc1.weight", (h, e)), (p + "mlp.fc1.bias", (h,)),
                  (p + "mlp.fc2.weight", (e, h)), (p + "mlp.fc2.bias", (e,))]
    names += [("norm.weight", (e,)), ("norm.bias", (e,)),
              ("head.weight", (config.classes, e)), ("head.bias", (config.classes,))]
    return names


class RgbImage:
    """cuvit::RgbImage (reference image.hpp:12-19): .pixels is a uint8 numpy
    array of shape [height, width, 3], interleaved RGB."""

    def __init__(self, width: int, height: int, pixels):
        self.width = width
        self.height = height
        self.pixels = pixels

    def empty(self) -> bool:
        return self.pixels is None or self.pixels.size == 0


def load_ppm(path: str) -> RgbImage:
    """load_ppm (reference image.cpp:57-93) through the C ABI; a malformed or
    missing file raises CuvitError with the reference's message."""
    import numpy as np

    lib = library()
    handle = ctypes.c_void_p()
    check(lib.cuvit_image_load_ppm(os.fsencode(path), ctypes.byref(handle)))
    try:
        width, height = lib.cuvit_image_width(handle), lib.cuvit_image_height(handle)
        count = width * height * 3
        buffer = (ctypes.c_uint8 * count).from_address(lib.cuvit_image_pixels(handle))
        pixels = np.frombuffer(buffer, dtype=np.uint8).reshape(height, width, 3).copy()
    finally:
        lib.cuvit_image_destroy(handle)
    return RgbImage(width, height, pixels)


def preprocess(pixels, tensor, batch: int, width: int, height: int,
               settings: Optional[Preprocessing] = None, stream=None) -> None:
    """cuvit_preprocess_u8: @p batch device images [batch, height, width, 3]
    uint8 into the device tensor [batch, 3, size, size] float (the reference's
    preprocess, image.cpp:95-135, batched on the GPU)."""
    settings = settings if settings is not None else Preprocessing()
    if _positive(batch, width, height, settings.size):
        pixels = _operand(pixels, "pixels", "uint8", batch * height * width * 3)
        tensor = _operand(tensor, "tensor", "float32", batch * 3 * settings.size * settings.size)
    check(library().cuvit_preprocess_u8(_ptr(pixels), batch, width, height,
                                        ctypes.byref(settings), _ptr(tensor),
                                        stream_handle(stream)))


def preprocess_image(image: RgbImage, settings: Optional[Preprocessing] = None):
    """The reference's preprocess(image, settings) -> [3, size, size] numpy
    float32, computed on cuda:0 by the library's kernel."""
    import numpy as np
    import torch

    settings = settings if settings is not None else Preprocessing()
    if image.empty():
        raise InvalidArgument(ERROR_INVALID_ARGUMENT, "Cannot preprocess an empty image")
    device = torch.device("cuda:0")
    pixels = torch.from_numpy(np.ascontiguousarray(image.pixels, dtype=np.uint8)).to(device)
    size = settings.size
    tensor = torch.empty(3 * max(size, 0) * max(size, 0), dtype=torch.float32, device=device)
    preprocess(pixels, tensor, 1, image.width, image.height, settings)
    torch.cuda.synchronize()
    return tensor.cpu().numpy().reshape(3, size, size)


def cli_path() -> str:
    """The cu-vit command-line program built beside the library."""
    return os.path.join(os.path.dirname(_HERE), "bin", "cu-vit")
