"""ctypes binding of the C ABI declared in ``include/fa2_mi355x.h``.

This is the binding a Python caller without the torch extension would write; the
tests use it to exercise the C ABI directly. Tensors are passed as device pointers
plus sizes, and the kernel is enqueued on the given HIP stream (default: torch's
current stream on the tensors' device).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import torch

PACKAGE_DIR = Path(__file__).resolve().parent
LIBRARY_PATH = PACKAGE_DIR / "libfa2_mi355x.so"
HEADER_PATH = PACKAGE_DIR.parent / "include" / "fa2_mi355x.h"

FA2_STATUS_SUCCESS = 0
FA2_STATUS_NULL_POINTER = 1
FA2_STATUS_NEGATIVE_DIMENSION = 2
FA2_STATUS_BAD_HEAD_DIM = 3
FA2_STATUS_BAD_SEQUENCE_LENGTH = 4
FA2_STATUS_MISALIGNED = 5
FA2_STATUS_TOO_LARGE = 6
FA2_STATUS_BAD_KEY_TILE = 7
FA2_STATUS_BAD_KERNEL = 8
FA2_STATUS_HIP_ERROR_BASE = 1000

# Kernels of the FP16 forward entries (fa2_forward_plan).
FA2_KERNEL_NONE = 0
FA2_KERNEL_256_QUERY = 1
FA2_KERNEL_256_QUERY_PAIRS = 2
FA2_KERNEL_128_QUERY = 3
FA2_KERNEL_KEY_SPLIT_64 = 4
FA2_KERNEL_KEY_SPLIT_32 = 5
FA2_KERNEL_KEY_SPLIT_8_WAVES = 6
FA2_KERNEL_KEY_SPLIT_PAIRS16 = 7
FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES = 8
FA2_KERNEL_128_QUERY_SPLIT_PAIRS = 9


class Fa2Error(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, function: str, status: int, message: str) -> None:
        super().__init__(f"{function} failed with status {status}: {message}")
        self.status = status


def _load() -> ctypes.CDLL:
    if not LIBRARY_PATH.exists():
        raise ImportError(
            f"{LIBRARY_PATH} is missing (run `python flash_attention_2_lab_amd/_build.py`)"
        )
    lib = ctypes.CDLL(str(LIBRARY_PATH))
    lib.fa2_forward_production_128x128.argtypes = [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_int, ctypes.c_void_p,
    ]
    lib.fa2_forward_production_128x128.restype = ctypes.c_int
    lib.fa2_forward_tensorcore.argtypes = [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_int64, ctypes.c_void_p,
    ]
    lib.fa2_forward_tensorcore.restype = ctypes.c_int
    lib.fa2_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    lib.fa2_copy.restype = ctypes.c_int
    lib.fa2_attention_scores_f32.argtypes = [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
    ]
    lib.fa2_attention_scores_f32.restype = ctypes.c_int
    lib.fa2_attention_forward_f32.argtypes = [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
    ]
    lib.fa2_attention_forward_f32.restype = ctypes.c_int
    lib.fa2_matmul_16x64x16_f16.argtypes = [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
    ]
    lib.fa2_matmul_16x64x16_f16.restype = ctypes.c_int
    lib.fa2_status_string.argtypes = [ctypes.c_int]
    lib.fa2_status_string.restype = ctypes.c_char_p
    lib.fa2_abi_version.argtypes = []
    lib.fa2_abi_version.restype = ctypes.c_int
    lib.fa2_forward_plan.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int]
    lib.fa2_forward_plan.restype = ctypes.c_int
    lib.fa2_forward_with_kernel.argtypes = [
        ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_int, ctypes.c_void_p,
    ]
    lib.fa2_forward_with_kernel.restype = ctypes.c_int
    return lib


lib = _load()


def declared_functions() -> list[str]:
    """Names of the functions declared in include/fa2_mi355x.h."""
    text = HEADER_PATH.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(fa2_\w+)\s*\(", text, flags=re.M)


def status_string(status: int) -> str:
    return lib.fa2_status_string(status).decode()


def abi_version() -> int:
    return lib.fa2_abi_version()


def forward_plan(batch: int, heads: int, seq_len: int, causal: bool) -> int:
    """FA2_KERNEL_* the FP16 forward entries launch for these sizes (no GPU work)."""
    return lib.fa2_forward_plan(batch, heads, seq_len, int(causal))


def forward_production_128x128_raw(query_ptr: int, key_ptr: int, value_ptr: int,
                                   output_ptr: int, batch: int, heads: int, seq_len: int,
                                   head_dim: int, causal: bool, stream: int | None) -> int:
    """Direct call of the C entry point; returns the status code."""
    return lib.fa2_forward_production_128x128(
        query_ptr, key_ptr, value_ptr, output_ptr, batch, heads, seq_len, head_dim,
        1 if causal else 0, stream,
    )


def forward_production_128x128(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                               causal: bool, *, output: torch.Tensor | None = None,
                               stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Attention forward through the C ABI on torch tensors (no validation beyond the ABI's)."""
    if output is None:
        output = torch.empty_like(query)
    if stream is None:
        stream = torch.cuda.current_stream(query.device)
    batch, heads, seq_len, head_dim = query.shape
    status = forward_production_128x128_raw(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), output.data_ptr(),
        batch, heads, seq_len, head_dim, causal, stream.cuda_stream,
    )
    if status != FA2_STATUS_SUCCESS:
        raise Fa2Error("fa2_forward_production_128x128", status, status_string(status))
    return output


def forward_with_kernel_raw(kernel: int, query_ptr: int, key_ptr: int, value_ptr: int,
                            output_ptr: int, batch: int, heads: int, seq_len: int, head_dim: int,
                            causal: bool, stream: int | None) -> int:
    """Direct call of fa2_forward_with_kernel; returns the status code."""
    return lib.fa2_forward_with_kernel(
        kernel, query_ptr, key_ptr, value_ptr, output_ptr, batch, heads, seq_len, head_dim,
        1 if causal else 0, stream,
    )


def forward_with_kernel(kernel: int, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                        causal: bool, *, output: torch.Tensor | None = None,
                        stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """The production forward on a chosen FA2_KERNEL_* (Fa2Error with status
    FA2_STATUS_BAD_KERNEL when that kernel does not compute these sizes)."""
    if output is None:
        output = torch.empty_like(query)
    if stream is None:
        stream = torch.cuda.current_stream(query.device)
    batch, heads, seq_len, head_dim = query.shape
    status = forward_with_kernel_raw(
        kernel, query.data_ptr(), key.data_ptr(), value.data_ptr(), output.data_ptr(),
        batch, heads, seq_len, head_dim, causal, stream.cuda_stream,
    )
    if status != FA2_STATUS_SUCCESS:
        raise Fa2Error("fa2_forward_with_kernel", status, status_string(status))
    return output


def forward_tensorcore_raw(query_ptr: int, key_ptr: int, value_ptr: int, output_ptr: int,
                           batch: int, heads: int, seq_len: int, head_dim: int, key_tile: int,
                           stream: int | None) -> int:
    """Direct call of the noncausal C entry point; returns the status code."""
    return lib.fa2_forward_tensorcore(
        query_ptr, key_ptr, value_ptr, output_ptr, batch, heads, seq_len, head_dim, key_tile,
        stream,
    )


def forward_tensorcore(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                       key_tile: int = 16, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Allocate the output and run the noncausal entry (seq_len % key_tile == 0)."""
    if query.dim() != 4:
        raise ValueError("query must have shape [B, H, N, D]")
    output = torch.empty_like(query)
    if stream is None:
        stream = torch.cuda.current_stream(query.device)
    batch, heads, seq_len, head_dim = query.shape
    status = forward_tensorcore_raw(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), output.data_ptr(),
        batch, heads, seq_len, head_dim, key_tile, stream.cuda_stream,
    )
    if status != FA2_STATUS_SUCCESS:
        raise Fa2Error("fa2_forward_tensorcore", status, status_string(status))
    return output


def _stream_handle(tensor: torch.Tensor, stream: torch.cuda.Stream | None) -> int:
    return (stream or torch.cuda.current_stream(tensor.device)).cuda_stream


def _check(function: str, status: int) -> None:
    if status != FA2_STATUS_SUCCESS:
        raise Fa2Error(function, status, status_string(status))


def copy(source: torch.Tensor, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Copy of a contiguous device tensor through fa2_copy."""
    output = torch.empty_like(source)
    _check("fa2_copy", lib.fa2_copy(source.data_ptr(), output.data_ptr(),
                                    source.numel() * source.element_size(),
                                    _stream_handle(source, stream)))
    return output


def attention_scores_f32(query: torch.Tensor, key: torch.Tensor,
                         stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """FP32 scores Q K^T / sqrt(D), [B, H, N, N], through fa2_attention_scores_f32."""
    batch, heads, seq_len, head_dim = query.shape
    scores = torch.empty((batch, heads, seq_len, seq_len), dtype=torch.float32, device=query.device)
    _check("fa2_attention_scores_f32",
           lib.fa2_attention_scores_f32(query.data_ptr(), key.data_ptr(), scores.data_ptr(),
                                        batch * heads, seq_len, head_dim,
                                        _stream_handle(query, stream)))
    return scores


def attention_forward_f32(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                          stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """FP32 noncausal attention through fa2_attention_forward_f32."""
    batch, heads, seq_len, head_dim = query.shape
    output = torch.empty_like(query)
    _check("fa2_attention_forward_f32",
           lib.fa2_attention_forward_f32(query.data_ptr(), key.data_ptr(), value.data_ptr(),
                                         output.data_ptr(), batch * heads, seq_len, head_dim,
                                         _stream_handle(query, stream)))
    return output


def matmul_16x64x16(a: torch.Tensor, b: torch.Tensor,
                    stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """[batch, 16, 64] x [batch, 64, 16] FP16 -> [batch, 16, 16] FP32 through fa2_matmul_16x64x16_f16."""
    batch = a.shape[0]
    c = torch.empty((batch, 16, 16), dtype=torch.float32, device=a.device)
    _check("fa2_matmul_16x64x16_f16",
           lib.fa2_matmul_16x64x16_f16(a.data_ptr(), b.data_ptr(), c.data_ptr(), batch,
                                       _stream_handle(a, stream)))
    return c
