"""CPU tests of the module's other operators: their presence, the reference's
validation order and text (checked through the `_check_op_inputs` hook with the
device checks skipped), the CPU-tensor rejection each raises first, and the C ABI
status codes of their entry points (no GPU work).

References: csrc/bindings.cpp:71-111; csrc/copy_kernel.cu:23-53;
csrc/naive_attention.cu:203-502; csrc/tiled_attention.cu:220-333;
csrc/tilewise_attention.cu:285-388; csrc/wmma_matmul.cu:195-315.
"""

from __future__ import annotations

import pytest
import torch

import flash_attention_2_lab_amd  # noqa: F401  (registers flash_attention_cuda)
import flash_attention_cuda
from flash_attention_2_lab_amd import capi

CHECK = flash_attention_cuda._check_op_inputs
OPS_QKV = ["naive_attention_forward", "block_attention_forward", "tiled_attention_forward",
           "tilewise_attention_forward"]


def _f32(shape=(1, 2, 17, 64)):
    return torch.zeros(shape, dtype=torch.float32)


def test_module_exposes_every_reference_operator():
    for name in ["copy_cuda", "naive_attention_forward", "naive_attention_scores",
                 "block_attention_forward", "tiled_attention_forward", "tilewise_attention_forward",
                 "wmma_matmul_16x64x16", "tensorcore_attention_forward",
                 "tensorcore_attention_forward_bc32", "tensorcore_attention_forward_bc32_raw_pv",
                 "tensorcore_attention_forward_bc32_raw_qk_raw_pv",
                 "tensorcore_attention_forward_production_128x128"]:
        assert callable(getattr(flash_attention_cuda, name)), name


@pytest.mark.parametrize("call, message", [
    (lambda m: m.copy_cuda(torch.zeros(8)), "input must be a CUDA tensor"),
    (lambda m: m.naive_attention_forward(_f32(), _f32(), _f32()), "query must be a CUDA tensor"),
    (lambda m: m.block_attention_forward(_f32(), _f32(), _f32()), "query must be a CUDA tensor"),
    (lambda m: m.naive_attention_scores(_f32(), _f32()), "query must be a CUDA tensor"),
    (lambda m: m.tiled_attention_forward(_f32(), _f32(), _f32()), "query, key, and value must be CUDA tensors"),
    (lambda m: m.tilewise_attention_forward(_f32(), _f32(), _f32()), "query, key, and value must be CUDA tensors"),
    (lambda m: m.wmma_matmul_16x64x16(torch.zeros(1, 16, 64).half(), torch.zeros(1, 64, 16).half()),
     "A and B must be CUDA tensors"),
])
def test_cpu_tensors_are_rejected_first(call, message):
    # Reference tests/test_extension.py:38-44 for copy_cuda; the others check the
    # device first as well.
    with pytest.raises(RuntimeError, match=message):
        call(flash_attention_cuda)


def _noncontig(t):
    return t.transpose(1, 2).contiguous().transpose(1, 2)


@pytest.mark.parametrize("op", ["naive_attention_forward", "block_attention_forward"])
@pytest.mark.parametrize("mutate, message", [
    (lambda q, k, v: (_noncontig(q), k, v), "query must be contiguous"),
    (lambda q, k, v: (q, _noncontig(k), v), "key must be contiguous"),
    (lambda q, k, v: (q, k, _noncontig(v)), "value must be contiguous"),
    (lambda q, k, v: (q[0], k, v), "query must be rank 4"),
    (lambda q, k, v: (q, k[0], v), "key must be rank 4"),
    (lambda q, k, v: (q, k, v[0]), "value must be rank 4"),
    (lambda q, k, v: (q.double(), k, v), "query must use float32"),
    (lambda q, k, v: (q, k.half(), v), "key must use float32"),
    (lambda q, k, v: (q, k, v.double()), "value must use float32"),
    (lambda q, k, v: (q, k[:, :1].contiguous(), v), "the initial naive kernel requires query, key, and value to have identical shapes"),
])
def test_naive_and_block_validation(op, mutate, message):
    with pytest.raises(RuntimeError, match=message):
        CHECK(op, list(mutate(_f32(), _f32(), _f32())), False)


@pytest.mark.parametrize("op", ["naive_attention_forward", "block_attention_forward"])
def test_naive_and_block_head_dimension(op):
    # Reference csrc/naive_attention.cu:317-322 and 492-497; tests/test_naive_attention.py:84-94.
    with pytest.raises(RuntimeError, match="64 and 128"):
        CHECK(op, [_f32((1, 1, 8, 32))] * 3, False)
    with pytest.raises(RuntimeError, match=f"{op} currently supports head dimensions 64 and 128"):
        CHECK(op, [_f32((1, 1, 8, 96))] * 3, False)
    CHECK(op, [_f32((1, 1, 8, 64))] * 3, False)
    CHECK(op, [_f32((1, 1, 8, 128))] * 3, False)


def test_empty_problems_skip_the_head_dimension_check():
    # naive returns before its head-dimension switch when rows or D is zero; block
    # only when rows is zero (csrc/naive_attention.cu:266-270, 444-449).
    CHECK("naive_attention_forward", [_f32((1, 1, 0, 32))] * 3, False)
    CHECK("naive_attention_forward", [_f32((1, 1, 4, 0))] * 3, False)
    CHECK("block_attention_forward", [_f32((1, 1, 0, 32))] * 3, False)
    with pytest.raises(RuntimeError, match="64 and 128"):
        CHECK("block_attention_forward", [_f32((1, 1, 4, 0))] * 3, False)


@pytest.mark.parametrize("mutate, message", [
    (lambda q, k: (_noncontig(q), k), "query must be contiguous"),
    (lambda q, k: (q, _noncontig(k)), "key must be contiguous"),
    (lambda q, k: (q[0], k), "query must be rank 4"),
    (lambda q, k: (q, k[0]), "key must be rank 4"),
    (lambda q, k: (q.half(), k), "query must use float32"),
    (lambda q, k: (q, k.double()), "key must use float32"),
    (lambda q, k: (q, k[:, :1].contiguous()), "the initial score kernel requires query and key to have identical shapes"),
])
def test_score_validation(mutate, message):
    with pytest.raises(RuntimeError, match=message):
        CHECK("naive_attention_scores", list(mutate(_f32((1, 2, 8, 32)), _f32((1, 2, 8, 32)))), False)


@pytest.mark.parametrize("op, dtype_text, shape_text, dim_text", [
    ("tiled_attention_forward", "the initial tiled kernel requires float32 inputs",
     "the initial tiled kernel requires identical Q, K, and V shapes",
     "the initial tiled kernel supports head dimension 64"),
    ("tilewise_attention_forward", "tilewise attention currently requires float32",
     "tilewise attention currently requires identical Q, K, and V shapes",
     "tilewise attention currently supports head dimension 64"),
])
def test_tiled_and_tilewise_validation(op, dtype_text, shape_text, dim_text):
    q = _f32()
    cases = [
        ([_noncontig(q), q, q], "query, key, and value must be contiguous"),
        ([q, q, q[0]], "query, key, and value must be rank 4"),
        ([q, q.double(), q], dtype_text),
        ([q, q, q[:, :1].contiguous()], shape_text),
        ([_f32((1, 2, 17, 128))] * 3, dim_text),
    ]
    for tensors, message in cases:
        with pytest.raises(RuntimeError, match=message):
            CHECK(op, tensors, False)
    CHECK(op, [q, q, q], False)


@pytest.mark.parametrize("op, message", [
    ("tiled_attention_forward", "batch x heads exceeds CUDA grid.y limit"),
    ("tilewise_attention_forward", r"batch \* num_heads exceeds CUDA grid.y limit"),
])
def test_tiled_grid_limit(op, message):
    # An expanded (stride-0) view is not contiguous, so use a real 65536-head tensor
    # of one query each: 65536 * 64 floats.
    big = torch.zeros((1, 65536, 1, 64), dtype=torch.float32)
    with pytest.raises(RuntimeError, match=message):
        CHECK(op, [big, big, big], False)


@pytest.mark.parametrize("a, b, message", [
    (torch.zeros(1, 16, 64).half().transpose(1, 2).contiguous().transpose(1, 2),
     torch.zeros(1, 64, 16).half(), "A and B must be contiguous"),
    (torch.zeros(1, 16, 64), torch.zeros(1, 64, 16).half(), "A and B must use float16"),
    (torch.zeros(16, 64).half(), torch.zeros(1, 64, 16).half(), "A and B must be rank-3 tensors"),
    (torch.zeros(2, 16, 64).half(), torch.zeros(1, 64, 16).half(), "A and B must have the same batch size"),
    (torch.zeros(1, 16, 32).half(), torch.zeros(1, 64, 16).half(), r"A must have shape \[batch, 16, 64\]"),
    (torch.zeros(1, 16, 64).half(), torch.zeros(1, 64, 32).half(), r"B must have shape \[batch, 64, 16\]"),
])
def test_matmul_validation(a, b, message):
    with pytest.raises(RuntimeError, match=message):
        CHECK("wmma_matmul_16x64x16", [a, b], False)


def test_unknown_operator_hook_message():
    with pytest.raises(RuntimeError, match="no validation hook for copy_cuda"):
        CHECK("copy_cuda", [torch.zeros(1)], False)


# C ABI status codes (nothing is launched).

def test_copy_status_codes():
    assert capi.lib.fa2_copy(None, None, 0, None) == capi.FA2_STATUS_SUCCESS
    assert capi.lib.fa2_copy(None, None, -1, None) == capi.FA2_STATUS_NEGATIVE_DIMENSION
    assert capi.lib.fa2_copy(None, 4096, 16, None) == capi.FA2_STATUS_NULL_POINTER


@pytest.mark.parametrize("head_dim, status", [(64, capi.FA2_STATUS_NULL_POINTER),
                                              (128, capi.FA2_STATUS_NULL_POINTER),
                                              (32, capi.FA2_STATUS_BAD_HEAD_DIM),
                                              (0, capi.FA2_STATUS_BAD_HEAD_DIM)])
def test_f32_forward_status_codes(head_dim, status):
    assert capi.lib.fa2_attention_forward_f32(None, None, None, None, 2, 17, head_dim, None) == status


def test_f32_forward_and_scores_empty_and_negative():
    f, s = capi.lib.fa2_attention_forward_f32, capi.lib.fa2_attention_scores_f32
    assert f(None, None, None, None, 0, 17, 64, None) == capi.FA2_STATUS_SUCCESS
    assert f(None, None, None, None, 3, 0, 64, None) == capi.FA2_STATUS_SUCCESS
    assert f(None, None, None, None, -1, 17, 64, None) == capi.FA2_STATUS_NEGATIVE_DIMENSION
    assert s(None, None, None, 0, 17, 32, None) == capi.FA2_STATUS_SUCCESS
    assert s(None, None, None, 2, -3, 32, None) == capi.FA2_STATUS_NEGATIVE_DIMENSION
    assert s(None, None, None, 2, 9, 32, None) == capi.FA2_STATUS_NULL_POINTER
    assert s(4096, 4098, 4096, 2, 9, 32, None) == capi.FA2_STATUS_MISALIGNED
    assert f(4096, 4096, 4096, 4097, 2, 9, 64, None) == capi.FA2_STATUS_MISALIGNED


def test_matmul_status_codes():
    m = capi.lib.fa2_matmul_16x64x16_f16
    assert m(None, None, None, 0, None) == capi.FA2_STATUS_SUCCESS
    assert m(None, None, None, -2, None) == capi.FA2_STATUS_NEGATIVE_DIMENSION
    assert m(None, 4096, 4096, 3, None) == capi.FA2_STATUS_NULL_POINTER
    assert m(4097, 4096, 4096, 3, None) == capi.FA2_STATUS_MISALIGNED
    assert m(4096, 4096, 4096, 1 << 33, None) == capi.FA2_STATUS_TOO_LARGE
