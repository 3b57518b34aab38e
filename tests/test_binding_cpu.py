"""CPU tests of the torch operator module `flash_attention_cuda`: import surface and the
validation text of reference csrc/tensorcore_attention.cu:2731-2823 and 3025-3038."""

from __future__ import annotations

import pytest
import torch

import flash_attention_2_lab_amd  # noqa: F401  (registers flash_attention_cuda)
import flash_attention_cuda

ENTRY = flash_attention_cuda.tensorcore_attention_forward_production_128x128
CHECK = flash_attention_cuda._check_production_inputs


def _half(shape=(1, 2, 128, 64)):
    return torch.zeros(shape, dtype=torch.float16)


def test_module_exposes_reference_entry_point():
    assert flash_attention_cuda.__name__.split(".")[-1] == "flash_attention_cuda"
    assert callable(ENTRY)
    assert flash_attention_2_lab_amd.tensorcore_attention_forward_production_128x128 is ENTRY


@pytest.mark.parametrize("bad, message", [(0, "query must be a CUDA tensor"),
                                          (1, "key must be a CUDA tensor"),
                                          (2, "value must be a CUDA tensor")])
def test_cpu_tensors_are_rejected_in_reference_order(bad, message):
    # The device check runs first; on CPU every argument fails it, so only q is
    # reported. Exercise k and v through the testing hook with q as the device probe.
    tensors = [_half(), _half(), _half()]
    if bad == 0:
        with pytest.raises(RuntimeError, match=message):
            ENTRY(*tensors, False)
    else:
        with pytest.raises(RuntimeError, match="query must be a CUDA tensor"):
            CHECK(*tensors, True)


@pytest.mark.parametrize("mutate, message", [
    (lambda q, k, v: (q.float(), k, v), "query must have dtype torch.float16"),
    (lambda q, k, v: (q, k.float(), v), "key must have dtype torch.float16"),
    (lambda q, k, v: (q, k, v.bfloat16()), "value must have dtype torch.float16"),
    (lambda q, k, v: (q[0], k, v), r"query must have shape \[B, H, N, D\]"),
    (lambda q, k, v: (q, k[0], v), r"key must have shape \[B, H, N, D\]"),
    (lambda q, k, v: (q, k, v[0]), r"value must have shape \[B, H, N, D\]"),
    (lambda q, k, v: (q, k[:, :1], v), "query and key must have identical shapes"),
    (lambda q, k, v: (q, k, v[:, :1]), "query and value must have identical shapes"),
    (lambda q, k, v: (q.transpose(1, 2).contiguous().transpose(1, 2), k, v), "query must be contiguous"),
    (lambda q, k, v: (q, k.transpose(1, 2).contiguous().transpose(1, 2), v), "key must be contiguous"),
    (lambda q, k, v: (q, k, v.transpose(1, 2).contiguous().transpose(1, 2)), "value must be contiguous"),
])
def test_validation_messages(mutate, message):
    q, k, v = mutate(_half(), _half(), _half())
    with pytest.raises(RuntimeError, match=message):
        CHECK(q, k, v, False)


def test_head_dimension_must_be_64():
    x = _half((1, 1, 128, 32))
    with pytest.raises(RuntimeError, match="head dimension must equal 64"):
        CHECK(x, x, x, False)


@pytest.mark.parametrize("seq_len", [64, 96, 130, 1000])
def test_sequence_length_must_divide_by_128(seq_len):
    x = _half((1, 1, seq_len, 64))
    with pytest.raises(RuntimeError, match="sequence length must be divisible by 128"):
        CHECK(x, x, x, False)


def test_reference_grid_limit_on_batch_times_heads():
    x = torch.empty((65536, 1, 128, 64), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="batch \\* heads exceeds CUDA grid.y limit"):
        CHECK(x, x, x, False)


def test_valid_inputs_pass_validation():
    CHECK(_half(), _half(), _half(), False)
    CHECK(_half((0, 2, 128, 64)), _half((0, 2, 128, 64)), _half((0, 2, 128, 64)), False)


TENSORCORE_ENTRIES = {
    "tensorcore_attention_forward": 16,
    "tensorcore_attention_forward_bc32": 32,
    "tensorcore_attention_forward_bc32_raw_pv": 32,
    "tensorcore_attention_forward_bc32_raw_qk_raw_pv": 32,
}


@pytest.mark.parametrize("name", sorted(TENSORCORE_ENTRIES))
def test_module_exposes_the_bc16_bc32_entry_points(name):
    # Reference csrc/bindings.cpp:113-134: three positional tensors, noncausal.
    entry = getattr(flash_attention_cuda, name)
    with pytest.raises(RuntimeError, match="query must be a CUDA tensor"):
        entry(_half((1, 1, 32, 64)), _half((1, 1, 32, 64)), _half((1, 1, 32, 64)))


@pytest.mark.parametrize("key_tile, seq_len", [(16, 8), (16, 40), (32, 48), (32, 80), (32, 1040)])
def test_tensorcore_entries_require_a_multiple_of_their_key_tile(key_tile, seq_len):
    # Reference csrc/tensorcore_attention.cu:2818-2822 and tests/test_tensorcore_attention.py:155-179.
    x = _half((1, 1, seq_len, 64))
    with pytest.raises(RuntimeError, match=f"sequence length must be divisible by {key_tile}"):
        flash_attention_cuda._check_tensorcore_inputs(x, x, x, key_tile, False)


@pytest.mark.parametrize("key_tile, seq_len", [(16, 16), (16, 80), (32, 96), (32, 512)])
def test_tensorcore_entries_accept_partial_128_tiles(key_tile, seq_len):
    x = _half((1, 1, seq_len, 64))
    flash_attention_cuda._check_tensorcore_inputs(x, x, x, key_tile, False)


def test_tensorcore_entries_share_the_reference_checks():
    with pytest.raises(RuntimeError, match="head dimension must equal 64"):
        x = _half((1, 1, 32, 16))
        flash_attention_cuda._check_tensorcore_inputs(x, x, x, 16, False)
    with pytest.raises(RuntimeError, match="query and key must have identical shapes"):
        flash_attention_cuda._check_tensorcore_inputs(_half((1, 2, 32, 64)), _half((1, 1, 32, 64)),
                                                      _half((1, 2, 32, 64)), 32, False)
    x = torch.empty((65536, 1, 32, 64), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="batch \\* heads exceeds CUDA grid.y limit"):
        flash_attention_cuda._check_tensorcore_inputs(x, x, x, 32, False)
