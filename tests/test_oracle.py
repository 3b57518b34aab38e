"""CPU tests that pin the oracle before it is trusted as the checker.

Each oracle function is checked against something other than its own formula:
torch's SDPA (a library routine, as reference tests/test_reference.py:10-52 does),
an independent float64 row-wise evaluation, closed-form known answers, the committed
golden vectors, and planted-mistake mutants that the same checks must reject.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import (
    attention_float64_rowwise,
    attention_reference,
    attention_reference_fp32,
    attention_rows_fp32,
    flash_forward_tiled,
)

GOLDEN = Path(__file__).resolve().parent / "golden" / "attention_fp16_d64.npz"

# North-star gate for FP16 outputs against the FP32 reference.
KERNEL_ATOL = 2e-3
KERNEL_RTOL = 1e-2


def _randn(shape, seed=0, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=gen, dtype=torch.float32).to(dtype)


# --- reference semantics pinned by SDPA (mirrors reference tests/test_reference.py:10-52)

@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 1, 1, 16), (1, 2, 17, 32), (2, 4, 64, 64), (1, 8, 65, 128)])
def test_reference_matches_sdpa(shape, causal):
    torch.manual_seed(0)
    q, k, v = (torch.randn(shape) for _ in range(3))
    actual = attention_reference(q, k, v, causal=causal)
    expected = F.scaled_dot_product_attention(q, k, v, is_causal=causal)
    torch.testing.assert_close(actual, expected, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 2, 5, 8), (2, 1, 9, 16), (1, 1, 16, 64)])
def test_float64_rowwise_matches_sdpa_in_float64(shape, causal):
    q, k, v = (_randn(shape, seed=s, dtype=torch.float64) for s in range(3))
    expected = F.scaled_dot_product_attention(q, k, v, is_causal=causal).numpy()
    np.testing.assert_allclose(attention_float64_rowwise(q, k, v, causal=causal), expected,
                               rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_reference_matches_float64_rowwise_on_fp16_inputs(causal):
    q, k, v = (_randn((2, 2, 48, 64), seed=s, dtype=torch.float16) for s in range(3))
    actual = attention_reference_fp32(q, k, v, causal=causal).double().numpy()
    np.testing.assert_allclose(actual, attention_float64_rowwise(q, k, v, causal=causal),
                               rtol=1e-5, atol=1e-6)


def test_reference_supports_different_query_and_key_lengths():
    q = _randn((2, 4, 7, 32), 0)
    k = _randn((2, 4, 11, 32), 1)
    v = _randn((2, 4, 11, 32), 2)
    out = attention_reference(q, k, v)
    assert out.shape == (2, 4, 7, 32)
    np.testing.assert_allclose(out.double().numpy(), attention_float64_rowwise(q, k, v),
                               rtol=1e-5, atol=1e-6)


# --- closed-form known answers (reference tests/test_reference.py:67-103)

def test_custom_scale_known_answer():
    q, k, v = (_randn((1, 2, 8, 32), s) for s in range(3))
    logits = np.einsum("bhid,bhjd->bhij", q.double().numpy(), k.double().numpy()) * 0.25
    w = np.exp(logits - logits.max(-1, keepdims=True))
    expected = (w / w.sum(-1, keepdims=True)) @ v.double().numpy()
    np.testing.assert_allclose(attention_reference(q, k, v, scale=0.25).numpy(), expected,
                               rtol=1e-5, atol=1e-6)


def test_default_scale_is_inverse_sqrt_head_dim():
    q, k, v = (_randn((1, 1, 4, 64), s) for s in range(3))
    torch.testing.assert_close(attention_reference(q, k, v),
                               attention_reference(q, k, v, scale=1.0 / math.sqrt(64)))
    with pytest.raises(AssertionError):
        torch.testing.assert_close(attention_reference(q, k, v),
                                   attention_reference(q, k, v, scale=1.0))


def test_causal_first_row_is_first_value_row():
    q, k, v = (_randn((1, 3, 32, 64), s) for s in range(3))
    out = attention_reference_fp32(q, k, v, causal=True)
    torch.testing.assert_close(out[:, :, 0], v[:, :, 0], rtol=0, atol=1e-6)


def test_constant_value_gives_constant_output():
    q, k = _randn((1, 2, 40, 64), 0), _randn((1, 2, 40, 64), 1)
    v = torch.full((1, 2, 40, 64), 0.375)
    for causal in (False, True):
        out = attention_reference_fp32(q, k, v, causal=causal)
        torch.testing.assert_close(out, torch.full_like(out, 0.375), rtol=0, atol=1e-6)


def test_zero_query_gives_mean_of_visible_values():
    k, v = _randn((1, 1, 24, 64), 1), _randn((1, 1, 24, 64), 2)
    q = torch.zeros_like(k)
    torch.testing.assert_close(attention_reference_fp32(q, k, v), v.mean(dim=2, keepdim=True)
                               .expand_as(v), rtol=1e-6, atol=1e-6)
    prefix_mean = torch.cumsum(v, dim=2) / torch.arange(1, 25).view(1, 1, 24, 1)
    torch.testing.assert_close(attention_reference_fp32(q, k, v, causal=True), prefix_mean,
                               rtol=1e-5, atol=1e-6)


def test_noncausal_output_is_invariant_to_key_permutation():
    q, k, v = (_randn((1, 2, 30, 64), s) for s in range(3))
    perm = torch.randperm(30, generator=torch.Generator().manual_seed(7))
    torch.testing.assert_close(attention_reference_fp32(q, k, v),
                               attention_reference_fp32(q, k[:, :, perm], v[:, :, perm]),
                               rtol=1e-5, atol=1e-6)


def test_large_logits_stay_finite():
    q, k = _randn((1, 1, 512, 64), 0) * 2, _randn((1, 1, 512, 64), 1) * 2
    v = _randn((1, 1, 512, 64), 2)
    out = attention_reference(q.half(), k.half(), v.half(), causal=True)
    assert torch.isfinite(out).all()


# --- validation (reference tests/test_reference.py:106-120)

def test_rejects_invalid_rank():
    x = torch.randn(8, 64)
    with pytest.raises(ValueError, match="must have shape"):
        attention_reference(x, x, x)


def test_rejects_mismatched_key_value_lengths():
    q, k = torch.randn(1, 1, 8, 64), torch.randn(1, 1, 8, 64)
    with pytest.raises(ValueError, match="same sequence length"):
        attention_reference(q, k, torch.randn(1, 1, 7, 64))


def test_rejects_integer_inputs():
    x = torch.zeros(1, 1, 4, 64, dtype=torch.int32)
    with pytest.raises(TypeError, match="floating-point"):
        attention_reference(x, x, x)


# --- row-sampled and tiled variants

@pytest.mark.parametrize("causal", [False, True])
def test_rows_variant_equals_full_reference(causal):
    q, k, v = (_randn((2, 3, 96, 64), s, torch.float16) for s in range(3))
    rows = [(0, 0, 0), (1, 2, 95), (0, 1, 47), (1, 0, 64), (0, 2, 1)]
    full = attention_reference_fp32(q, k, v, causal=causal)
    expected = torch.stack([full[b, h, i] for b, h, i in rows])
    torch.testing.assert_close(attention_rows_fp32(q, k, v, rows, causal=causal), expected,
                               rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("causal", [False, True])
def test_tiled_model_without_rounding_matches_reference(causal):
    q, k, v = (_randn((1, 2, 256, 64), s, torch.float16) for s in range(3))
    tiled = flash_forward_tiled(q, k, v, causal=causal, block_n=256, round_p_to_fp16=False)
    torch.testing.assert_close(tiled, attention_reference(q, k, v, causal=causal), rtol=0, atol=1e-3)


@pytest.mark.parametrize("sigma", [1.0, 2.0])
@pytest.mark.parametrize("causal", [False, True])
def test_tiled_model_of_reference_kernel_within_kernel_tolerance(causal, sigma):
    q = (_randn((1, 2, 512, 64), 0) * sigma).half()
    k = (_randn((1, 2, 512, 64), 1) * sigma).half()
    v = _randn((1, 2, 512, 64), 2).half()
    tiled = flash_forward_tiled(q, k, v, causal=causal)
    expected = attention_reference_fp32(q, k, v, causal=causal)
    torch.testing.assert_close(tiled.float(), expected, rtol=KERNEL_RTOL, atol=KERNEL_ATOL)


# --- golden vectors

def _golden():
    with np.load(GOLDEN) as data:
        return {name: data[name] for name in data.files}


def test_golden_vectors_match_reference():
    data = _golden()
    cases = sorted({name.split("/")[0] for name in data})
    assert cases, "no golden cases"
    checked = 0
    for case in cases:
        q, k, v = (torch.from_numpy(data[f"{case}/{t}"]) for t in ("query", "key", "value"))
        assert q.dtype == torch.float16 and q.shape[-1] == 64
        for mode in ("noncausal", "causal"):
            name = f"{case}/{mode}"
            if name not in data:
                continue
            actual = attention_reference_fp32(q, k, v, causal=(mode == "causal")).numpy()
            np.testing.assert_allclose(actual, data[name], rtol=1e-5, atol=1e-5)
            checked += 1
    assert checked >= 5


# --- planted mistakes: each mutant of the oracle must fail the pinning checks above

def _mutant_no_scale(q, k, v, causal):
    logits = torch.matmul(q.float(), k.float().transpose(-2, -1))
    if causal:
        logits = logits.masked_fill(torch.triu(torch.ones(q.shape[2], k.shape[2], dtype=torch.bool), 1),
                                    float("-inf"))
    return torch.matmul(torch.softmax(logits, -1), v.float())


def _mutant_mask_includes_diagonal(q, k, v, causal):
    logits = torch.matmul(q.float(), k.float().transpose(-2, -1)) / 8.0
    if causal:
        mask = torch.triu(torch.ones(q.shape[2], k.shape[2], dtype=torch.bool), 0)
        mask[0, 0] = False  # keep row 0 defined
        logits = logits.masked_fill(mask, float("-inf"))
    return torch.matmul(torch.softmax(logits, -1), v.float())


def _mutant_softmax_over_queries(q, k, v, causal):
    logits = torch.matmul(q.float(), k.float().transpose(-2, -1)) / 8.0
    if causal:
        logits = logits.masked_fill(torch.triu(torch.ones(q.shape[2], k.shape[2], dtype=torch.bool), 1),
                                    float("-inf"))
    return torch.matmul(torch.softmax(logits, -2).nan_to_num(0.0), v.float())


def _mutant_value_transposed_per_head(q, k, v, causal):
    return attention_reference_fp32(q, k, v.transpose(-2, -1).reshape(v.shape), causal=causal)


@pytest.mark.parametrize("mutant", [_mutant_no_scale, _mutant_mask_includes_diagonal,
                                    _mutant_softmax_over_queries, _mutant_value_transposed_per_head])
def test_planted_mistakes_are_caught(mutant):
    data = _golden()
    q, k, v = (torch.from_numpy(data[f"b1h1n128/{t}"]) for t in ("query", "key", "value"))
    caught = 0
    for mode in ("noncausal", "causal"):
        out = mutant(q, k, v, mode == "causal").numpy()
        if not np.allclose(out, data[f"b1h1n128/{mode}"], rtol=1e-5, atol=1e-5):
            caught += 1
    assert caught >= 1, f"{mutant.__name__} passed the golden check"
