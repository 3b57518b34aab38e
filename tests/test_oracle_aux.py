"""Pins of the oracle functions for the module's other operators (CPU only).

attention_scores_fp32 and matmul_16x64x16_fp32 are checked against float64 loops
written out element by element and against closed-form known answers, including
planted mistakes that the checks must reject. The FP32 attention oracle used for the
FP32 SIMT forwards is pinned at head dimension 128 too (the reference's naive and
block forwards accept 64 and 128).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import (
    attention_float64_rowwise,
    attention_reference_fp32,
    attention_scores_fp32,
    matmul_16x64x16_fp32,
)


def _scores_loop_float64(query: np.ndarray, key: np.ndarray) -> np.ndarray:
    b, h, n, d = query.shape
    out = np.zeros((b, h, n, n))
    for bi in range(b):
        for hi in range(h):
            for i in range(n):
                for j in range(n):
                    acc = 0.0
                    for k in range(d):
                        acc += float(query[bi, hi, i, k]) * float(key[bi, hi, j, k])
                    out[bi, hi, i, j] = acc / math.sqrt(d)
    return out


@pytest.mark.parametrize("shape", [(1, 1, 1, 16), (1, 2, 5, 8), (2, 1, 7, 4)])
def test_scores_match_float64_loop(shape):
    gen = torch.Generator().manual_seed(1)
    q = torch.randn(shape, generator=gen)
    k = torch.randn(shape, generator=gen)
    expected = _scores_loop_float64(q.double().numpy(), k.double().numpy())
    np.testing.assert_allclose(attention_scores_fp32(q, k).double().numpy(), expected, rtol=1e-5, atol=1e-6)


def test_scores_constant_known_answer():
    # Reference tests/test_naive_scores.py:71-107: each (batch, head) pair filled with
    # its own constants gives D * cq * ck / sqrt(D) in every score of that pair.
    q = torch.zeros(2, 2, 3, 4)
    k = torch.zeros_like(q)
    for (b, h), (cq, ck) in {(0, 0): (1.0, 5.0), (0, 1): (2.0, 6.0), (1, 0): (3.0, 7.0), (1, 1): (4.0, 8.0)}.items():
        q[b, h].fill_(cq)
        k[b, h].fill_(ck)
        scores = attention_scores_fp32(q, k)
        assert torch.all(scores[b, h] == 4 * cq * ck / 2.0)


def test_scores_custom_scale_and_shape():
    q = torch.randn(1, 3, 6, 32)
    k = torch.randn(1, 3, 6, 32)
    s = attention_scores_fp32(q, k, scale=0.5)
    assert s.shape == (1, 3, 6, 6) and s.dtype == torch.float32
    torch.testing.assert_close(s, (q @ k.transpose(-2, -1)) * 0.5)


@pytest.mark.parametrize("mutant", ["no_scale", "k_times_q", "sqrt_n"])
def test_scores_planted_mistakes_are_caught(mutant):
    gen = torch.Generator().manual_seed(2)
    q = torch.randn(1, 2, 5, 8, generator=gen)
    k = torch.randn(1, 2, 5, 8, generator=gen)
    if mutant == "no_scale":
        wrong = q @ k.transpose(-2, -1)
    elif mutant == "k_times_q":
        wrong = (k @ q.transpose(-2, -1)) / math.sqrt(8)
    else:
        wrong = (q @ k.transpose(-2, -1)) / math.sqrt(5)
    expected = _scores_loop_float64(q.double().numpy(), k.double().numpy())
    assert not np.allclose(wrong.double().numpy(), expected, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(attention_scores_fp32(q, k).double().numpy(), expected, rtol=1e-5, atol=1e-6)


def _matmul_loop_float64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    out = np.zeros((a.shape[0], 16, 16))
    for m in range(a.shape[0]):
        for i in range(16):
            for j in range(16):
                out[m, i, j] = sum(float(a[m, i, k]) * float(b[m, k, j]) for k in range(64))
    return out


def test_matmul_matches_float64_loop():
    gen = torch.Generator().manual_seed(3)
    a = torch.randn(3, 16, 64, generator=gen).half()
    b = torch.randn(3, 64, 16, generator=gen).half()
    expected = _matmul_loop_float64(a.double().numpy(), b.double().numpy())
    np.testing.assert_allclose(matmul_16x64x16_fp32(a, b).double().numpy(), expected, rtol=1e-5, atol=1e-5)


def test_matmul_identity_block_known_answer():
    # Reference tests/test_wmma_matmul.py:13-75: B = [I; 0] selects A[:, :, :16].
    a = torch.randn(4, 16, 64).half()
    b = torch.zeros(4, 64, 16).half()
    b[:, :16, :] = torch.eye(16).half()
    assert torch.equal(matmul_16x64x16_fp32(a, b), a[:, :, :16].float())


def test_matmul_planted_transpose_is_caught():
    gen = torch.Generator().manual_seed(4)
    a = torch.randn(1, 16, 64, generator=gen).half()
    b = torch.randn(1, 64, 16, generator=gen).half()
    expected = _matmul_loop_float64(a.double().numpy(), b.double().numpy())
    wrong = (a.float() @ b.float()).transpose(1, 2)
    assert not np.allclose(wrong.double().numpy(), expected, rtol=1e-3, atol=1e-3)


def test_matmul_rejects_wrong_shapes():
    with pytest.raises(ValueError, match=r"\[batch, 16, 64\]"):
        matmul_16x64x16_fp32(torch.zeros(1, 16, 32).half(), torch.zeros(1, 64, 16).half())
    with pytest.raises(ValueError, match=r"\[batch, 64, 16\]"):
        matmul_16x64x16_fp32(torch.zeros(1, 16, 64).half(), torch.zeros(1, 64, 8).half())


@pytest.mark.parametrize("seq_len", [1, 17, 33])
def test_fp32_reference_at_head_dim_128(seq_len):
    # The FP32 SIMT forwards accept D = 128 (reference csrc/naive_attention.cu:299-315,
    # 474-490); the oracle agrees with SDPA and with the float64 row-wise evaluation there.
    gen = torch.Generator().manual_seed(seq_len)
    q, k, v = (torch.randn(1, 2, seq_len, 128, generator=gen) for _ in range(3))
    out = attention_reference_fp32(q, k, v)
    torch.testing.assert_close(out, F.scaled_dot_product_attention(q, k, v), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(out.double().numpy(), attention_float64_rowwise(q, k, v), rtol=1e-5, atol=1e-6)
