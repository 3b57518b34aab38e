"""NaN and infinite inputs on the GPU: the output rows they make non-finite, against the oracle.

The reference's FP32 formula (flash_attention/reference.py:46-59) propagates a NaN in
Q, K or V through the scores, the softmax and P.V. The kernels are compiled with
-fno-honor-nans (their running max uses v_max_f32, which returns the non-NaN operand),
and they follow the formula for every output row that sees the NaN:
* a NaN in query row i makes row i NaN (every dimension) and leaves the others as the
  oracle computes them;
* a NaN in key row j makes every row that sees key j NaN (noncausal: all rows; causal:
  rows i >= j); causal rows i < j are masked before the softmax in both and match;
* a NaN in value (j, d) makes dimension d NaN in every row that sees key j, and no
  other dimension.
One case is not covered: causal rows i < j with a NaN in value row j. The formula's
P.V multiplies their zero probability by the NaN (0 * NaN = NaN in every row of the
head); the kernels skip key tiles past a row's diagonal, so such a row is NaN only when
key j falls in a key tile its wave computes.

Infinities are honoured (no -fno-honor-infs) and follow the formula the same way:
* +inf in query row i gives that row scores of both signs of infinity; its max is +inf
  and inf - inf makes the row NaN;
* +inf in key row j, dimension e, gives +inf scores in the rows whose q[e] > 0 (NaN
  rows) and -inf in the rows whose q[e] < 0 (key j gets probability 0, the row stays
  finite);
* +inf in value (j, d) makes dimension d infinite in every row that sees key j, with
  the same exception as the NaN case for causal rows i < j.
"""

from __future__ import annotations

import pytest
import torch

import flash_attention_2_lab_amd as fa
from flash_attention_2_lab_amd import capi
from oracle import attention_reference_fp32

pytestmark = pytest.mark.gpu

PRODUCTION = fa.flash_attention_cuda.tensorcore_attention_forward_production_128x128
KEY_TILE_16 = fa.flash_attention_cuda.tensorcore_attention_forward  # noncausal, N % 16 == 0


def ENTRY(q, k, v, causal):
    """The production entry; sequence lengths that are not a multiple of 128 go through the
    key-tile-16 entry (noncausal only), whose partial last query block and key tile run the
    kernels' partial-tile builds."""
    if q.shape[2] % 128 == 0:
        return PRODUCTION(q, k, v, causal)
    assert not causal
    return KEY_TILE_16(q, k, v)


# Every kernel the forward entries route to, and the partial-tile builds of the two key-split
# kernels that sequence lengths off the 32-key grid reach.
SHAPES = [
    ((1, 8, 1024), False, capi.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES), ((1, 8, 1024), True, capi.FA2_KERNEL_KEY_SPLIT_PAIRS16),
    ((1, 8, 768), False, capi.FA2_KERNEL_KEY_SPLIT_64),
    ((1, 9, 1024), False, capi.FA2_KERNEL_KEY_SPLIT_32), ((1, 8, 384), True, capi.FA2_KERNEL_KEY_SPLIT_32),
    ((1, 64, 1024), False, capi.FA2_KERNEL_128_QUERY), ((1, 64, 1024), True, capi.FA2_KERNEL_128_QUERY),
    ((8, 16, 1024), False, capi.FA2_KERNEL_256_QUERY), ((8, 256, 256), True, capi.FA2_KERNEL_256_QUERY),
    ((8, 64, 512), True, capi.FA2_KERNEL_256_QUERY_PAIRS), ((1, 4, 2048), False, capi.FA2_KERNEL_KEY_SPLIT_8_WAVES),
    ((1, 2, 4096), True, capi.FA2_KERNEL_KEY_SPLIT_8_WAVES),
    ((1, 5, 8192), True, capi.FA2_KERNEL_128_QUERY_SPLIT_PAIRS),
    ((1, 8, 2000), False, capi.FA2_KERNEL_KEY_SPLIT_32), ((1, 3, 2000), False, capi.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES),
]
IDS = [f"{'causal' if c else 'noncausal'}-{b}x{h}x{n}" for (b, h, n), c, _ in SHAPES]


def _inputs(shape, seed):
    gen = torch.Generator().manual_seed(seed)
    return tuple(torch.randn((*shape, 64), generator=gen).half() for _ in range(3))


def _check(out, expected, nan_mask):
    """NaN exactly where nan_mask is set; elsewhere within the north-star gate."""
    out = out.float().cpu()
    assert torch.equal(torch.isnan(out), nan_mask)
    keep = ~nan_mask
    torch.testing.assert_close(out[keep], expected[keep], atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("shape, causal, kernel", SHAPES, ids=IDS)
def test_nan_in_query_row(shape, causal, kernel):
    assert capi.forward_plan(*shape, causal) == kernel
    q, k, v = _inputs(shape, seed=71)
    n = shape[2]
    b, h, i = shape[0] - 1, shape[1] // 2, n // 2 + 5
    q[b, h, i, 17] = float("nan")
    expected = attention_reference_fp32(q, k, v, causal=causal)
    mask = torch.zeros(expected.shape, dtype=torch.bool)
    mask[b, h, i] = True
    assert torch.equal(torch.isnan(expected), mask)
    _check(ENTRY(q.cuda(), k.cuda(), v.cuda(), causal), expected, mask)


@pytest.mark.parametrize("shape, causal, kernel", SHAPES, ids=IDS)
def test_nan_in_key_row(shape, causal, kernel):
    assert capi.forward_plan(*shape, causal) == kernel
    q, k, v = _inputs(shape, seed=72)
    n = shape[2]
    b, h, j = 0, shape[1] - 1, n // 3
    k[b, h, j, 40] = float("nan")
    expected = attention_reference_fp32(q, k, v, causal=causal)
    mask = torch.zeros(expected.shape, dtype=torch.bool)
    mask[b, h, j if causal else 0:] = True
    assert torch.equal(torch.isnan(expected), mask)
    _check(ENTRY(q.cuda(), k.cuda(), v.cuda(), causal), expected, mask)


@pytest.mark.parametrize("shape, causal, kernel", SHAPES, ids=IDS)
def test_nan_in_value_element(shape, causal, kernel):
    assert capi.forward_plan(*shape, causal) == kernel
    q, k, v = _inputs(shape, seed=73)
    n = shape[2]
    b, h, j, d = 0, 0, n - 70, 9
    v[b, h, j, d] = float("nan")
    expected = attention_reference_fp32(q, k, v, causal=causal)
    out = ENTRY(q.cuda(), k.cuda(), v.cuda(), causal).float().cpu()
    if causal:
        # Rows before the key: compared outside dimension d only (see the module docstring).
        out[b, h, :j, d] = 0.0
        expected[b, h, :j, d] = 0.0
    mask = torch.zeros(expected.shape, dtype=torch.bool)
    mask[b, h, j if causal else 0:, d] = True
    assert torch.equal(torch.isnan(expected), mask)
    _check(out, expected, mask)


def _check_nonfinite(out, expected):
    """NaN and +-inf exactly where the oracle has them; elsewhere within the gate."""
    out = out.float().cpu()
    assert torch.equal(torch.isnan(out), torch.isnan(expected))
    assert torch.equal(torch.isposinf(out), torch.isposinf(expected))
    assert torch.equal(torch.isneginf(out), torch.isneginf(expected))
    finite = torch.isfinite(expected)
    torch.testing.assert_close(out[finite], expected[finite], atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("shape, causal, kernel", SHAPES, ids=IDS)
def test_inf_in_query_row(shape, causal, kernel):
    assert capi.forward_plan(*shape, causal) == kernel
    q, k, v = _inputs(shape, seed=74)
    n = shape[2]
    b, h, i = shape[0] - 1, 0, n - 3
    q[b, h, i, 17] = float("inf")
    expected = attention_reference_fp32(q, k, v, causal=causal)
    assert torch.isnan(expected[b, h, i]).all() and int(torch.isnan(expected).sum()) == 64
    _check_nonfinite(ENTRY(q.cuda(), k.cuda(), v.cuda(), causal), expected)


@pytest.mark.parametrize("shape, causal, kernel", SHAPES, ids=IDS)
def test_inf_in_key_row(shape, causal, kernel):
    assert capi.forward_plan(*shape, causal) == kernel
    q, k, v = _inputs(shape, seed=75)
    n = shape[2]
    b, h, j, e = 0, shape[1] // 3, n // 4 + 1, 40
    k[b, h, j, e] = float("inf")
    expected = attention_reference_fp32(q, k, v, causal=causal)
    nan_rows = q[b, h, :, e].float() > 0
    if causal:
        nan_rows[:j] = False
    assert torch.equal(torch.isnan(expected[b, h]).all(-1), nan_rows)
    assert 0 < int(nan_rows.sum()) < n - j
    _check_nonfinite(ENTRY(q.cuda(), k.cuda(), v.cuda(), causal), expected)


@pytest.mark.parametrize("shape, causal, kernel", SHAPES, ids=IDS)
def test_inf_in_value_element(shape, causal, kernel):
    assert capi.forward_plan(*shape, causal) == kernel
    q, k, v = _inputs(shape, seed=76)
    n = shape[2]
    b, h, j, d = shape[0] - 1, shape[1] - 1, 33, 50
    v[b, h, j, d] = float("inf")
    expected = attention_reference_fp32(q, k, v, causal=causal)
    out = ENTRY(q.cuda(), k.cuda(), v.cuda(), causal).float().cpu()
    if causal:
        # Rows before the key: compared outside dimension d only (see the module docstring).
        out[b, h, :j, d] = 0.0
        expected[b, h, :j, d] = 0.0
    assert int(torch.isinf(expected).sum()) == n - (j if causal else 0)
    _check_nonfinite(out, expected)
