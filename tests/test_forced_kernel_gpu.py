"""Every FP16 forward kernel held to the oracle through fa2_forward_with_kernel, on shapes
the kernel choice routes to it and on shapes it routes elsewhere (the neighbours of each
routing threshold run both ways when the choice is re-measured)."""

from __future__ import annotations

import pytest
import torch

from flash_attention_2_lab_amd import capi
from oracle import attention_reference_fp32

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RTOL = 1e-2
K = capi

# (kernel, (batch, heads, seq_len), causal): every kernel in each mode it computes, at
# lengths from its shortest to past its routed range.
CASES = [
    (K.FA2_KERNEL_256_QUERY, (1, 2, 256), False), (K.FA2_KERNEL_256_QUERY, (1, 3, 768), True),
    (K.FA2_KERNEL_256_QUERY, (2, 2, 1024), False), (K.FA2_KERNEL_256_QUERY, (1, 2, 2048), True),
    (K.FA2_KERNEL_256_QUERY_PAIRS, (1, 3, 512), True), (K.FA2_KERNEL_256_QUERY_PAIRS, (1, 2, 2048), True),
    (K.FA2_KERNEL_128_QUERY, (1, 2, 128), False), (K.FA2_KERNEL_128_QUERY, (1, 3, 640), True),
    (K.FA2_KERNEL_128_QUERY, (2, 1, 2048), False), (K.FA2_KERNEL_128_QUERY, (1, 2, 2048), True),
    (K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS, (1, 2, 1024), True), (K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS, (1, 3, 2048), True),
    (K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS, (1, 1, 4096), True),
    (K.FA2_KERNEL_KEY_SPLIT_64, (1, 2, 128), False), (K.FA2_KERNEL_KEY_SPLIT_64, (1, 3, 1152), True),
    (K.FA2_KERNEL_KEY_SPLIT_64, (1, 2, 2048), False),
    (K.FA2_KERNEL_KEY_SPLIT_32, (1, 2, 128), True), (K.FA2_KERNEL_KEY_SPLIT_32, (2, 2, 1024), False),
    (K.FA2_KERNEL_KEY_SPLIT_32, (1, 2, 2048), True),
    (K.FA2_KERNEL_KEY_SPLIT_8_WAVES, (1, 2, 256), False), (K.FA2_KERNEL_KEY_SPLIT_8_WAVES, (1, 3, 1024), True),
    (K.FA2_KERNEL_KEY_SPLIT_8_WAVES, (1, 1, 4096), False),
    (K.FA2_KERNEL_KEY_SPLIT_PAIRS16, (1, 2, 512), True), (K.FA2_KERNEL_KEY_SPLIT_PAIRS16, (1, 3, 1536), True),
    (K.FA2_KERNEL_KEY_SPLIT_PAIRS16, (1, 1, 4096), True),
    (K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES, (1, 2, 128), False), (K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES, (1, 3, 640), False),
    (K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES, (1, 2, 4096), False),
]
IDS = [f"k{k}-{'causal' if c else 'noncausal'}-{b}x{h}x{n}" for k, (b, h, n), c in CASES]


def _inputs(shape, seed):
    gen = torch.Generator().manual_seed(seed)
    return tuple(torch.randn((*shape, 64), generator=gen).half() for _ in range(3))


@pytest.mark.parametrize("kernel, shape, causal", CASES, ids=IDS)
def test_forced_kernel_matches_oracle(kernel, shape, causal):
    q, k, v = _inputs(shape, seed=91)
    out = capi.forward_with_kernel(kernel, q.cuda(), k.cuda(), v.cuda(), causal)
    torch.cuda.synchronize()
    expected = attention_reference_fp32(q, k, v, causal=causal)
    torch.testing.assert_close(out.float().cpu(), expected, atol=ATOL, rtol=RTOL)
    if capi.forward_plan(*shape, causal) == kernel:
        routed = capi.forward_production_128x128(q.cuda(), k.cuda(), v.cuda(), causal)
        torch.cuda.synchronize()
        assert torch.equal(out, routed), "the forced and the routed call of one kernel differ"


@pytest.mark.parametrize("kernel, seq_len, causal", [
    (K.FA2_KERNEL_256_QUERY, 384, False), (K.FA2_KERNEL_256_QUERY_PAIRS, 512, False),
    (K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS, 768, True), (K.FA2_KERNEL_KEY_SPLIT_PAIRS16, 384, True),
    (K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES, 1024, True), (K.FA2_KERNEL_NONE, 1024, False),
])
def test_forced_kernel_outside_its_domain_is_refused_without_a_launch(kernel, seq_len, causal):
    q = torch.zeros(1, 1, seq_len, 64, dtype=torch.float16, device="cuda")
    out = torch.full_like(q, 7.0)
    with pytest.raises(capi.Fa2Error) as info:
        capi.forward_with_kernel(kernel, q, q, q, causal, output=out)
    assert info.value.status == capi.FA2_STATUS_BAD_KERNEL
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)
