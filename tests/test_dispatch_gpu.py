"""GPU parity on both sides of every kernel-choice threshold of the forward.

The forward picks its kernel from (batch*heads, seq_len, causal) (fa2_forward.hip,
`choose_kernel`): the 256-query kernel from 512 workgroups (noncausal: unless its grid
ends in a partial round that the 128-query kernel's finer rounds finish sooner; causal:
pairs of query tiles at T = 2, 4 and 8 tiles per head, and at any even T when batch*heads
is below 32 and not a multiple of 8; otherwise one query tile per
workgroup in level order, per-XCD head groups when batch*heads is a multiple of 8, odd T
from 2048 tiles), causal problems of 320 to 512 groups of 128 queries with at least 4096
keys (a multiple of 256) in pairs of 128-query tiles whose keys two wave groups split, the
128-query kernel from 200 (noncausal) or 320 (causal) groups of 128 queries, and otherwise
the key-split kernel: up to 256 query blocks of 32, 4 waves with 64-key tiles
(noncausal from 1024 keys with dedicated DMA waves; causal from 512 to 2047 keys, pairs of
16-query blocks; 8 waves with 32-key tiles from 2048 keys on; 32-key tiles when 64-key
tiles would split unevenly over the waves, and causal below 512 keys), and 32-key tiles
beyond. Each case below sits one step below or at a threshold, and `fa2_forward_plan`
(the function the forward dispatches through) must name the kernel the case is meant
to reach; every row of the first and last head and sampled rows of the others are
checked against the FP32 oracle (atol 2e-3 + rtol 1e-2). A second set of shapes, drawn
from a seeded generator over the whole routing table, is checked the same way.
"""

from __future__ import annotations

import math

import pytest
import torch

import flash_attention_2_lab_amd as fa
from flash_attention_2_lab_amd import capi
from oracle import attention_rows_fp32

pytestmark = pytest.mark.gpu

ENTRY = fa.flash_attention_cuda.tensorcore_attention_forward_production_128x128

K = capi
CASES = [
    # (batch, heads, seq_len, causal, kernel it runs, FA2_KERNEL_* id)
    (1, 127, 1024, False, "128-query (508 groups of 256)", K.FA2_KERNEL_128_QUERY),
    (1, 128, 1024, False, "256-query (512 groups of 256)", K.FA2_KERNEL_256_QUERY),
    (1, 36, 4096, False, "128-query (576 wide workgroups: a partial last round)", K.FA2_KERNEL_128_QUERY),
    (3, 16, 4096, False, "256-query (768 wide workgroups: a half-full last round)", K.FA2_KERNEL_256_QUERY),
    (1, 24, 1024, False, "key-split, 32-key tiles (192 groups of 128)", K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 25, 1024, False, "128-query (200 groups of 128)", K.FA2_KERNEL_128_QUERY),
    (1, 32, 1024, False, "128-query (256 groups of 128)", K.FA2_KERNEL_128_QUERY),
    (1, 8, 1024, False, "key-split, 64-key tiles, DMA waves (256 query blocks)", K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES),
    (1, 8, 768, False, "key-split, 64-key tiles (192 blocks, 12 tiles over 4 waves)", K.FA2_KERNEL_KEY_SPLIT_64),
    (1, 8, 896, False, "key-split, 32-key tiles (224 blocks, 14 64-key tiles would split unevenly)", K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 4, 1920, False, "key-split, 64-key tiles, DMA waves (the longest below 2048 keys)",
     K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES),
    (1, 9, 1024, False, "key-split, 32-key tiles (288 query blocks)", K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 255, 1024, True, "128-query (510 tile pairs)", K.FA2_KERNEL_128_QUERY),
    (1, 256, 1024, True, "256-query, tile pairs (512 pairs)", K.FA2_KERNEL_256_QUERY_PAIRS),
    (1, 409, 1280, True, "128-query (2045 single tiles, odd count per head)", K.FA2_KERNEL_128_QUERY),
    (1, 410, 1280, True, "256-query, single tiles (2050, odd count per head)", K.FA2_KERNEL_256_QUERY),
    (1, 39, 1024, True, "key-split, 32-key tiles (312 groups of 128)", K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 57, 1024, True, "128-query (456 groups of 128, heads split across XCDs)", K.FA2_KERNEL_128_QUERY),
    (1, 72, 512, True, "key-split, 32-key tiles (288 groups of 128)", K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 40, 1024, True, "128-query (320 groups of 128, head groups)", K.FA2_KERNEL_128_QUERY),
    (1, 64, 1024, True, "128-query (512 groups of 128)", K.FA2_KERNEL_128_QUERY),
    (1, 8, 1024, True, "key-split, pairs of 16-query blocks (256 pairs)", K.FA2_KERNEL_KEY_SPLIT_PAIRS16),
    (1, 4, 1920, True, "key-split, pairs of 16-query blocks (the longest below 2048 keys)",
     K.FA2_KERNEL_KEY_SPLIT_PAIRS16),
    (1, 8, 896, True, "key-split, pairs of 16-query blocks (896 keys)", K.FA2_KERNEL_KEY_SPLIT_PAIRS16),
    (1, 8, 512, True, "key-split, pairs of 16-query blocks (the shortest, 512 keys)", K.FA2_KERNEL_KEY_SPLIT_PAIRS16),
    (1, 8, 384, True, "key-split, 32-key tiles (causal below 512 keys)", K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 2, 1024, True, "key-split, pairs of 16-query blocks (64 pairs)", K.FA2_KERNEL_KEY_SPLIT_PAIRS16),
    (3, 3, 1024, True, "key-split, 32-key tiles (288 query blocks)", K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 4, 1024, False, "key-split, 64-key tiles, DMA waves (1024 keys)", K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES),
    (1, 4, 2048, False, "key-split, 8 waves (2048 keys, 256 query blocks)", K.FA2_KERNEL_KEY_SPLIT_8_WAVES),
    (1, 2, 4096, True, "key-split, 8 waves (4096 keys)", K.FA2_KERNEL_KEY_SPLIT_8_WAVES),
    (1, 8, 2048, True, "key-split, 32-key tiles (512 query blocks of 2048 keys)", K.FA2_KERNEL_KEY_SPLIT_32),
    (2, 256, 256, False, "256-query (512 groups, the shortest key stream: 4 tiles)", K.FA2_KERNEL_256_QUERY),
    (8, 256, 256, True, "256-query, single tiles (2048 heads of one query tile)", K.FA2_KERNEL_256_QUERY),
    (1, 504, 1024, True, "256-query, tile pairs (2016 tiles of T = 4)", K.FA2_KERNEL_256_QUERY_PAIRS),
    (32, 16, 1024, True, "256-query, tile pairs (2048 tiles of T = 4)", K.FA2_KERNEL_256_QUERY_PAIRS),
    (8, 16, 2048, True, "256-query, tile pairs (1024 tiles of T = 8)", K.FA2_KERNEL_256_QUERY_PAIRS),
    (1, 64, 4096, True, "256-query, head groups (1024 tiles of T = 16)", K.FA2_KERNEL_256_QUERY),
    (1, 66, 4096, True, "256-query, single tiles (XCD ranges splitting heads)", K.FA2_KERNEL_256_QUERY),
    (64, 16, 512, True, "256-query, tile pairs (2048 tiles of T = 2)", K.FA2_KERNEL_256_QUERY_PAIRS),
    (128, 16, 512, True, "256-query, tile pairs (4096 tiles of T = 2)", K.FA2_KERNEL_256_QUERY_PAIRS),
    (1, 20, 16384, True, "256-query, tile pairs (20 heads: XCD ranges would split heads)", K.FA2_KERNEL_256_QUERY_PAIRS),
    (1, 8, 8192, True, "128-query tile pairs split over two wave groups (512 groups of 128)",
     K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS),
    (1, 5, 8192, True, "128-query tile pairs split over two wave groups (320 groups, the fewest)",
     K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS),
    (1, 3, 16384, True, "128-query tile pairs split over two wave groups (16384 keys)",
     K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS),
    (1, 9, 8192, True, "128-query (576 groups of 128, beyond one round)", K.FA2_KERNEL_128_QUERY),
    (1, 16, 4096, True, "128-query tile pairs split over two wave groups (512 groups, 4096 keys)",
     K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS),
    (1, 10, 4096, True, "128-query tile pairs split over two wave groups (320 groups of 4096 keys)",
     K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS),
    (1, 32, 2048, True, "128-query (512 groups of 128, below 4096 keys)", K.FA2_KERNEL_128_QUERY),
    (1, 5, 8320, True, "128-query (325 groups, an odd number of 128-query tiles per head)", K.FA2_KERNEL_128_QUERY),
]


def _random_shapes(per_route, seed):
    # (batch, heads, seq_len, causal) drawn from one seeded stream: seq_len a multiple of
    # 128 up to 4096, batch*heads log-uniform from 1 to 576, at most 576 heads of 1024
    # keys' worth of work. The first `per_route` draws for each (kernel, mode) that the
    # routing table can produce are kept, so every kernel and schedule is checked on
    # shapes nobody picked by hand.
    gen = torch.Generator().manual_seed(seed)
    picked = {}
    for _ in range(40000):
        seq_len = 128 * int(torch.randint(1, 33, (1,), generator=gen))
        batch = int(torch.randint(1, 5, (1,), generator=gen))
        heads = max(1, round(math.exp(float(torch.rand(1, generator=gen)) * math.log(576 / batch))))
        causal = bool(torch.randint(0, 2, (1,), generator=gen))
        if batch * heads * seq_len > 576 * 1024:
            continue
        route = (capi.forward_plan(batch, heads, seq_len, causal), causal)
        shapes = picked.setdefault(route, [])
        if len(shapes) < per_route:
            shapes.append((batch, heads, seq_len, causal))
    return [shape for route in sorted(picked) for shape in picked[route]]


def _random_long_shapes(per_route, seed):
    # The same over long sequences: seq_len a multiple of 256 from 4096 to 16384, causal or
    # not, batch*heads up to the same work cap (576 heads of 1024 keys), so that the
    # routes only long key streams reach (the causal split pairs, 8-wave key-split) are
    # drawn too.
    gen = torch.Generator().manual_seed(seed)
    picked = {}
    for _ in range(20000):
        seq_len = 256 * int(torch.randint(16, 65, (1,), generator=gen))
        limit = max(1, (576 * 1024) // seq_len)
        batch = int(torch.randint(1, 3, (1,), generator=gen))
        heads = max(1, round(math.exp(float(torch.rand(1, generator=gen)) * math.log(max(1, limit // batch)))))
        causal = bool(torch.randint(0, 2, (1,), generator=gen))
        if batch * heads * seq_len > 576 * 1024:
            continue
        route = (capi.forward_plan(batch, heads, seq_len, causal), causal)
        shapes = picked.setdefault(route, [])
        if len(shapes) < per_route:
            shapes.append((batch, heads, seq_len, causal))
    return [shape for route in sorted(picked) for shape in picked[route]]


RANDOM_SHAPES = _random_shapes(3, seed=2024) + _random_long_shapes(2, seed=2025)


def _inputs(batch, heads, seq_len, seed):
    gen = torch.Generator().manual_seed(seed)
    shape = (batch, heads, seq_len, 64)
    return tuple(torch.randn(shape, generator=gen).half() for _ in range(3))


def _check_against_oracle(batch, heads, seq_len, causal, seed):
    q, k, v = _inputs(batch, heads, seq_len, seed=seed)
    out = ENTRY(q.cuda(), k.cuda(), v.cuda(), causal)
    torch.cuda.synchronize()
    out = out.cpu()
    assert torch.isfinite(out).all()
    gen = torch.Generator().manual_seed(seed + 1)
    rows = [(0, 0, i) for i in range(seq_len)] + [(batch - 1, heads - 1, i) for i in range(seq_len)]
    rows += [(int(torch.randint(batch, (1,), generator=gen)), int(torch.randint(heads, (1,), generator=gen)),
              int(torch.randint(seq_len, (1,), generator=gen))) for _ in range(96)]
    rows = sorted(set(rows))
    expected = attention_rows_fp32(q, k, v, rows, causal=causal)
    actual = torch.stack([out[b, h, i] for b, h, i in rows]).float()
    torch.testing.assert_close(actual, expected, atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("batch, heads, seq_len, causal, kernel, kernel_id", CASES,
                         ids=[("causal: " if c[3] else "noncausal: ") + c[4] for c in CASES])
def test_threshold_shapes_match_oracle(batch, heads, seq_len, causal, kernel, kernel_id):
    assert capi.forward_plan(batch, heads, seq_len, causal) == kernel_id
    _check_against_oracle(batch, heads, seq_len, causal, seed=31)


@pytest.mark.parametrize("batch, heads, seq_len, causal", RANDOM_SHAPES,
                         ids=[f"B{b}H{h}N{n}{'c' if c else 'nc'}" for b, h, n, c in RANDOM_SHAPES])
def test_random_shapes_match_oracle(batch, heads, seq_len, causal):
    _check_against_oracle(batch, heads, seq_len, causal, seed=41)
