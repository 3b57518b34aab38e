"""CPU tests of the C ABI library: it loads, exports every declared symbol, and rejects
bad arguments with the documented status codes before any HIP call is made."""

from __future__ import annotations

import ctypes
import re

import pytest

import flash_attention_2_lab_amd as fa
from flash_attention_2_lab_amd import capi


def test_library_exports_every_declared_function():
    declared = capi.declared_functions()
    assert {"fa2_forward_production_128x128", "fa2_forward_tensorcore", "fa2_status_string",
            "fa2_abi_version"} <= set(declared)
    lib = ctypes.CDLL(str(capi.LIBRARY_PATH))
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/fa2_mi355x.h but not exported"


def test_abi_version_matches_header():
    text = capi.HEADER_PATH.read_text()
    version = int(re.search(r"#define FA2_MI355X_ABI_VERSION (\d+)", text).group(1))
    assert capi.abi_version() == version == fa.flash_attention_cuda.abi_version


def test_status_codes_match_header():
    text = capi.HEADER_PATH.read_text()
    for name in ("SUCCESS", "NULL_POINTER", "NEGATIVE_DIMENSION", "BAD_HEAD_DIM",
                 "BAD_SEQUENCE_LENGTH", "MISALIGNED", "TOO_LARGE", "BAD_KEY_TILE",
                 "BAD_KERNEL", "HIP_ERROR_BASE"):
        value = int(re.search(rf"FA2_STATUS_{name} = (\d+)", text).group(1))
        assert getattr(capi, f"FA2_STATUS_{name}") == value


def test_kernel_ids_match_header():
    text = capi.HEADER_PATH.read_text()
    for name in ("NONE", "256_QUERY", "256_QUERY_PAIRS", "128_QUERY", "KEY_SPLIT_64", "KEY_SPLIT_32",
                 "KEY_SPLIT_8_WAVES", "KEY_SPLIT_PAIRS16", "KEY_SPLIT_64_DMA_WAVES", "128_QUERY_SPLIT_PAIRS"):
        value = int(re.search(rf"FA2_KERNEL_{name} = (\d+)", text).group(1))
        assert getattr(capi, f"FA2_KERNEL_{name}") == value


K = capi


@pytest.mark.parametrize("batch, heads, seq_len, causal, kernel", [
    # Noncausal: 256-query from 512 groups of 256 queries, 128-query from 200 groups of
    # 128, key-split below (64-key tiles up to 256 blocks of 32 queries; from 1024 keys
    # with separate DMA waves).
    (1, 128, 1024, False, K.FA2_KERNEL_256_QUERY), (1, 127, 1024, False, K.FA2_KERNEL_128_QUERY),
    (16, 16, 4096, False, K.FA2_KERNEL_256_QUERY), (1, 25, 1024, False, K.FA2_KERNEL_128_QUERY),
    (1, 24, 1024, False, K.FA2_KERNEL_KEY_SPLIT_32), (1, 8, 1024, False, K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES),
    (1, 9, 1024, False, K.FA2_KERNEL_KEY_SPLIT_32), (1, 8, 128, False, K.FA2_KERNEL_KEY_SPLIT_32),
    # ... except where the 256-query grid ends in a last round at most half full and
    # the 128-query kernel's finer rounds are modeled more than 5% faster.
    (1, 36, 4096, False, K.FA2_KERNEL_128_QUERY), (5, 16, 2048, False, K.FA2_KERNEL_128_QUERY),
    (9, 16, 2048, False, K.FA2_KERNEL_128_QUERY), (3, 16, 4096, False, K.FA2_KERNEL_256_QUERY),
    (7, 16, 2048, False, K.FA2_KERNEL_256_QUERY), (6, 16, 4096, False, K.FA2_KERNEL_256_QUERY),
    # Causal: 256-query from 512 workgroups of tile pairs when a head has an even
    # number T of tiles, single tiles from 2048 with an odd number. Single tiles in
    # level order at T >= 16; pairs at T = 2, 4 and 8.
    (16, 16, 4096, True, K.FA2_KERNEL_256_QUERY), (1, 256, 1024, True, K.FA2_KERNEL_256_QUERY_PAIRS),
    (1, 255, 1024, True, K.FA2_KERNEL_128_QUERY), (2, 32, 16384, True, K.FA2_KERNEL_256_QUERY),
    (32, 16, 1024, True, K.FA2_KERNEL_256_QUERY_PAIRS), (1, 504, 1024, True, K.FA2_KERNEL_256_QUERY_PAIRS),
    (8, 16, 2048, True, K.FA2_KERNEL_256_QUERY_PAIRS), (1, 64, 4096, True, K.FA2_KERNEL_256_QUERY),
    (1, 66, 4096, True, K.FA2_KERNEL_256_QUERY), (1, 510, 1024, True, K.FA2_KERNEL_256_QUERY_PAIRS),
    (1, 410, 1280, True, K.FA2_KERNEL_256_QUERY), (1, 409, 1280, True, K.FA2_KERNEL_128_QUERY),
    (1, 64, 1024, True, K.FA2_KERNEL_128_QUERY),
    # Causal, 320 to 512 groups of 128 with 4096 keys or more (a multiple of 256): pairs
    # of 128-query tiles split over two wave groups.
    (1, 8, 8192, True, K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS), (1, 5, 8192, True, K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS),
    (1, 3, 16384, True, K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS), (2, 4, 8192, True, K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS),
    (1, 2, 32768, True, K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS), (1, 9, 8192, True, K.FA2_KERNEL_128_QUERY),
    (1, 16, 4096, True, K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS), (1, 5, 8320, True, K.FA2_KERNEL_128_QUERY),
    (1, 4, 8192, True, K.FA2_KERNEL_KEY_SPLIT_32), (1, 8, 8192, False, K.FA2_KERNEL_128_QUERY),
    # 128-query from 320 groups of 128.
    (1, 40, 1024, True, K.FA2_KERNEL_128_QUERY), (1, 72, 512, True, K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 57, 1024, True, K.FA2_KERNEL_128_QUERY), (1, 39, 1024, True, K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 12, 4096, True, K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS), (1, 24, 2048, True, K.FA2_KERNEL_128_QUERY),
    (1, 10, 4096, True, K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS), (1, 8, 4096, True, K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 8, 1024, True, K.FA2_KERNEL_KEY_SPLIT_PAIRS16), (1, 2, 128, True, K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 8, 896, True, K.FA2_KERNEL_KEY_SPLIT_PAIRS16), (1, 2, 1024, True, K.FA2_KERNEL_KEY_SPLIT_PAIRS16),
    (1, 8, 512, True, K.FA2_KERNEL_KEY_SPLIT_PAIRS16), (1, 8, 384, True, K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 8, 544, True, K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 4, 1920, True, K.FA2_KERNEL_KEY_SPLIT_PAIRS16), (1, 4, 1040, True, K.FA2_KERNEL_KEY_SPLIT_32),
    # Key-split shapes from 2048 keys on split each block's keys over 8 waves.
    (1, 2, 4096, False, K.FA2_KERNEL_KEY_SPLIT_8_WAVES), (1, 1, 2048, True, K.FA2_KERNEL_KEY_SPLIT_8_WAVES),
    (1, 4, 2048, False, K.FA2_KERNEL_KEY_SPLIT_8_WAVES), (1, 1, 8192, True, K.FA2_KERNEL_KEY_SPLIT_8_WAVES),
    (1, 4, 1024, False, K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES), (1, 8, 2048, True, K.FA2_KERNEL_KEY_SPLIT_32),
    (1, 8, 896, False, K.FA2_KERNEL_KEY_SPLIT_32), (1, 8, 768, False, K.FA2_KERNEL_KEY_SPLIT_64), (1, 4, 1920, False, K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES),
    (1, 4, 1040, False, K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES), (1, 2, 2000, False, K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES),
    (1, 1, 2064, False, K.FA2_KERNEL_KEY_SPLIT_8_WAVES),
    # Sequence lengths the production entry rejects but the Bc16/Bc32 entries take
    # (partial last block) run the key-split kernel.
    (4, 64, 1040, False, K.FA2_KERNEL_KEY_SPLIT_32), (1, 2, 80, False, K.FA2_KERNEL_KEY_SPLIT_32), (1, 2, 240, False, K.FA2_KERNEL_KEY_SPLIT_64),
    # Causal 256-query: pairs of tiles at T = 2, 4 and 8, head groups
    # at T >= 16 or odd; split pairs from 4096 keys at 320-512 groups of 128.
    (32, 16, 1024, True, K.FA2_KERNEL_256_QUERY_PAIRS), (8, 16, 2048, True, K.FA2_KERNEL_256_QUERY_PAIRS),
    (16, 16, 4096, True, K.FA2_KERNEL_256_QUERY), (128, 16, 512, True, K.FA2_KERNEL_256_QUERY_PAIRS),
    (64, 16, 512, True, K.FA2_KERNEL_256_QUERY_PAIRS), (1, 20, 16384, True, K.FA2_KERNEL_256_QUERY_PAIRS),
    (1, 16, 4096, True, K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS), (1, 32, 2048, True, K.FA2_KERNEL_128_QUERY),
    # Nothing to launch.
    (0, 8, 1024, False, K.FA2_KERNEL_NONE), (1, 0, 1024, True, K.FA2_KERNEL_NONE),
    (1, 8, 0, False, K.FA2_KERNEL_NONE), (1, 1, (1 << 24) + 128, False, K.FA2_KERNEL_NONE),
])
def test_forward_plan_follows_the_measured_thresholds(batch, heads, seq_len, causal, kernel):
    assert capi.forward_plan(batch, heads, seq_len, causal) == kernel


@pytest.mark.parametrize("status, text", [
    (capi.FA2_STATUS_SUCCESS, "success"),
    (capi.FA2_STATUS_BAD_HEAD_DIM, "head dimension must equal 64"),
    (capi.FA2_STATUS_BAD_SEQUENCE_LENGTH, "sequence length not a multiple of the entry's key tile"),
    (capi.FA2_STATUS_BAD_KEY_TILE, "key tile must be 16 or 32"),
    (capi.FA2_STATUS_BAD_KERNEL, "kernel does not compute these sizes"),
    (capi.FA2_STATUS_NULL_POINTER, "null tensor pointer"),
    (capi.FA2_STATUS_MISALIGNED, "tensor pointer not 16-byte aligned"),
    (999, "unknown status"),
    (-1, "unknown status"),
])
def test_status_strings(status, text):
    assert capi.status_string(status) == text


def _call(batch=1, heads=1, seq_len=128, head_dim=64, ptrs=(0, 0, 0, 0)):
    q, k, v, o = ptrs
    return capi.forward_production_128x128_raw(q, k, v, o, batch, heads, seq_len, head_dim,
                                               False, None)


def test_rejects_head_dim_other_than_64():
    assert _call(head_dim=32) == capi.FA2_STATUS_BAD_HEAD_DIM
    assert _call(head_dim=128) == capi.FA2_STATUS_BAD_HEAD_DIM


@pytest.mark.parametrize("seq_len", [1, 64, 100, 129, 4095])
def test_rejects_sequence_length_not_multiple_of_128(seq_len):
    assert _call(seq_len=seq_len) == capi.FA2_STATUS_BAD_SEQUENCE_LENGTH


def test_rejects_negative_dimensions():
    for kwargs in ({"batch": -1}, {"heads": -2}, {"seq_len": -128}, {"head_dim": -64}):
        assert _call(**kwargs) == capi.FA2_STATUS_NEGATIVE_DIMENSION


def test_empty_problem_succeeds_without_pointers():
    # Reference csrc/tensorcore_attention.cu:3003-3009: empty input returns early.
    assert _call(batch=0) == capi.FA2_STATUS_SUCCESS
    assert _call(heads=0) == capi.FA2_STATUS_SUCCESS
    assert _call(seq_len=0) == capi.FA2_STATUS_SUCCESS


def test_empty_problem_still_checks_head_dim():
    assert _call(batch=0, head_dim=16) == capi.FA2_STATUS_BAD_HEAD_DIM


def test_rejects_null_pointers_for_non_empty_problem():
    assert _call() == capi.FA2_STATUS_NULL_POINTER
    assert _call(ptrs=(4096, 4096, 0, 4096)) == capi.FA2_STATUS_NULL_POINTER


def test_rejects_misaligned_pointers():
    assert _call(ptrs=(4096, 4096 + 8, 4096, 4096)) == capi.FA2_STATUS_MISALIGNED


def test_rejects_problem_beyond_launch_grid():
    # Rejected on sizes alone; the (never dereferenced) pointers are aligned and non-null.
    assert _call(seq_len=1 << 31, ptrs=(4096,) * 4) == capi.FA2_STATUS_TOO_LARGE
    assert _call(batch=1 << 20, heads=1 << 20, ptrs=(4096,) * 4) == capi.FA2_STATUS_TOO_LARGE


def _call_tc(batch=1, heads=1, seq_len=32, head_dim=64, key_tile=16, ptrs=(0, 0, 0, 0)):
    q, k, v, o = ptrs
    return capi.forward_tensorcore_raw(q, k, v, o, batch, heads, seq_len, head_dim, key_tile, None)


@pytest.mark.parametrize("key_tile", [0, 8, 64, 128, -16])
def test_tensorcore_entry_rejects_key_tiles_other_than_16_and_32(key_tile):
    assert _call_tc(key_tile=key_tile) == capi.FA2_STATUS_BAD_KEY_TILE


@pytest.mark.parametrize("key_tile, seq_len", [(16, 8), (16, 24), (16, 100), (32, 16), (32, 48), (32, 1040)])
def test_tensorcore_entry_rejects_sequence_not_multiple_of_key_tile(key_tile, seq_len):
    assert _call_tc(key_tile=key_tile, seq_len=seq_len) == capi.FA2_STATUS_BAD_SEQUENCE_LENGTH


@pytest.mark.parametrize("key_tile, seq_len", [(16, 16), (16, 80), (32, 96), (32, 1056)])
def test_tensorcore_entry_accepts_multiples_of_key_tile(key_tile, seq_len):
    # Accepted shapes get as far as the pointer checks (nothing is launched).
    assert _call_tc(key_tile=key_tile, seq_len=seq_len) == capi.FA2_STATUS_NULL_POINTER


def test_tensorcore_entry_shares_the_other_checks():
    assert _call_tc(head_dim=32) == capi.FA2_STATUS_BAD_HEAD_DIM
    assert _call_tc(batch=-1) == capi.FA2_STATUS_NEGATIVE_DIMENSION
    assert _call_tc(seq_len=0) == capi.FA2_STATUS_SUCCESS
    assert _call_tc(ptrs=(4096, 4104, 4096, 4096)) == capi.FA2_STATUS_MISALIGNED
    assert _call_tc(seq_len=1 << 30, ptrs=(4096,) * 4) == capi.FA2_STATUS_TOO_LARGE


def _call_with(kernel, batch=1, heads=1, seq_len=128, head_dim=64, causal=False, ptrs=(4096,) * 4):
    # Aligned, non-null pointers that are never dereferenced: every call here is rejected
    # before a launch.
    q, k, v, o = ptrs
    return capi.forward_with_kernel_raw(kernel, q, k, v, o, batch, heads, seq_len, head_dim, causal, None)


@pytest.mark.parametrize("kernel, seq_len, causal", [
    (capi.FA2_KERNEL_256_QUERY, 128, False), (capi.FA2_KERNEL_256_QUERY, 384, True),
    (capi.FA2_KERNEL_256_QUERY_PAIRS, 1024, False), (capi.FA2_KERNEL_256_QUERY_PAIRS, 768, True),
    (capi.FA2_KERNEL_128_QUERY_SPLIT_PAIRS, 8192, False), (capi.FA2_KERNEL_128_QUERY_SPLIT_PAIRS, 768, True),
    (capi.FA2_KERNEL_128_QUERY_SPLIT_PAIRS, 1152, True),
    (capi.FA2_KERNEL_KEY_SPLIT_PAIRS16, 1024, False), (capi.FA2_KERNEL_KEY_SPLIT_PAIRS16, 384, True),
    (capi.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES, 1024, True),
    (capi.FA2_KERNEL_NONE, 1024, False), (10, 1024, False), (-1, 1024, True), (1000, 1024, False),
])
def test_forced_kernel_rejects_sizes_it_does_not_compute(kernel, seq_len, causal):
    assert _call_with(kernel, seq_len=seq_len, causal=causal) == capi.FA2_STATUS_BAD_KERNEL


def test_forced_kernel_shares_the_production_checks_first():
    # The entry's own checks come before the kernel's domain, in the production order.
    k = capi.FA2_KERNEL_256_QUERY
    assert _call_with(k, head_dim=32) == capi.FA2_STATUS_BAD_HEAD_DIM
    assert _call_with(k, batch=-1) == capi.FA2_STATUS_NEGATIVE_DIMENSION
    assert _call_with(k, seq_len=100) == capi.FA2_STATUS_BAD_SEQUENCE_LENGTH
    assert _call_with(k, seq_len=0) == capi.FA2_STATUS_SUCCESS
    assert _call_with(k, ptrs=(0, 4096, 4096, 4096)) == capi.FA2_STATUS_NULL_POINTER
    assert _call_with(k, ptrs=(4096, 4104, 4096, 4096)) == capi.FA2_STATUS_MISALIGNED
    assert _call_with(k, seq_len=1 << 31) == capi.FA2_STATUS_TOO_LARGE
    # An unknown kernel id is rejected before anything else.
    assert _call_with(0, head_dim=32) == capi.FA2_STATUS_BAD_KERNEL
