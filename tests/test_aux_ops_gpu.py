"""GPU tests of the module's other operators against the CPU oracle, mirroring the
reference's tests (shapes and tolerances): tests/test_extension.py,
tests/test_naive_scores.py, tests/test_naive_attention.py, tests/test_block_attention.py,
tests/test_tiled_attention.py, tests/test_tilewise_attention.py and
tests/test_wmma_matmul.py. Inputs are drawn on the CPU and copied, so the oracle sees
the same values; the binding and the C ABI (ctypes) must agree bitwise.
"""

from __future__ import annotations

import pytest
import torch

import flash_attention_2_lab_amd as fa
from flash_attention_2_lab_amd import capi
from oracle import attention_reference_fp32, attention_scores_fp32, matmul_16x64x16_fp32

pytestmark = pytest.mark.gpu

M = fa.flash_attention_cuda


def _randn(*shape, seed=0, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=gen).to(dtype)


# copy_cuda ------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("shape", [(2, 3, 17, 64), (7,), (3, 5, 1), (4096, 33)])
def test_copy_cuda(dtype, shape):
    # Reference tests/test_extension.py:9-35.
    x = _randn(*shape, dtype=dtype).cuda()
    out = M.copy_cuda(x)
    assert out.device == x.device and out.dtype == x.dtype and out.shape == x.shape
    assert out.data_ptr() != x.data_ptr()
    assert torch.equal(out, x)
    assert torch.equal(capi.copy(x), x)


def test_copy_cuda_misaligned_view_and_empty():
    base = _randn(1001, dtype=torch.float16).cuda()
    view = base[1:]                      # contiguous, 2-byte aligned
    assert torch.equal(M.copy_cuda(view), view)
    empty = torch.empty(0, 5, device="cuda")
    assert M.copy_cuda(empty).shape == (0, 5)


def test_copy_cuda_rejects_noncontiguous_and_integer():
    x = _randn(4, 6).cuda().t()
    with pytest.raises(RuntimeError, match="input must be contiguous"):
        M.copy_cuda(x)
    with pytest.raises(NotImplementedError, match="\"copy_cuda\" not implemented for 'Int'"):
        M.copy_cuda(torch.zeros(8, dtype=torch.int32, device="cuda"))


# naive_attention_scores -------------------------------------------------------

@pytest.mark.parametrize("shape", [(1, 1, 1, 16), (1, 1, 7, 32), (1, 2, 17, 64), (2, 3, 31, 32),
                                   (1, 4, 65, 64), (2, 2, 300, 64), (1, 1, 130, 100)])
def test_scores_match_oracle(shape):
    # Reference tests/test_naive_scores.py:10-67 (rtol = atol = 1e-5).
    q, k = _randn(*shape, seed=1), _randn(*shape, seed=2)
    out = M.naive_attention_scores(q.cuda(), k.cuda())
    assert out.shape == (*shape[:3], shape[2]) and out.dtype == torch.float32 and out.is_contiguous()
    torch.testing.assert_close(out.cpu(), attention_scores_fp32(q, k), rtol=1e-5, atol=1e-5)
    assert torch.equal(capi.attention_scores_f32(q.cuda(), k.cuda()), out)


def test_scores_preserve_batch_head_separation():
    # Reference tests/test_naive_scores.py:71-107.
    q = torch.zeros(2, 2, 3, 4)
    k = torch.zeros_like(q)
    for i, (b, h) in enumerate([(0, 0), (0, 1), (1, 0), (1, 1)]):
        q[b, h].fill_(1.0 + i)
        k[b, h].fill_(5.0 + i)
    out = M.naive_attention_scores(q.cuda(), k.cuda()).cpu()
    torch.testing.assert_close(out, attention_scores_fp32(q, k))


def test_scores_reject_noncontiguous():
    # Reference tests/test_naive_scores.py:111-129.
    q = _randn(1, 2, 8, 32).cuda()
    with pytest.raises(RuntimeError, match="contiguous"):
        M.naive_attention_scores(q.transpose(1, 2), q)


# FP32 SIMT attention forwards -----------------------------------------------

@pytest.mark.parametrize("shape", [(1, 1, 1, 64), (1, 2, 17, 64), (2, 3, 31, 64), (1, 4, 65, 64),
                                   (1, 2, 17, 128)])
def test_naive_attention_matches_oracle(shape):
    # Reference tests/test_naive_attention.py:10-55 (rtol = atol = 1e-4).
    q, k, v = (_randn(*shape, seed=s) for s in (3, 4, 5))
    out = M.naive_attention_forward(q.cuda(), k.cuda(), v.cuda())
    torch.testing.assert_close(out.cpu(), attention_reference_fp32(q, k, v), rtol=1e-4, atol=1e-4)


def test_naive_attention_does_not_modify_inputs():
    # Reference tests/test_naive_attention.py:58-81.
    q, k, v = (_randn(1, 2, 17, 64, seed=s).cuda() for s in (6, 7, 8))
    before = [t.clone() for t in (q, k, v)]
    M.naive_attention_forward(q, k, v)
    torch.cuda.synchronize()
    for t, b in zip((q, k, v), before):
        assert torch.equal(t, b)


def test_naive_attention_rejects_unsupported_head_dimension():
    # Reference tests/test_naive_attention.py:84-94.
    x = _randn(1, 1, 8, 32).cuda()
    with pytest.raises(RuntimeError, match="64 and 128"):
        M.naive_attention_forward(x, x, x)


@pytest.mark.parametrize("shape", [(1, 1, 1, 64), (1, 2, 17, 64), (2, 3, 31, 64), (1, 8, 128, 64),
                                   (1, 2, 17, 128), (1, 8, 128, 128)])
def test_block_attention_matches_oracle(shape):
    # Reference tests/test_block_attention.py:10-61 (rtol = atol = 1e-4).
    q, k, v = (_randn(*shape, seed=s) for s in (9, 10, 11))
    out = M.block_attention_forward(q.cuda(), k.cuda(), v.cuda())
    torch.testing.assert_close(out.cpu(), attention_reference_fp32(q, k, v), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("name", ["tiled_attention_forward", "tilewise_attention_forward"])
@pytest.mark.parametrize("batch, heads, seq_len", [(1, 1, 1), (1, 1, 15), (1, 2, 16), (1, 2, 17),
                                                   (1, 4, 31), (1, 4, 32), (1, 4, 33), (2, 3, 65),
                                                   (1, 8, 128), (1, 8, 512)])
def test_tiled_and_tilewise_match_oracle(name, batch, heads, seq_len):
    # Reference tests/test_tiled_attention.py and test_tilewise_attention.py:10-68
    # (rtol = atol = 2e-4).
    q, k, v = (_randn(batch, heads, seq_len, 64, seed=s) for s in (12, 13, 14))
    out = getattr(M, name)(q.cuda(), k.cuda(), v.cuda())
    torch.testing.assert_close(out.cpu(), attention_reference_fp32(q, k, v), rtol=2e-4, atol=2e-4)


@pytest.mark.parametrize("shape", [(2, 4, 1000, 64), (1, 2, 513, 128)])
def test_f32_forward_larger_shapes_and_c_abi(shape):
    q, k, v = (_randn(*shape, seed=s) for s in (15, 16, 17))
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    out = M.block_attention_forward(qd, kd, vd)
    torch.testing.assert_close(out.cpu(), attention_reference_fp32(q, k, v), rtol=1e-4, atol=1e-4)
    assert torch.equal(capi.attention_forward_f32(qd, kd, vd), out)
    assert torch.equal(M.naive_attention_forward(qd, kd, vd), out)


def test_f32_forwards_on_empty_sequences():
    x = torch.empty(2, 3, 0, 64, device="cuda")
    for name in ["naive_attention_forward", "block_attention_forward", "tiled_attention_forward",
                 "tilewise_attention_forward"]:
        assert getattr(M, name)(x, x, x).shape == x.shape
    assert M.naive_attention_scores(x, x).shape == (2, 3, 0, 0)


# wmma_matmul_16x64x16 --------------------------------------------------------

@pytest.mark.parametrize("batch", [1, 4])
def test_matmul_identity_block(batch):
    # Reference tests/test_wmma_matmul.py:13-75 (rtol = atol = 1e-3).
    a = _randn(batch, 16, 64, seed=18, dtype=torch.float16)
    b = torch.zeros(batch, 64, 16, dtype=torch.float16)
    b[:, :16, :] = torch.eye(16, dtype=torch.float16)
    out = M.wmma_matmul_16x64x16(a.cuda(), b.cuda())
    assert out.dtype == torch.float32 and out.shape == (batch, 16, 16)
    torch.testing.assert_close(out.cpu(), a[:, :, :16].float(), rtol=1e-3, atol=1e-3)
    # Products of FP16 values by 1 and 0 are exact: the fragment layout is exact too.
    assert torch.equal(out.cpu(), a[:, :, :16].float())


@pytest.mark.parametrize("batch", [1, 4, 17, 1000])
def test_matmul_matches_oracle(batch):
    # Reference tests/test_wmma_matmul.py:78-120 (rtol = atol = 5e-3); FP16 products
    # are exact in FP32, so the MFMA result is held to 1e-4 here.
    a = _randn(batch, 16, 64, seed=19, dtype=torch.float16)
    b = _randn(batch, 64, 16, seed=20, dtype=torch.float16)
    out = M.wmma_matmul_16x64x16(a.cuda(), b.cuda())
    torch.testing.assert_close(out.cpu(), matmul_16x64x16_fp32(a, b), rtol=1e-4, atol=1e-4)
    assert torch.equal(capi.matmul_16x64x16(a.cuda(), b.cuda()), out)
    assert M.wmma_matmul_16x64x16(a[:0].cuda(), b[:0].cuda()).shape == (0, 16, 16)
