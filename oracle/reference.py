"""CPU restatement of the reference attention semantics - TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
See oracle/__init__.py for how each function is pinned.
"""

from __future__ import annotations

import math
from collections.abc import Iterable

import numpy as np
import torch
from torch import Tensor


def validate_inputs(query: Tensor, key: Tensor, value: Tensor) -> None:
    """Input checks of the reference oracle (flash_attention/reference.py:65-100).

    Same exception types and the message fragments the reference tests match on
    ("must have shape", "same sequence length"; tests/test_reference.py:106-120).
    """
    for name, tensor in (("query", query), ("key", key), ("value", value)):
        if tensor.ndim != 4:
            raise ValueError(
                f"{name} must have shape [batch, heads, sequence, head_dimension], "
                f"got {tuple(tensor.shape)}"
            )
        if not tensor.is_floating_point():
            raise TypeError(f"{name} must use a floating-point dtype, got {tensor.dtype}")
    if not (query.device == key.device == value.device):
        raise ValueError("query, key, and value must be on the same device")
    if not (query.dtype == key.dtype == value.dtype):
        raise ValueError("query, key, and value must use the same dtype")
    if not (query.shape[0] == key.shape[0] == value.shape[0]):
        raise ValueError("query, key, and value must have the same batch size")
    if not (query.shape[1] == key.shape[1] == value.shape[1]):
        raise ValueError("query, key, and value must have the same number of heads")
    if query.shape[-1] != key.shape[-1]:
        raise ValueError("query and key must have the same head dimension")
    if key.shape[-2] != value.shape[-2]:
        raise ValueError("key and value must have the same sequence length")


def _default_scale(head_dim: int, scale: float | None) -> float:
    # flash_attention/reference.py:35 - 1/sqrt(D) unless given.
    return scale if scale is not None else 1.0 / math.sqrt(head_dim)


def attention_reference_fp32(query: Tensor, key: Tensor, value: Tensor, *,
                             causal: bool = False, scale: float | None = None) -> Tensor:
    """FP32 attention before the final cast (flash_attention/reference.py:9-59).

    Scores are formed in FP32 from the FP32-converted inputs, scaled after the
    product, masked with -inf where key index > query index (strict upper triangle,
    reference.py:49-56), normalised with softmax over keys and applied to V.
    """
    validate_inputs(query, key, value)
    s = _default_scale(query.shape[-1], scale)
    q32, k32, v32 = query.float(), key.float(), value.float()
    logits = torch.matmul(q32, k32.transpose(-2, -1)) * s
    if causal:
        n_q, n_k = query.shape[-2], key.shape[-2]
        future = torch.triu(torch.ones(n_q, n_k, dtype=torch.bool, device=query.device), 1)
        logits = logits.masked_fill(future, float("-inf"))
    weights = torch.softmax(logits, dim=-1)
    return torch.matmul(weights, v32)


def attention_reference(query: Tensor, key: Tensor, value: Tensor, *,
                        causal: bool = False, scale: float | None = None) -> Tensor:
    """Reference attention cast back to the input dtype (flash_attention/reference.py:9-61)."""
    out = attention_reference_fp32(query, key, value, causal=causal, scale=scale)
    return out.to(dtype=query.dtype)


def attention_rows_fp32(query: Tensor, key: Tensor, value: Tensor,
                        rows: Iterable[tuple[int, int, int]], *, causal: bool = False,
                        scale: float | None = None) -> Tensor:
    """FP32 reference output for selected (batch, head, query_row) triples.

    The same arithmetic as attention_reference_fp32 restricted to the listed rows,
    so shapes whose full score tensor would not fit (B16 H16 N4096, B2 H32 N16384)
    can still be checked row by row. Returns [len(rows), D] in FP32, in input order.
    """
    validate_inputs(query, key, value)
    s = _default_scale(query.shape[-1], scale)
    rows = [tuple(int(x) for x in r) for r in rows]
    out = torch.empty(len(rows), value.shape[-1], dtype=torch.float32)
    by_head: dict[tuple[int, int], list[int]] = {}
    for idx, (b, h, _) in enumerate(rows):
        by_head.setdefault((b, h), []).append(idx)
    n_k = key.shape[-2]
    for (b, h), idxs in by_head.items():
        qi = torch.tensor([rows[i][2] for i in idxs], dtype=torch.long)
        q32 = query[b, h].index_select(0, qi.to(query.device)).float().cpu()
        k32 = key[b, h].float().cpu()
        v32 = value[b, h].float().cpu()
        logits = torch.matmul(q32, k32.transpose(0, 1)) * s
        if causal:
            future = torch.arange(n_k).unsqueeze(0) > qi.unsqueeze(1)
            logits = logits.masked_fill(future, float("-inf"))
        out[idxs] = torch.matmul(torch.softmax(logits, dim=-1), v32)
    return out


def attention_float64_rowwise(query, key, value, *, causal: bool = False,
                              scale: float | None = None) -> np.ndarray:
    """Independent float64 evaluation, one query row at a time (tiny shapes only).

    For every (b, h, i): logits_j = scale * <q_i, k_j>; keys j > i dropped when
    causal; weights = exp(logits - max) / sum; out = sum_j weights_j v_j.
    Accepts tensors or arrays; returns a float64 numpy array [B, H, Nq, Dv].
    """
    q = np.asarray(torch.as_tensor(query).double().cpu())
    k = np.asarray(torch.as_tensor(key).double().cpu())
    v = np.asarray(torch.as_tensor(value).double().cpu())
    s = _default_scale(q.shape[-1], scale)
    batch, heads, n_q, _ = q.shape
    out = np.zeros((batch, heads, n_q, v.shape[-1]), dtype=np.float64)
    for b in range(batch):
        for h in range(heads):
            for i in range(n_q):
                visible = k.shape[2] if not causal else min(i + 1, k.shape[2])
                logits = (k[b, h, :visible] @ q[b, h, i]) * s
                w = np.exp(logits - logits.max())
                out[b, h, i] = (w @ v[b, h, :visible]) / w.sum()
    return out


def flash_forward_tiled(query: Tensor, key: Tensor, value: Tensor, *, causal: bool = False,
                        block_n: int = 128, round_p_to_fp16: bool = True) -> Tensor:
    """Model of the reference production kernel's arithmetic, in FP32 on the CPU.

    Streams keys in tiles of ``block_n`` (csrc/tensorcore_attention.cu:2229-2561) with
    the online softmax of :448-671: tile row max of scaled scores, m_new = max(m,
    tile max), alpha = 0 when the running sum is 0 else exp(m - m_new), p =
    exp(s * scale - m_new), l = alpha * l + sum(p) over FP32 p, O = alpha * O + P V
    with P rounded to FP16 (:434-447, :2479-2552); output O / l rounded to FP16
    (:2575-2683). Masked entries are -inf (:674-698). Returns FP16 [B, H, N, D].
    """
    validate_inputs(query, key, value)
    scale = 1.0 / math.sqrt(query.shape[-1])
    q = query.float().cpu()
    k = key.float().cpu()
    v = value.float().cpu()
    batch, heads, n_q, d = q.shape
    n_k = k.shape[2]
    m = torch.full((batch, heads, n_q, 1), float("-inf"))
    l = torch.zeros((batch, heads, n_q, 1))
    acc = torch.zeros((batch, heads, n_q, v.shape[-1]))
    query_index = torch.arange(n_q).view(1, 1, n_q, 1)
    for k0 in range(0, n_k, block_n):
        k1 = min(k0 + block_n, n_k)
        s = torch.matmul(q, k[:, :, k0:k1].transpose(-2, -1)) * scale
        if causal:
            key_index = torch.arange(k0, k1).view(1, 1, 1, k1 - k0)
            s = s.masked_fill(key_index > query_index, float("-inf"))
        m_new = torch.maximum(m, s.amax(dim=-1, keepdim=True))
        alpha = torch.where(l == 0, torch.zeros_like(l), torch.exp(m - m_new))
        # Rows whose every key so far is masked keep m = -inf; their p is 0.
        p = torch.exp(s - torch.where(torch.isinf(m_new), torch.zeros_like(m_new), m_new))
        p = torch.where(torch.isinf(s), torch.zeros_like(p), p)
        l = alpha * l + p.sum(dim=-1, keepdim=True)
        p_mma = p.half().float() if round_p_to_fp16 else p
        acc = alpha * acc + torch.matmul(p_mma, v[:, :, k0:k1])
        m = m_new
    return (acc / l).half()


def attention_scores_fp32(query: Tensor, key: Tensor, *, scale: float | None = None) -> Tensor:
    """FP32 scaled scores Q K^T * s, [B, H, N, N] (reference naive_attention_scores,
    csrc/naive_attention.cu:174-201 and 330-418; its test formula,
    tests/test_naive_scores.py:48-54): the product of the FP32-converted inputs,
    then the scale 1/sqrt(D) unless given."""
    if query.ndim != 4 or key.ndim != 4:
        raise ValueError("query and key must have shape [batch, heads, sequence, head_dimension]")
    s = _default_scale(query.shape[-1], scale)
    return torch.matmul(query.float().cpu(), key.float().cpu().transpose(-2, -1)) * s


def matmul_16x64x16_fp32(matrix_a: Tensor, matrix_b: Tensor) -> Tensor:
    """FP32 product of [batch, 16, 64] and [batch, 64, 16] FP16 matrices (reference
    wmma_matmul_16x64x16, csrc/wmma_matmul.cu:51-193: four 16x16x16 FP16 products
    accumulated in FP32; its test formula, tests/test_wmma_matmul.py:94-120)."""
    if matrix_a.ndim != 3 or tuple(matrix_a.shape[1:]) != (16, 64):
        raise ValueError("A must have shape [batch, 16, 64]")
    if matrix_b.ndim != 3 or tuple(matrix_b.shape[1:]) != (64, 16):
        raise ValueError("B must have shape [batch, 64, 16]")
    return torch.matmul(matrix_a.float().cpu(), matrix_b.float().cpu())
