"""Registry of benchmarkable attention implementations (reference
benchmarks/kernels.py:15-240).

Each spec names a callable of (inputs, workload) and the workloads it supports. The
kernel names and support predicates are the reference's, served by this library's
HIP kernels (the four FP32 SIMT names share one FP32 kernel); `pytorch_sdpa` is the
device comparator and `pytorch_sdpa_cpu` an FP32 CPU comparator (torch's library
routine on host copies of the inputs).
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .workloads import AttentionInputs, AttentionWorkload


@dataclass(frozen=True)
class KernelSpec:
    name: str
    function: Callable[[AttentionInputs, AttentionWorkload], torch.Tensor]
    supported: Callable[[AttentionWorkload], bool]
    on_device: bool = True


def _module():
    import flash_attention_2_lab_amd

    return flash_attention_2_lab_amd.flash_attention_cuda


def _entry(entry: str) -> Callable[[AttentionInputs, AttentionWorkload], torch.Tensor]:
    def run(inputs: AttentionInputs, workload: AttentionWorkload) -> torch.Tensor:
        return getattr(_module(), entry)(inputs.query, inputs.key, inputs.value)
    run.__name__ = entry
    return run


def _production(inputs: AttentionInputs, workload: AttentionWorkload) -> torch.Tensor:
    return _module().tensorcore_attention_forward_production_128x128(
        inputs.query, inputs.key, inputs.value, workload.causal)


def _sdpa(inputs: AttentionInputs, workload: AttentionWorkload) -> torch.Tensor:
    return F.scaled_dot_product_attention(inputs.query, inputs.key, inputs.value,
                                          is_causal=workload.causal)


def _square_fp16_d64(workload: AttentionWorkload) -> bool:
    return (workload.dtype == torch.float16 and workload.query_length == workload.key_length
            and workload.head_dimension == 64)


def _simt_support(head_dims: tuple[int, ...]) -> Callable[[AttentionWorkload], bool]:
    # reference benchmarks/kernels.py:137-183
    return lambda w: (w.dtype == torch.float32 and w.query_length == w.key_length
                      and w.head_dimension in head_dims and not w.causal)


def _tensorcore_support(multiple: int) -> Callable[[AttentionWorkload], bool]:
    return lambda w: _square_fp16_d64(w) and w.query_length % multiple == 0 and not w.causal


class _CpuSdpa:
    """SDPA on FP32 host copies of the inputs (copied once per input set)."""

    def __init__(self) -> None:
        self._source: AttentionInputs | None = None
        self._host: AttentionInputs | None = None

    def __call__(self, inputs: AttentionInputs, workload: AttentionWorkload) -> torch.Tensor:
        if self._source is not inputs:
            self._source = inputs
            self._host = AttentionInputs(*(t.detach().float().cpu()
                                           for t in (inputs.query, inputs.key, inputs.value)))
        return F.scaled_dot_product_attention(self._host.query, self._host.key, self._host.value,
                                              is_causal=workload.causal)


KERNELS: list[KernelSpec] = [
    KernelSpec("naive_online", _entry("naive_attention_forward"), _simt_support((64, 128))),
    # bfloat16 SDPA on the device is left out (the reference offers it for every
    # workload, benchmarks/kernels.py:148-152): torch's bf16 batched products with a
    # transposed right operand, which SDPA's math path issues, are listed by the GPU
    # pool this runs on as faulting its GPUs. This harness has never run that call.
    KernelSpec("pytorch_sdpa", _sdpa, lambda w: w.dtype in (torch.float16, torch.float32)),
    KernelSpec("block_online", _entry("block_attention_forward"), _simt_support((64, 128))),
    KernelSpec("tiled_simt", _entry("tiled_attention_forward"), _simt_support((64,))),
    KernelSpec("tilewise_simt", _entry("tilewise_attention_forward"), _simt_support((64,))),
    KernelSpec("tensorcore_attention", _entry("tensorcore_attention_forward"),
               _tensorcore_support(16)),
    KernelSpec("tensorcore_attention_bc32", _entry("tensorcore_attention_forward_bc32"),
               _tensorcore_support(32)),
    KernelSpec("tensorcore_bc32_raw_pv", _entry("tensorcore_attention_forward_bc32_raw_pv"),
               _tensorcore_support(32)),
    KernelSpec("tensorcore_bc32_raw_qk_raw_pv",
               _entry("tensorcore_attention_forward_bc32_raw_qk_raw_pv"), _tensorcore_support(32)),
    KernelSpec("tensorcore_production_128x128", _production,
               lambda w: _square_fp16_d64(w) and w.query_length % 128 == 0),
    KernelSpec("pytorch_sdpa_cpu", _CpuSdpa(), lambda w: True, on_device=False),
]


def find_kernel(name: str) -> KernelSpec:
    for spec in KERNELS:
        if spec.name == name:
            return spec
    raise KeyError(name)
