"""Attention workloads (reference benchmarks/workloads.py:9-88).

A workload is the shape, dtype, mask flag and seed of one benchmark case. Inputs are
drawn q, k, v in that order from one generator seeded with ``seed``, as the
reference does. The reference draws on the GPU; ``generate_attention_inputs`` can
draw on the CPU and copy (``generator_device="cpu"``) so that a CPU comparator sees
exactly the same values.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class AttentionWorkload:
    batch: int
    heads: int
    query_length: int
    key_length: int
    head_dimension: int
    dtype: torch.dtype = torch.float32
    causal: bool = False
    seed: int = 0

    @property
    def query_shape(self) -> tuple[int, int, int, int]:
        return (self.batch, self.heads, self.query_length, self.head_dimension)

    @property
    def key_value_shape(self) -> tuple[int, int, int, int]:
        return (self.batch, self.heads, self.key_length, self.head_dimension)

    @property
    def label(self) -> str:
        dtype = str(self.dtype).removeprefix("torch.")
        return (f"B={self.batch}, H={self.heads}, Nq={self.query_length}, Nk={self.key_length}, "
                f"D={self.head_dimension}, dtype={dtype}, causal={self.causal}")


@dataclass
class AttentionInputs:
    query: torch.Tensor
    key: torch.Tensor
    value: torch.Tensor

    def to(self, device: torch.device | str) -> "AttentionInputs":
        return AttentionInputs(self.query.to(device), self.key.to(device), self.value.to(device))


def attention_flops(workload: AttentionWorkload) -> float:
    """Algorithmic FLOPs of one forward: 4*B*H*Nq*Nk*D (QK^T and PV), halved when
    causal (square case), the convention of the throughput figures."""
    flops = 4.0 * workload.batch * workload.heads * workload.query_length * workload.key_length \
        * workload.head_dimension
    return flops / 2.0 if workload.causal else flops


def generate_attention_inputs(workload: AttentionWorkload, *, device: torch.device | str = "cuda",
                              generator_device: torch.device | str | None = None) -> AttentionInputs:
    """Seeded N(0, 1) inputs on `device`; drawn on `generator_device` (default: `device`)."""
    draw_on = torch.device(generator_device if generator_device is not None else device)
    generator = torch.Generator(device=draw_on)
    generator.manual_seed(workload.seed)
    tensors = [torch.randn(shape, device=draw_on, dtype=workload.dtype, generator=generator)
               for shape in (workload.query_shape, workload.key_value_shape, workload.key_value_shape)]
    return AttentionInputs(*(t.to(device).contiguous() for t in tensors))
