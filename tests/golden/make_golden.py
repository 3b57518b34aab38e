"""Writes tests/golden/attention_fp16_d64.npz - fixed input/output vectors.

Inputs are FP16 Q, K, V drawn from one seeded CPU torch.Generator in the order
q, k, v (the order of reference benchmarks/workloads.py:56-89); "sigma2" cases
multiply Q and K by 2 after drawing (the large-logit case of the benchmark
configurations). Expected outputs are the float64 row-wise evaluation of
softmax(Q K^T / 8 [+ causal mask]) V (oracle.attention_float64_rowwise), stored
in float32. The reference ships no fixtures of its own for this path.

Run from the repository root: python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import attention_float64_rowwise  # noqa: E402

OUT = Path(__file__).resolve().parent / "attention_fp16_d64.npz"

# name -> (batch, heads, seq_len, seed, sigma, modes)
CASES = {
    "b1h1n128": (1, 1, 128, 0, 1.0, ("noncausal", "causal")),
    "b1h2n128": (1, 2, 128, 1, 1.0, ("noncausal", "causal")),
    "b1h1n256_sigma2": (1, 1, 256, 2, 2.0, ("causal",)),
}


def make_inputs(batch: int, heads: int, seq_len: int, seed: int, sigma: float):
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    shape = (batch, heads, seq_len, 64)
    q = torch.randn(shape, generator=gen, dtype=torch.float32)
    k = torch.randn(shape, generator=gen, dtype=torch.float32)
    v = torch.randn(shape, generator=gen, dtype=torch.float32)
    return (q * sigma).half(), (k * sigma).half(), v.half()


def main() -> None:
    arrays: dict[str, np.ndarray] = {}
    for name, (b, h, n, seed, sigma, modes) in CASES.items():
        q, k, v = make_inputs(b, h, n, seed, sigma)
        arrays[f"{name}/query"] = q.numpy()
        arrays[f"{name}/key"] = k.numpy()
        arrays[f"{name}/value"] = v.numpy()
        for mode in modes:
            expected = attention_float64_rowwise(q, k, v, causal=(mode == "causal"))
            arrays[f"{name}/{mode}"] = expected.astype(np.float32)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()
