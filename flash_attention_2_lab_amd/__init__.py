"""MI355X-native FlashAttention-2 forward (FP16, head_dim 64, causal or not).

Drop-in for the operator surface of joshprinzel/flash_attention_2_lab:

* ``flash_attention_cuda`` - the PyTorch operator module, same name and operators as
  the reference's: the tensor-core attention forwards (the hot path,
  ``tensorcore_attention_forward_production_128x128`` and the four Bc=16/32
  entries) and the module's other operators (copy, FP32 scores and forwards, the
  16x64x16 FP16 product). Importing this package also registers it under the
  top-level name ``flash_attention_cuda`` so the reference's callers
  (``benchmarks/kernels.py``, ``tests/``) import it unchanged.
* ``capi`` - a ctypes binding of the C ABI in ``include/fa2_mi355x.h``.
* ``benchmarks`` - the counterpart of the reference's benchmark harness.

The compute path is hand-written HIP for gfx950 (``csrc/fa2_forward.hip``,
``csrc/fa2_aux.hip``); there is no CPU or PyTorch fallback. If the built libraries are missing the import fails;
build them with ``python flash_attention_2_lab_amd/_build.py``.
"""

from __future__ import annotations

import sys

# torch first: its bundled HIP runtime (same soname as ROCm's) is then the one the
# kernel library binds to, so the process holds a single HIP runtime.
import torch  # noqa: F401

try:
    from . import flash_attention_cuda
except ImportError as exc:  # pragma: no cover - exercised only on an unbuilt tree
    raise ImportError(
        "flash_attention_2_lab_amd: the HIP extension is not built "
        "(run `python flash_attention_2_lab_amd/_build.py`)"
    ) from exc

from . import capi

sys.modules.setdefault("flash_attention_cuda", flash_attention_cuda)

tensorcore_attention_forward_production_128x128 = (
    flash_attention_cuda.tensorcore_attention_forward_production_128x128
)

__all__ = [
    "capi",
    "flash_attention_cuda",
    "tensorcore_attention_forward_production_128x128",
]
