"""Module-level caller of the SSD op, as the reference's models use it.

``SsdCore`` keeps the constructor and forward of the reference's backend-neutral
call boundary (mamba_torch/vmamba2_network.py:31-87): a module that resolves the
SSD op once from the input's device and calls it with D, z, dt_bias and
``dt_softplus=True``, returning only the output.  Here a ROCm tensor
(``device.type == "cuda"``) resolves to this package's ``mamba2_ssd_fwd`` (the
reference sends "cuda" to mamba_ssm, which has no MI355X build); "reference"
is not offered, since the CPU oracle is test infrastructure.  The reference's
own SsdCore(backend="npu") also lands here unchanged, because its "npu" branch
imports ``ascend_kernel`` (this package's import name).
"""

from __future__ import annotations

from typing import Callable, Optional

import torch
from torch import nn

from .mamba2 import mamba2_ssd_fwd


class SsdCore(nn.Module):
    """Backend-neutral ``mamba_chunk_scan_combined`` call boundary."""

    def __init__(self, backend: str = "auto") -> None:
        super().__init__()
        if backend not in {"auto", "cuda", "rocm", "npu"}:
            raise ValueError(f"unsupported SSD backend: {backend}")
        self.backend = backend
        self._op: Optional[Callable] = None

    def _resolve(self, device_type: str) -> Callable:
        if device_type != "cuda":
            raise RuntimeError(f"SsdCore: no SSD backend for device type {device_type!r} "
                               "(this build runs on ROCm GPUs)")
        return mamba2_ssd_fwd

    def forward(self, x: torch.Tensor, dt: torch.Tensor, A: torch.Tensor, B: torch.Tensor,
                C: torch.Tensor, chunk_size: int, D: torch.Tensor, z: torch.Tensor,
                dt_bias: torch.Tensor) -> torch.Tensor:
        if self._op is None:
            self._op = self._resolve(x.device.type)
        output = self._op(x, dt, A, B, C, chunk_size, D=D, z=z, dt_bias=dt_bias, dt_softplus=True)
        return output[0] if isinstance(output, tuple) else output
