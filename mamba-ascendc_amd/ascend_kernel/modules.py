"""Module-level caller of the SSD op, as the reference's models use it.

The reference's Vision-Mamba2 blocks call the SSD through one small module
(mamba_torch/vmamba2_network.py:31-87, ``SsdCore``): it is built with a backend
name, binds the op on its first call from the input's device, and always calls
it with D, z, dt_bias and the softplus discretisation, returning the output
tensor alone.  This module keeps that constructor and call signature, so a model
written against the reference runs unchanged.  On this build every backend name
binds to this package's ``mamba2_ssd_fwd`` for ROCm tensors (``device.type ==
"cuda"``); the reference's "cuda" backend would import mamba_ssm, which has no
MI355X build, and its "reference" backend is the CPU oracle, which is test
infrastructure here and not offered.  The reference's own module, built with
``backend="npu"``, lands on this package too, since its "npu" branch imports
``ascend_kernel``.
"""

from __future__ import annotations

from typing import Callable, Optional

import torch
from torch import nn

from .mamba2 import mamba2_ssd_fwd

_BACKENDS = ("auto", "cuda", "rocm", "npu")


class SsdCore(nn.Module):
    """The SSD op as a model block calls it: ``forward(x, dt, A, B, C,
    chunk_size, D, z, dt_bias) -> out`` with dt discretised by softplus."""

    def __init__(self, backend: str = "auto") -> None:
        super().__init__()
        if backend not in _BACKENDS:
            raise ValueError(f"SsdCore: backend {backend!r} is not one of {', '.join(_BACKENDS)}")
        self.backend = backend
        self._op: Optional[Callable] = None

    @staticmethod
    def _bind(device_type: str) -> Callable:
        if device_type != "cuda":
            raise RuntimeError(f"SsdCore: no SSD kernel for {device_type!r} tensors "
                               "(this build runs on ROCm GPUs)")
        return mamba2_ssd_fwd

    def forward(self, x: torch.Tensor, dt: torch.Tensor, A: torch.Tensor, B: torch.Tensor,
                C: torch.Tensor, chunk_size: int, D: torch.Tensor, z: torch.Tensor,
                dt_bias: torch.Tensor) -> torch.Tensor:
        if self._op is None:
            self._op = self._bind(x.device.type)
        result = self._op(x, dt, A, B, C, chunk_size, D=D, z=z, dt_bias=dt_bias, dt_softplus=True)
        # mamba2_ssd_fwd returns a tuple only when a final state is asked for
        return result if torch.is_tensor(result) else result[0]
