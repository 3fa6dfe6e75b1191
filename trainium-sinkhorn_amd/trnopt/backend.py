"""Device settings for the solver, chosen once and passed in SinkhornOptions.backend.

Same interface as the reference's Backend (src/trnopt/backend.py:23-72): a frozen dataclass with device,
dtype, compile and compile_backend, named presets with keyword overrides, compile_fn() and tensor().

Presets kept from the reference: "cpu" (float64), "cpu-float32", "cuda", "neuron", "emulate-neuron", "mps".
Added: "rocm" -- the AMD GPU through PyTorch-ROCm (whose device string is "cuda"), float32, no torch.compile.
With kernel="auto" (or "hip") sinkhorn() runs its half-steps and its whole iteration loop in the fused HIP
kernels of hip_sinkhorn.py on this preset; kernel="torch" runs the plain PyTorch half-step on the GPU.
"""

from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np
import torch

_compiled: dict = {}      # (function, compiler, dynamic) -> compiled function, for the process lifetime


@dataclass(frozen=True)
class Backend:
    device: str = "cpu"
    dtype: torch.dtype = torch.float64
    compile: bool = False
    compile_backend: str | None = None       # None: PyTorch's default compiler for the device

    @classmethod
    def preset(cls, name: str, **overrides) -> "Backend":
        """A named starting point; any field can be overridden, e.g. Backend.preset("rocm", compile=True)."""
        table = {
            "cpu": cls(),
            "cpu-float32": cls(dtype=torch.float32),
            "cuda": cls(device="cuda"),
            "rocm": cls(device="cuda", dtype=torch.float32),
            "neuron": cls(device="neuron", dtype=torch.float32, compile=True, compile_backend="neuron"),
            "emulate-neuron": cls(device="cpu", dtype=torch.float32, compile=True),
            "mps": cls(device="mps", dtype=torch.float32),
        }
        if name not in table:
            raise ValueError(f"unknown backend preset {name!r}; choose from {sorted(table)}")
        return replace(table[name], **overrides)

    @property
    def is_rocm_gpu(self) -> bool:
        """A GPU device of a ROCm build of PyTorch that is present (where the fused HIP kernels run)."""
        return (self.device.startswith("cuda") and torch.version.hip is not None
                and torch.cuda.is_available())

    def compile_fn(self, f):
        """f through torch.compile when this backend compiles, else f itself. One compiled function per
        (function, compiler) for the whole process: pass problem data as arguments. (The Neuron presets' static
        shape mode has no device to run on here; torch.compile picks its own shape mode.)"""
        if not self.compile:
            return f
        key = (f, self.compile_backend or "inductor")
        fn = _compiled.get(key)
        if fn is None:
            fn = _compiled[key] = torch.compile(f, backend=key[1])
        return fn

    def tensor(self, a) -> torch.Tensor:
        """a as a tensor of this backend's dtype on its device (converted on the host first)."""
        return torch.as_tensor(np.asarray(a), dtype=self.dtype).to(self.device)
