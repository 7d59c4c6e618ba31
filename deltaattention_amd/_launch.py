"""Kernel objects that accept the reference's Triton launch syntax.

``kernel[grid](*args, **meta)`` binds arguments by the parameter names of the
reference kernel (the same way Triton binds them), checks what the native kernels
assume (bf16 data, contiguous head dimension, the 128x128 logical blocks), and calls
libdeltaattn.so.  ``num_warps`` / ``num_stages`` are accepted and ignored: tiling is
fixed by the HIP kernels.
"""
from __future__ import annotations

from typing import Dict, Sequence

import torch

_IGNORED_META = ("num_warps", "num_stages", "num_ctas", "maxnreg")


class KernelLauncher:
    """Base class: subclasses define PARAMS (the reference signature) and launch()."""

    PARAMS: Sequence[str] = ()
    NAME = "kernel"

    def __getitem__(self, grid):
        if callable(grid):
            raise TypeError(f"{self.NAME}: grid callables are not supported; pass a tuple")
        grid = tuple(int(g) for g in grid) + (1,) * (3 - len(tuple(grid)))

        def run(*args, **kwargs):
            return self.launch(grid, self.bind(args, kwargs))
        return run

    def bind(self, args, kwargs) -> Dict[str, object]:
        if len(args) > len(self.PARAMS):
            raise TypeError(f"{self.NAME}: {len(args)} positional arguments, expected at most "
                            f"{len(self.PARAMS)}")
        bound = dict(zip(self.PARAMS, args))
        for k, v in kwargs.items():
            if k in _IGNORED_META:
                continue
            if k not in self.PARAMS:
                raise TypeError(f"{self.NAME}: unexpected argument {k!r}")
            if k in bound:
                raise TypeError(f"{self.NAME}: argument {k!r} given twice")
            bound[k] = v
        missing = [p for p in self.PARAMS if p not in bound]
        if missing:
            raise TypeError(f"{self.NAME}: missing arguments {missing}")
        return bound

    def launch(self, grid, a):  # pragma: no cover - abstract
        raise NotImplementedError


# the 16-bit element types the kernels take (one of them per call)
HALF = (torch.bfloat16, torch.float16)


def tensor(a, name: str, dtype=None) -> torch.Tensor:
    """Argument `name` as a GPU tensor; dtype is one torch dtype or a tuple of them."""
    t = a[name]
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} is on {t.device}; the native kernels take GPU tensors")
    allowed = dtype if isinstance(dtype, tuple) else (dtype,)
    if dtype is not None and t.dtype not in allowed:
        raise TypeError(f"{name} must be {' or '.join(str(d) for d in allowed)}, got {t.dtype}")
    return t


def unit_stride(a, *names) -> None:
    for n in names:
        if int(a[n]) != 1:
            raise ValueError(f"{n} must be 1 (the head dimension must be contiguous)")
