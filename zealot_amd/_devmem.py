"""Torch tensors that alias device memory owned by the C library."""
from __future__ import annotations

import torch

_TYPESTR = {torch.float32: ("<f4", None), torch.bfloat16: ("<u2", torch.bfloat16),
            torch.uint8: ("|u1", None)}
if hasattr(torch, "float8_e4m3fn"):
    _TYPESTR[torch.float8_e4m3fn] = ("|u1", torch.float8_e4m3fn)


class _DeviceArray:
    """__cuda_array_interface__ holder; keeps the owning object alive."""

    def __init__(self, ptr: int, shape, typestr: str, owner):
        self._owner = owner
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": typestr,
                                         "data": (int(ptr), False), "version": 2, "strides": None}


def tensor_from_device_ptr(ptr: int, shape, dtype, owner=None) -> torch.Tensor:
    typestr, view = _TYPESTR[dtype]
    t = torch.as_tensor(_DeviceArray(ptr, shape, typestr, owner), device="cuda")
    return t.view(view) if view is not None else t
