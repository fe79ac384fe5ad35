"""Device buffers for the Python host layer.

``DeviceBuffer`` stands in for the reference's ``cuda_core::DeviceBuffer<T>``
(typed device memory with ``from_host`` / ``zeroed`` / ``to_host_vec``). Device
memory and streams come from PyTorch; tensors are held with a signed dtype of
the same width so that every element type (including u32/u64) round-trips
bit-exactly.
"""
from __future__ import annotations

import numpy as np
import torch

_TORCH_STORAGE = {
    1: torch.uint8,
    2: torch.int16,
    4: torch.int32,
    8: torch.int64,
}
_NP_STORAGE = {1: np.uint8, 2: np.int16, 4: np.int32, 8: np.int64}

KIND_DTYPES = {
    "u32": np.dtype(np.uint32), "i32": np.dtype(np.int32), "f32": np.dtype(np.float32),
    "u64": np.dtype(np.uint64), "i64": np.dtype(np.int64), "f64": np.dtype(np.float64),
    "u8": np.dtype(np.uint8), "i8": np.dtype(np.int8), "u16": np.dtype(np.uint16),
    "i16": np.dtype(np.int16),
}


def kind_of(dtype) -> str:
    dtype = np.dtype(dtype)
    for k, d in KIND_DTYPES.items():
        if d == dtype:
            return k
    raise TypeError(f"no key kind for dtype {dtype}")


def _storage_dtype(itemsize: int):
    if itemsize in _TORCH_STORAGE:
        return _TORCH_STORAGE[itemsize], _NP_STORAGE[itemsize]
    if itemsize == 16:
        return torch.int64, np.int64
    raise TypeError(f"unsupported element size {itemsize}")


class DeviceBuffer:
    """Typed device allocation of ``len`` elements of numpy dtype ``dtype``."""

    def __init__(self, tensor: torch.Tensor, dtype, length: int):
        self.tensor = tensor
        self.dtype = np.dtype(dtype)
        self._len = int(length)

    @staticmethod
    def zeroed(dtype, length: int, device: int = 0) -> "DeviceBuffer":
        dtype = np.dtype(dtype)
        tdt, _ = _storage_dtype(dtype.itemsize)
        words = length * dtype.itemsize // torch.empty(0, dtype=tdt).element_size()
        t = torch.zeros(max(words, 1), dtype=tdt, device=f"cuda:{device}")
        return DeviceBuffer(t, dtype, length)

    @staticmethod
    def empty(dtype, length: int, device: int = 0) -> "DeviceBuffer":
        dtype = np.dtype(dtype)
        tdt, _ = _storage_dtype(dtype.itemsize)
        words = length * dtype.itemsize // torch.empty(0, dtype=tdt).element_size()
        t = torch.empty(max(words, 1), dtype=tdt, device=f"cuda:{device}")
        return DeviceBuffer(t, dtype, length)

    @staticmethod
    def from_host(array, dtype=None, device: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(array if dtype is None else np.asarray(array, dtype=dtype))
        tdt, ndt = _storage_dtype(a.dtype.itemsize)
        if a.size == 0:
            return DeviceBuffer(torch.zeros(1, dtype=tdt, device=f"cuda:{device}"), a.dtype, 0)
        host = torch.from_numpy(a.view(ndt).reshape(-1))
        return DeviceBuffer(host.to(f"cuda:{device}"), a.dtype, a.size)

    @staticmethod
    def bytes(nbytes: int, device: int = 0) -> "DeviceBuffer":
        t = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=f"cuda:{device}")
        return DeviceBuffer(t, np.uint8, int(nbytes))

    def len(self) -> int:
        return self._len

    def __len__(self) -> int:
        return self._len

    @property
    def nbytes(self) -> int:
        return self._len * self.dtype.itemsize

    @property
    def ptr(self) -> int:
        return self.tensor.data_ptr()

    def to_host_vec(self) -> np.ndarray:
        if self._len == 0:
            return np.empty(0, dtype=self.dtype)
        h = self.tensor.cpu().numpy()
        return h.view(self.dtype)[: self._len].copy()

    def copy_from(self, other: "DeviceBuffer") -> None:
        """Device-to-device copy of ``other`` into this buffer (same size)."""
        self.tensor.copy_(other.tensor)

    def clone(self) -> "DeviceBuffer":
        return DeviceBuffer(self.tensor.clone(), self.dtype, self._len)
