"""GGUF files through the library's loader (include/qwen35_gguf.h).

`GgufFile(path)` parses the file (metadata, tensor infos, range checks) in the
C library; `load()` uploads the tensors to device memory, after which
`tensor(name)` returns a torch uint8 tensor aliasing the tensor's device bytes
(valid until `unload()` / `close()`).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

from ._lib import QwenError, check, load


class _Info(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint32), ("tensor_count", ctypes.c_uint64),
                ("metadata_count", ctypes.c_uint64), ("payload_offset", ctypes.c_uint64),
                ("device_bytes", ctypes.c_uint64)]


class _Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_uint32), ("n_dims", ctypes.c_uint32),
                ("shape", ctypes.c_int64 * 4), ("num_elements", ctypes.c_uint64), ("size_bytes", ctypes.c_uint64),
                ("offset", ctypes.c_uint64), ("device_ptr", ctypes.c_void_p)]


@dataclass
class TensorInfo:
    name: str
    type: int
    shape: tuple
    num_elements: int
    size_bytes: int
    offset: int
    device_ptr: int | None


class _DeviceBytes:
    """__cuda_array_interface__ view of device memory owned by the loader."""

    def __init__(self, ptr: int, nbytes: int):
        self.__cuda_array_interface__ = {"shape": (nbytes,), "typestr": "|u1", "data": (ptr, False),
                                         "version": 2, "strides": None}


class GgufFile:
    def __init__(self, path: str):
        self._lib = load()
        self._h = ctypes.c_void_p()
        check(self._lib.qwen_gguf_open(str(path).encode(), ctypes.byref(self._h)))

    def close(self) -> None:
        if self._h:
            self._lib.qwen_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self) -> dict:
        i = _Info()
        check(self._lib.qwen_gguf_get_info(self._h, ctypes.byref(i)))
        return {f: getattr(i, f) for f, _ in _Info._fields_}

    def tensors(self) -> list[TensorInfo]:
        out = []
        for k in range(self.info()["tensor_count"]):
            t = _Tensor()
            check(self._lib.qwen_gguf_get_tensor(self._h, k, ctypes.byref(t)))
            out.append(TensorInfo(t.name.decode(), t.type, tuple(t.shape[:t.n_dims]), t.num_elements, t.size_bytes,
                                  t.offset, t.device_ptr))
        return out

    def find(self, name: str) -> int:
        idx = ctypes.c_int64()
        check(self._lib.qwen_gguf_find_tensor(self._h, name.encode(), ctypes.byref(idx)))
        return idx.value

    def meta(self, key: str) -> str | None:
        v = ctypes.c_char_p()
        check(self._lib.qwen_gguf_get_meta(self._h, key.encode(), ctypes.byref(v)))
        return None if v.value is None else v.value.decode()

    def meta_array(self, key: str) -> list[str] | None:
        n = ctypes.c_int64()
        check(self._lib.qwen_gguf_get_meta_array_size(self._h, key.encode(), ctypes.byref(n)))
        if n.value < 0:
            return None
        out = []
        for i in range(n.value):
            v = ctypes.c_char_p()
            check(self._lib.qwen_gguf_get_meta_array_item(self._h, key.encode(), i, ctypes.byref(v)))
            out.append(v.value.decode())
        return out

    def keys(self) -> list[tuple[str, bool]]:
        out = []
        for i in range(self.info()["metadata_count"]):
            k, a = ctypes.c_char_p(), ctypes.c_int()
            check(self._lib.qwen_gguf_get_meta_key(self._h, i, ctypes.byref(k), ctypes.byref(a)))
            out.append((k.value.decode(), bool(a.value)))
        return out

    def load(self, base_layer_count: int = -1, stream=None) -> None:
        check(self._lib.qwen_gguf_load(self._h, base_layer_count, stream))

    def unload(self) -> None:
        check(self._lib.qwen_gguf_unload(self._h))

    def tensor(self, name: str):
        """torch uint8 tensor aliasing the loaded device bytes of `name`."""
        import torch

        k = self.find(name)
        if k < 0:
            raise KeyError(name)
        t = self.tensors()[k]
        if not t.device_ptr:
            raise QwenError(0, f"tensor {name} is not loaded")
        return torch.as_tensor(_DeviceBytes(t.device_ptr, t.size_bytes), device="cuda")
