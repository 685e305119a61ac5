"""GGUF reader and device weight upload: Ferrum's gguf::load / GgufModel over the C ABI.

``GgufFile(path)`` is ``gguf::load(path)`` (crates/gguf/src/parse.rs:53-64): the file is
memory-mapped and decoded by libferrum_kv.so with the reference's checks, order and
messages (``GgufError``, "gguf: ..."). ``version``, ``alignment``, ``metadata_len``,
``tensors``, ``tensor(name)``, ``metadata(key)`` and ``dump()`` follow the ``GgufModel``
trait (crates/core-types/src/source.rs:58-68). ``upload(dst)`` copies the tensor data
section into a device buffer through pinned staging, every tensor at its data_offset;
``device_tensor(dst, name)`` is then the tensor's bytes in HBM, the same bytes
``tensor_bytes`` borrows from the map.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Tuple

from . import _lib
from .errors import check

__all__ = ["GgufFile", "GgufTensor", "GGML_TYPE_NAMES"]

GGML_TYPE_NAMES = {
    0: "f32", 1: "f16", 2: "q4_0", 3: "q4_1", 4: "q4_2", 5: "q4_3", 6: "q5_0", 7: "q5_1",
    8: "q8_0", 9: "q8_1", 10: "q2_K", 11: "q3_K", 12: "q4_K", 13: "q5_K", 14: "q6_K",
    15: "q8_K", 16: "iq2_xxs", 17: "iq2_xs", 18: "iq3_xxs", 19: "iq1_s", 20: "iq4_nl",
    21: "iq3_s", 22: "iq2_s", 23: "iq4_xs", 24: "i8", 25: "i16", 26: "i32", 27: "i64",
    28: "f64", 29: "iq1_m", 30: "bf16", 34: "tq1_0", 35: "tq2_0", 39: "mxfp4",
}


@dataclass(frozen=True)
class GgufTensor:
    """TensorDesc (source.rs:13-22): shape in GGUF order, shape[0] contiguous."""
    name: str
    shape: Tuple[int, ...]
    ggml_type: int
    data_offset: int
    nbytes: int


class GgufFile:
    def __init__(self, path: str):
        self._lib = _lib.load()
        h = ctypes.c_void_p()
        check(self._lib.fkv_gguf_open(str(path).encode(), ctypes.byref(h)))
        self._h = h
        v, a = ctypes.c_uint32(), ctypes.c_uint64()
        nm, nt, ds, db = (ctypes.c_uint64() for _ in range(4))
        check(self._lib.fkv_gguf_info(self._h, ctypes.byref(v), ctypes.byref(a), ctypes.byref(nm),
                                      ctypes.byref(nt), ctypes.byref(ds), ctypes.byref(db)))
        self.version, self.alignment = v.value, a.value
        self.metadata_len, self.data_start, self.data_bytes = nm.value, ds.value, db.value
        self.tensors = []
        for i in range(nt.value):
            t = _lib.GgufTensorInfoC()
            check(self._lib.fkv_gguf_tensor(self._h, i, ctypes.byref(t)))
            self.tensors.append(GgufTensor(ctypes.string_at(t.name, t.name_len).decode(),
                                           tuple(t.shape[:t.n_dims]), t.ggml_type,
                                           t.data_offset, t.nbytes))

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.fkv_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def tensor(self, name: str) -> GgufTensor:
        """GgufModel::tensor: "gguf: missing tensor <name>" when absent."""
        i = ctypes.c_uint64()
        b = name.encode()
        check(self._lib.fkv_gguf_find(self._h, b, len(b), ctypes.byref(i)))
        return self.tensors[i.value]

    def _value(self, v, key: str, elem_of: Optional[str] = None):
        if v.type == 9:  # array
            return [self._array_elem(key, i) for i in range(v.count)] if elem_of is None else \
                ("array", v.elem_type, v.count)
        if v.type == 8:
            return ctypes.string_at(v.str, v.str_len).decode()
        if v.type in (6, 12):
            return v.f
        if v.type == 7:
            return bool(v.u)
        if v.type in (1, 3, 5, 11):
            return v.i
        return v.u

    def _array_elem(self, key: str, i: int):
        v = _lib.GgufValueC()
        b = key.encode()
        check(self._lib.fkv_gguf_meta_array_elem(self._h, b, len(b), i, ctypes.byref(v)))
        return self._value(v, key, elem_of=key)

    def metadata(self, key: str):
        """The value (int, float, bool, str or list), or None when the key is absent
        (GgufModel::metadata returns Option). Nested arrays show as ("array", type, n)."""
        v = _lib.GgufValueC()
        b = key.encode()
        if self._lib.fkv_gguf_meta(self._h, b, len(b), ctypes.byref(v)) != 0:
            return None
        return self._value(v, key)

    def metadata_type(self, key: str) -> Optional[int]:
        v = _lib.GgufValueC()
        b = key.encode()
        if self._lib.fkv_gguf_meta(self._h, b, len(b), ctypes.byref(v)) != 0:
            return None
        return v.type

    def dump(self) -> str:
        """GgufModel::dump (format_gguf_dump, source.rs:70-92)."""
        n = ctypes.c_uint64()
        check(self._lib.fkv_gguf_dump(self._h, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(n.value + 1)
        check(self._lib.fkv_gguf_dump(self._h, buf, n.value + 1, ctypes.byref(n)))
        return buf.value.decode()

    def upload(self, dst, chunk_bytes: int = 0, threads: int = 0) -> None:
        """Copy the data section into dst (a uint8 device tensor of >= data_bytes)."""
        import torch
        if not isinstance(dst, torch.Tensor) or not dst.is_cuda or dst.dtype != torch.uint8:
            raise TypeError("dst must be a uint8 device tensor")
        check(self._lib.fkv_gguf_upload(self._h, dst.data_ptr(), dst.numel(), chunk_bytes,
                                        threads))

    def device_tensor(self, dst, name: str):
        """The tensor's bytes inside an uploaded buffer (a uint8 view)."""
        t = self.tensor(name)
        return dst[t.data_offset: t.data_offset + t.nbytes]
