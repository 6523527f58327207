"""Safetensors weight files read straight into device tensors (over the tsc_st_* C ABI).

Mirrors the reference's SafetensorsFile and MultiFileLoader (src/runtime/weights.ts:58-237) and
the per-tensor upload of its model loader (src/model/loader.ts:134-162):

  SafetensorsFile(path).open()      header only (8-byte length + JSON); data stays on disk
  .header                           SafetensorsHeader(metadata, tensors, data_byte_offset)
  .tensor_count / .list_tensors()   tensors in header order
  .get_tensors_by_prefix(p)         names starting with p
  .get_tensor_info(name)            TensorEntry(dtype, shape, data_offsets, numel) or None
  .read_tensor_raw(name)            the stored bytes, as a device uint8 tensor
  .read_tensor_f32(name)            readTensorF32: F32 as stored, BF16 bits << 16, F16 widened
  .read_tensor(name, dtype)         F32/F16/BF16 converted on the GPU to dtype (round to nearest
                                    even), or the stored type when dtype is None
  .close()

The reference reads into host memory and converts on the CPU; here each tensor streams through
pinned chunks to the device and is converted there.  Non-float tensors (I64, I32, U8, ...) load
with their stored type only.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field

import torch

from . import _lib
from ._lib import TscError, check

_TORCH_OF_ST = {
    "F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16, "F64": torch.float64,
    "I64": torch.int64, "I32": torch.int32, "I16": torch.int16, "I8": torch.int8,
    "U8": torch.uint8, "BOOL": torch.bool, "U16": torch.uint16, "U32": torch.uint32,
    "U64": torch.uint64, "F8_E4M3": torch.float8_e4m3fn, "F8_E5M2": torch.float8_e5m2,
}
_OUT_CODES = {torch.float32: _lib.TSC_F32, torch.float16: _lib.TSC_F16,
              torch.bfloat16: _lib.TSC_BF16}
_MAX_DIMS = 64


@dataclass(frozen=True)
class TensorEntry:
    """One header entry (weights.ts:11-16): dtype string, shape, byte range in the data block."""

    dtype: str
    shape: tuple
    data_offsets: tuple
    numel: int


@dataclass
class SafetensorsHeader:
    """Parsed header (weights.ts:18-22)."""

    metadata: dict = field(default_factory=dict)
    tensors: dict = field(default_factory=dict)  # name -> TensorEntry, header order
    data_byte_offset: int = 0


class SafetensorsFile:
    """A .safetensors file whose tensors are read on demand into device memory."""

    def __init__(self, path, device=None):
        self.path = os.fspath(path)
        self.device = device
        self._h = None
        self._header = None

    # -- header -------------------------------------------------------------------------------
    def open(self) -> SafetensorsHeader:
        """Open the file and parse its header (weights.ts:67-99); reads no tensor data."""
        lib = _lib.load_library()
        if self._h is not None:
            return self._header
        h = ctypes.c_void_p()
        check(lib.tsc_st_open(self.path.encode(), ctypes.byref(h)))
        self._h = h
        try:
            self._header = self._read_header(lib)
        except Exception:
            self.close()
            raise
        return self._header

    def _read_header(self, lib) -> SafetensorsHeader:
        nt, nm, off = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        check(lib.tsc_st_counts(self._h, ctypes.byref(nt), ctypes.byref(nm), ctypes.byref(off)))
        hdr = SafetensorsHeader(data_byte_offset=off.value)
        for i in range(nm.value):
            k, v = self._strings(lambda kb, kl, vb, vl: lib.tsc_st_metadata(self._h, i, kb, kl, vb, vl))
            hdr.metadata[k] = v
        dt, nd = ctypes.c_int32(), ctypes.c_int32()
        shape = (ctypes.c_int64 * _MAX_DIMS)()
        offs = (ctypes.c_int64 * 2)()
        for i in range(nt.value):
            name = self._string(lambda b, n: lib.tsc_st_name(self._h, i, b, n))
            check(lib.tsc_st_info(self._h, name.encode(), ctypes.byref(dt), ctypes.byref(nd), shape,
                                  _MAX_DIMS, offs))
            shp = tuple(shape[d] for d in range(nd.value))
            numel = 1
            for d in shp:
                numel *= d
            hdr.tensors[name] = TensorEntry(_lib.ST_DTYPES[dt.value], shp, (offs[0], offs[1]), numel)
        return hdr

    @staticmethod
    def _string(call, size=256) -> str:
        while True:
            buf = ctypes.create_string_buffer(size)
            st = call(buf, size)
            if st == _lib.TSC_OK:
                return buf.value.decode()
            if "needs a buffer" not in _lib.load_library().tsc_last_error().decode() or size > 1 << 26:
                check(st)
            size *= 16

    @staticmethod
    def _strings(call, size=256):
        while True:
            kb, vb = ctypes.create_string_buffer(size), ctypes.create_string_buffer(size)
            st = call(kb, size, vb, size)
            if st == _lib.TSC_OK:
                return kb.value.decode(), vb.value.decode()
            if "needs a buffer" not in _lib.load_library().tsc_last_error().decode() or size > 1 << 26:
                check(st)
            size *= 16

    @property
    def header(self) -> SafetensorsHeader:
        if self._header is None:
            raise TscError(_lib.TSC_ERR_INVALID, "file not opened; call open() first")
        return self._header

    @property
    def tensor_count(self) -> int:
        return len(self.header.tensors)

    def list_tensors(self) -> list:
        return list(self.header.tensors)

    def get_tensors_by_prefix(self, prefix: str) -> list:
        return [n for n in self.header.tensors if n.startswith(prefix)]

    def get_tensor_info(self, name: str):
        return self.header.tensors.get(name)

    # -- data ---------------------------------------------------------------------------------
    def _target_device(self, device):
        dev = torch.device(device if device is not None else
                           (self.device if self.device is not None else "cuda"))
        if dev.type != "cuda":
            raise TscError(_lib.TSC_ERR_INVALID, "tensors load to a GPU; this path has no CPU reader")
        return dev.index if dev.index is not None else torch.cuda.current_device()

    def _load(self, name: str, code: int, out: torch.Tensor) -> torch.Tensor:
        if self._h is None:
            raise TscError(_lib.TSC_ERR_INVALID, "file not opened; call open() first")
        ctx = _lib.context(out.device.index)
        with torch.cuda.device(out.device.index):
            check(ctx.lib.tsc_st_load(ctx.bind(), self._h, name.encode(), code,
                                      ctypes.c_void_p(out.data_ptr()) if out.numel() else None))
        return out

    def _entry(self, name: str) -> TensorEntry:
        e = self.header.tensors.get(name)
        if e is None:
            raise TscError(_lib.TSC_ERR_INVALID, f'tensor "{name}" not found')
        return e

    def read_tensor_raw(self, name: str, device=None) -> torch.Tensor:
        """The tensor's stored bytes (weights.ts:125-142) as a flat device uint8 tensor."""
        e = self._entry(name)
        dev = self._target_device(device)
        out = torch.empty(e.data_offsets[1] - e.data_offsets[0], dtype=torch.uint8,
                          device=f"cuda:{dev}")
        return self._load(name, _lib.TSC_ST_RAW, out)

    def read_tensor(self, name: str, dtype=None, device=None) -> torch.Tensor:
        """The tensor with its shape on the device: as stored (dtype None or the stored type), or
        an F32/F16/BF16 tensor converted to dtype float32/float16/bfloat16 on the GPU."""
        e = self._entry(name)
        dev = self._target_device(device)
        stored = _TORCH_OF_ST[e.dtype]
        if dtype is None or dtype == stored:
            out = torch.empty(e.shape, dtype=stored, device=f"cuda:{dev}")
            return self._load(name, _lib.TSC_ST_RAW, out)
        if dtype not in _OUT_CODES:
            raise TscError(_lib.TSC_ERR_INVALID, f"cannot convert to {dtype}")
        out = torch.empty(e.shape, dtype=dtype, device=f"cuda:{dev}")
        return self._load(name, _OUT_CODES[dtype], out)

    def read_tensor_f32(self, name: str, device=None) -> torch.Tensor:
        """readTensorF32 (weights.ts:150-188): F32/F16/BF16 tensors widened to float32 on the
        device (shaped); any other dtype's stored bytes reinterpreted as a flat float32 array, as
        the reference's `new Float32Array(raw)` does (its byte length must be a multiple of 4)."""
        e = self._entry(name)
        if e.dtype in ("F32", "F16", "BF16"):
            return self.read_tensor(name, torch.float32, device)
        raw = self.read_tensor_raw(name, device)
        if raw.numel() % 4:
            raise TscError(_lib.TSC_ERR_INVALID,
                           f"{name}: {raw.numel()} bytes are not a whole number of float32 values")
        return raw.view(torch.float32)

    def get_tensor(self, name: str, device=None) -> torch.Tensor:
        """The model loader's getTensor (loader.ts:154-160): read_tensor_f32 with its shape."""
        return self.read_tensor_f32(name, device)

    def close(self) -> None:
        if self._h is not None:
            _lib.load_library().tsc_st_close(self._h)
        self._h = None
        self._header = None

    def __enter__(self):
        self.open()
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MultiFileLoader:
    """Several safetensors files behind one "label:tensor_name" lookup (weights.ts:196-237)."""

    def __init__(self, device=None):
        self.device = device
        self.files = {}
        self.tensor_to_file = {}

    def add_file(self, file_path, label: str) -> None:
        sf = SafetensorsFile(file_path, self.device)
        sf.open()
        self.files[label] = sf
        for name in sf.list_tensors():
            self.tensor_to_file[f"{label}:{name}"] = label

    def _split(self, label_and_name: str):
        label, _, name = label_and_name.partition(":")
        sf = self.files.get(label)
        if sf is None:
            raise TscError(_lib.TSC_ERR_INVALID, f'file "{label}" not found')
        return sf, name

    def read_tensor(self, label_and_name: str) -> torch.Tensor:
        """The stored bytes of "label:name" (readTensor, weights.ts:215-223), device uint8."""
        sf, name = self._split(label_and_name)
        return sf.read_tensor_raw(name)

    def read_tensor_as(self, label_and_name: str, dtype=None) -> torch.Tensor:
        """SafetensorsFile.read_tensor of "label:name": shaped, optionally converted."""
        sf, name = self._split(label_and_name)
        return sf.read_tensor(name, dtype)

    def close_all(self) -> None:
        for sf in self.files.values():
            sf.close()
        self.files.clear()
        self.tensor_to_file.clear()
