"""numpy restatement of the reference's safetensors reader — TEST INFRASTRUCTURE ONLY.

Follows SafetensorsFile (src/runtime/weights.ts:58-194):
  read_header   weights.ts:67-99   8-byte little-endian length, JSON header, __metadata__ split
                                   off, data block at 8 + length
  read_raw      weights.ts:125-142 the bytes data[begin, end)
  read_f32      weights.ts:150-177 F32 as stored, BF16 bits << 16, F16 via f16_to_f32_bits
  f16_to_f32_bits  weights.ts:28-56 field-by-field IEEE half -> float (subnormals normalised,
                                   NaN -> sign | 0x7fc00000), restated with integer numpy ops
and adds the narrowing conversions the device loader offers (float -> bf16 / f16, round to
nearest even, NaN -> sign | canonical quiet NaN), written from the IEEE 754 definition.

Pinning (tests/test_oracle.py): read_header / read_raw against the `safetensors` package's own
reader on files it wrote; f16_to_f32_bits against numpy's float16 -> float32 cast over all 65536
half patterns (NaNs compared as canonical); bf16 widening against torch's bfloat16 -> float32 over
all 65536 patterns; f32_to_bf16_bits against torch's float32 -> bfloat16 cast and
f32_to_f16_bits against numpy's float32 -> float16 cast on ties, subnormals, overflow and random
values.
"""
from __future__ import annotations

import json
import struct

import numpy as np

# header dtype -> numpy dtype of the stored elements
NP_OF_ST = {
    "F32": "<f4", "F16": "<f2", "BF16": "<u2", "F64": "<f8", "I64": "<i8", "I32": "<i4",
    "I16": "<i2", "I8": "i1", "U8": "u1", "BOOL": "?", "U16": "<u2", "U32": "<u4", "U64": "<u8",
    "F8_E4M3": "u1", "F8_E5M2": "u1",
}
SIZE_OF_ST = {k: np.dtype(v).itemsize for k, v in NP_OF_ST.items()}


def read_header(path):
    """(metadata dict, {name: (dtype, shape tuple, (begin, end))} in header order, data offset)."""
    with open(path, "rb") as f:
        (n,) = struct.unpack("<Q", f.read(8))
        raw = json.loads(f.read(n).decode())
    meta = raw.pop("__metadata__", {}) or {}
    tensors = {k: (v["dtype"], tuple(v["shape"]), tuple(v["data_offsets"])) for k, v in raw.items()}
    return meta, tensors, 8 + n


def read_raw(path, name) -> np.ndarray:
    """The stored bytes of one tensor as uint8."""
    _, tensors, data = read_header(path)
    b, e = tensors[name][2]
    with open(path, "rb") as f:
        f.seek(data + b)
        return np.frombuffer(f.read(e - b), np.uint8).copy()


def f16_to_f32_bits(h) -> np.ndarray:
    """IEEE half bit patterns (uint16) -> float32 bit patterns (uint32), field by field."""
    h = np.asarray(h, np.uint32)
    s = (h & 0x8000) << 16
    e = (h >> 10) & 0x1F
    m = h & 0x3FF
    out = s | ((e + 112) << 23) | (m << 13)  # normal: exponent rebias 15 -> 127
    sub = (e == 0) & (m != 0)
    if sub.any():
        ms = m[sub].astype(np.int64)
        lead = np.floor(np.log2(ms)).astype(np.int64)  # position of the leading one, 0..9
        mant = (ms << (10 - lead)) & 0x3FF
        exp = lead - 24 + 127  # value = ms * 2^-24
        out[sub] = s[sub] | (exp.astype(np.uint32) << 23) | (mant.astype(np.uint32) << 13)
    out[(e == 0) & (m == 0)] = s[(e == 0) & (m == 0)]
    out[(e == 31) & (m == 0)] = s[(e == 31) & (m == 0)] | 0x7F800000
    out[(e == 31) & (m != 0)] = s[(e == 31) & (m != 0)] | 0x7FC00000
    return out.astype(np.uint32)


def bf16_to_f32_bits(b) -> np.ndarray:
    return np.asarray(b, np.uint32) << 16


def f32_to_bf16_bits(x) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even; NaN -> sign | 0x7fc0."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, np.float32))
    r[nan] = ((u[nan] >> 16) & 0x8000).astype(np.uint16) | 0x7FC0
    return r


def f32_to_f16_bits(x) -> np.ndarray:
    """float32 -> IEEE half bit patterns, round to nearest even (subnormal halves kept, overflow to
    infinity); NaN -> sign | 0x7e00.  Written from the definition, not through numpy's cast."""
    x = np.asarray(x, np.float32)
    u = x.view(np.uint32).astype(np.int64)
    s = ((u >> 16) & 0x8000).astype(np.int64)
    a = u & 0x7FFFFFFF
    e = (a >> 23) - 127  # unbiased exponent of the float
    m = (a & 0x7FFFFF) | 0x800000  # 24-bit significand with the implicit one
    out = np.zeros_like(u)
    # shift so that the result is an integer count of half ulps at the target exponent
    # normal half: exponent -14..15, 10 fraction bits -> keep 11 bits: shift 13
    # subnormal half: value / 2^-24, shift 13 + (-14 - e)
    shift = np.where(e >= -14, 13, 13 + (-14 - e))
    big = shift > 40
    shift = np.minimum(shift, 40)
    q = m >> shift
    rem = m & ((1 << shift) - 1)
    half = 1 << (shift - 1)
    q = q + ((rem > half) | ((rem == half) & ((q & 1) == 1)))
    q[big] = 0
    normal = e >= -14
    # normal: q holds 11 bits (may carry to 12); exponent field = e + 15 (+1 on carry)
    en = np.where(q >= 2048, e + 16, e + 15)
    qn = np.where(q >= 2048, q >> 1, q)
    val_n = (en << 10) | (qn & 0x3FF)
    val_s = q  # subnormal: q counts 2^-24 units (a carry to 1024 is the smallest normal)
    out = np.where(normal, val_n, val_s)
    out = np.where(normal & (en >= 31), 0x7C00, out)  # overflow -> infinity
    out = np.where(a == 0, 0, out)
    out = np.where(a == 0x7F800000, 0x7C00, out)
    out = np.where(a > 0x7F800000, 0x7E00, out)
    return (s | out).astype(np.uint16)


def widen_f32_bits(raw: np.ndarray, dtype: str) -> np.ndarray:
    """readTensorF32 of a float tensor's bytes, as float32 bit patterns."""
    if dtype == "F32":
        return raw.view("<u4").astype(np.uint32)
    if dtype == "BF16":
        return bf16_to_f32_bits(raw.view("<u2"))
    if dtype == "F16":
        return f16_to_f32_bits(raw.view("<u2"))
    raise ValueError(f"{dtype} is not a float type")


def read_f32(path, name) -> np.ndarray:
    """readTensorF32: float32 array with the tensor's shape."""
    _, tensors, _ = read_header(path)
    dtype, shape, _ = tensors[name]
    return widen_f32_bits(read_raw(path, name), dtype).view(np.float32).reshape(shape)


def convert_bits(raw: np.ndarray, src: str, dst: str) -> np.ndarray:
    """A float tensor's bytes converted to dst ("F32", "F16", "BF16") bit patterns."""
    if src == dst:
        return raw.view({"F32": "<u4", "F16": "<u2", "BF16": "<u2"}[dst]).copy()
    wide = widen_f32_bits(raw, src)
    if dst == "F32":
        return wide
    f = wide.view(np.float32)
    return f32_to_bf16_bits(f) if dst == "BF16" else f32_to_f16_bits(f)
