"""Safetensors reading on the CPU: the oracle's conversions and reader pinned against numpy, torch
and the `safetensors` package, and the native header parser (tsc_st_open / counts / name /
metadata / info, no GPU call) against both."""
import json
import struct

import numpy as np
import pytest
import torch
from safetensors.numpy import load_file, save_file

from oracle import st_reader as S


# ---- oracle conversions --------------------------------------------------------------------
def test_f16_widening_all_patterns():
    h = np.arange(65536, dtype=np.uint32)
    got = S.f16_to_f32_bits(h)
    half = h.astype(np.uint16).view(np.float16)
    nan = np.isnan(half)
    want = half.astype(np.float32).view(np.uint32)
    np.testing.assert_array_equal(got[~nan], want[~nan])
    np.testing.assert_array_equal(got[nan], ((h[nan] & 0x8000) << 16) | 0x7FC00000)
    assert nan.sum() == 2 * 1023


def test_bf16_widening_all_patterns():
    h = np.arange(65536, dtype=np.uint32)
    want = (torch.from_numpy(h.astype(np.uint16).view(np.int16)).view(torch.bfloat16).float()
            .view(torch.int32).numpy().view(np.uint32))
    np.testing.assert_array_equal(S.bf16_to_f32_bits(h), want)


def _narrowing_inputs():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(200000) * 10.0 ** rng.integers(-12, 8, 200000)).astype(np.float32)
    halves = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((halves[:-1] + halves[1:]) / 2).astype(np.float32)  # exact ties of the f16 grid
    bf = np.arange(0, 0x7F80, dtype=np.uint32) << 16
    bf_ties = (bf | 0x8000).view(np.float32)                     # exact ties of the bf16 grid
    special = np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65519.99, 65520, 1e5, 2.0 ** -24,
                        2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 1e-45,
                        -1e-40, 3.4e38], np.float32)
    return np.concatenate([x, mids, -mids, halves.astype(np.float32), bf_ties, -bf_ties, special])


def test_f16_narrowing_matches_numpy():
    x = _narrowing_inputs()
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(S.f32_to_f16_bits(x), want)
    nan = np.array([np.nan, -np.nan], np.float32)
    np.testing.assert_array_equal(S.f32_to_f16_bits(nan), [0x7E00, 0xFE00])


def test_bf16_narrowing_matches_torch():
    x = _narrowing_inputs()
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(S.f32_to_bf16_bits(x), want)
    nan = np.array([np.nan, -np.nan], np.float32)
    np.testing.assert_array_equal(S.f32_to_bf16_bits(nan), [0x7FC0, 0xFFC0])


# ---- files ---------------------------------------------------------------------------------
def _sample(rng):
    return {
        "decoder.blocks.0.conv1.weight": rng.standard_normal((16, 3, 3, 3, 8)).astype(np.float16),
        "decoder.blocks.0.conv1.bias": rng.standard_normal(16).astype(np.float32),
        "ids": np.arange(-3, 7, dtype=np.int64),
        "mask": rng.integers(0, 2, (3, 5)).astype(bool),
        "bytes": rng.integers(0, 256, 11).astype(np.uint8),
        "i32": rng.integers(-1 << 30, 1 << 30, (2, 2)).astype(np.int32),
        "f64": rng.standard_normal(3),
        "empty": np.zeros((0, 4), np.float32),
        "scalar": np.array(2.5, np.float32),
    }


def test_oracle_reader_matches_safetensors(tmp_path):
    rng = np.random.default_rng(1)
    d = _sample(rng)
    p = tmp_path / "m.safetensors"
    save_file(d, str(p), metadata={"format": "pt", "note": 'a "quoted" \\ value'})
    ref = load_file(str(p))
    meta, tensors, off = S.read_header(p)
    assert meta == {"format": "pt", "note": 'a "quoted" \\ value'}
    assert set(tensors) == set(d)
    for name, arr in ref.items():
        dt, shape, _ = tensors[name]
        assert shape == arr.shape
        got = S.read_raw(p, name).view(S.NP_OF_ST[dt]).reshape(shape)
        np.testing.assert_array_equal(got, arr)
    np.testing.assert_array_equal(S.read_f32(p, "decoder.blocks.0.conv1.weight"),
                                  d["decoder.blocks.0.conv1.weight"].astype(np.float32))
    assert off == 8 + struct.unpack("<Q", p.read_bytes()[:8])[0]


def _native_header(pkg, path):
    sf = pkg.SafetensorsFile(path)
    try:
        return sf.open()
    finally:
        sf.close()


def test_native_header_matches_oracle(pkg, tmp_path):
    rng = np.random.default_rng(2)
    d = _sample(rng)
    d["a" * 700] = np.ones(2, np.float32)                 # longer than the first name buffer
    for i in range(300):
        d[f"many.{i}"] = np.full(i % 3 + 1, i, np.int16)
    p = tmp_path / "m.safetensors"
    save_file(d, str(p), metadata={"format": "pt", "k\"ey": "vé中\U0001f600", "x" * 5000: ""})
    hdr = _native_header(pkg, p)
    meta, tensors, off = S.read_header(p)
    assert hdr.metadata == meta and hdr.data_byte_offset == off
    assert list(hdr.tensors) == list(tensors)             # header order
    for name, (dt, shape, offs) in tensors.items():
        e = hdr.tensors[name]
        assert (e.dtype, e.shape, e.data_offsets) == (dt, shape, offs)
        assert e.numel == int(np.prod(shape))


def _write(path, header_obj_or_text, data=b"", pad=0):
    text = header_obj_or_text if isinstance(header_obj_or_text, str) else json.dumps(header_obj_or_text)
    hb = text.encode() + b" " * pad
    path.write_bytes(struct.pack("<Q", len(hb)) + hb + data)
    return path


def test_native_header_edge_cases(pkg, tmp_path):
    # no tensors; padding after the JSON; unknown fields skipped; escaped names
    h = _native_header(pkg, _write(tmp_path / "a", {}))
    assert h.tensors == {} and h.metadata == {}
    obj = {"x\ty": {"dtype": "BF16", "shape": [2, 3], "data_offsets": [0, 12], "extra": [1, {"a": None}]},
           "__metadata__": {"k": "v", "\u00e9/": "\U0001f600\u4e2d"}}  # \u escapes, surrogates
    h = _native_header(pkg, _write(tmp_path / "b", obj, bytes(12), pad=5))
    assert h.tensors["x\ty"].shape == (2, 3) and h.metadata == obj["__metadata__"]
    assert h.data_byte_offset == 8 + len(json.dumps(obj)) + 5


@pytest.mark.parametrize("case", [
    "short", "len_too_big", "not_json", "unknown_dtype", "offsets_past_end", "size_mismatch",
    "duplicate", "trailing", "metadata_not_string", "missing_shape", "negative_dim",
    "float_offsets", "lone_low_surrogate", "raw_control_char", "invalid_utf8"])
def test_native_header_rejects(pkg, tmp_path, case):
    p = tmp_path / "bad.safetensors"
    ok = {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}
    if case == "short":
        p.write_bytes(b"\x05\x00\x00")
    elif case == "len_too_big":
        p.write_bytes(struct.pack("<Q", 1000) + b"{}")
    elif case == "not_json":
        _write(p, "{\"t\": ", bytes(8))
    elif case == "unknown_dtype":
        _write(p, {"t": {"dtype": "Q7", "shape": [2], "data_offsets": [0, 8]}}, bytes(8))
    elif case == "offsets_past_end":
        _write(p, ok, bytes(4))
    elif case == "size_mismatch":
        _write(p, {"t": {"dtype": "F16", "shape": [2], "data_offsets": [0, 8]}}, bytes(8))
    elif case == "duplicate":
        _write(p, '{"t": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}, '
                  '"t": {"dtype": "U8", "shape": [1], "data_offsets": [1, 2]}}', bytes(2))
    elif case == "trailing":
        _write(p, json.dumps(ok) + "x", bytes(8))
    elif case == "metadata_not_string":
        _write(p, {"__metadata__": {"k": 1}, **ok}, bytes(8))
    elif case == "missing_shape":
        _write(p, {"t": {"dtype": "F32", "data_offsets": [0, 8]}}, bytes(8))
    elif case == "negative_dim":
        _write(p, {"t": {"dtype": "F32", "shape": [-2], "data_offsets": [0, 8]}}, bytes(8))
    elif case == "float_offsets":
        _write(p, {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8.0]}}, bytes(8))
    elif case in STRING_CASES:
        _write_raw(p, STRING_CASES[case], 1)
    with pytest.raises(pkg.TscError) as ei:
        _native_header(pkg, p)
    assert ei.value.status == 1, str(ei.value)
    if case in STRING_CASES:  # the safetensors package refuses these headers too
        from safetensors.numpy import load_file
        with pytest.raises(Exception):
            load_file(str(p))


# Tensor names the safetensors package's JSON reader refuses: a \u escape of a low surrogate with
# no high surrogate before it, an unescaped control byte, and bytes that are not UTF-8.
STRING_CASES = {
    "lone_low_surrogate": b'{"\\udc00": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}',
    "raw_control_char": b'{"a\x01b": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}',
    "invalid_utf8": b'{"a\xffb": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}',
}


def _write_raw(path, header: bytes, data_len: int):
    path.write_bytes(struct.pack("<Q", len(header)) + header + bytes(data_len))
    return path


def test_native_missing_file_and_unknown_tensor(pkg, tmp_path):
    with pytest.raises(pkg.TscError):
        _native_header(pkg, tmp_path / "nope.safetensors")
    p = tmp_path / "m.safetensors"
    save_file({"a": np.zeros(3, np.float32)}, str(p))
    sf = pkg.SafetensorsFile(p)
    sf.open()
    assert sf.get_tensor_info("b") is None and sf.list_tensors() == ["a"]
    with pytest.raises(pkg.TscError):
        sf.read_tensor("b")
    sf.close()
