"""The safetensors header parser (host C++, untrusted input) under AddressSanitizer and
UndefinedBehaviorSanitizer on the CPU: tests/fuzz/st_header_fuzz.cpp + csrc/st_header.cpp built
with g++ -fsanitize=address,undefined -fno-sanitize-recover=all, fed a corpus of valid files
(written by the safetensors package) and of the malformed files the native tests reject, then
200 000 seeded mutations of them.  Any memory error or undefined behaviour aborts the harness;
for every header it accepts it checks the parser's promises (ranges inside the data block,
length = numel x element size, unique names).  No GPU is involved.
"""
import json
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HARNESS = ROOT / "tests" / "fuzz" / "st_header_fuzz.cpp"
PARSER = ROOT / "trellis.2-stableprojectorz_amd" / "csrc" / "st_header.cpp"


def _write(path, header, data=b"", pad=0):
    text = header if isinstance(header, str) else json.dumps(header)
    hb = text.encode() + b" " * pad
    path.write_bytes(struct.pack("<Q", len(hb)) + hb + data)
    return path


def _corpus(d: Path) -> list:
    from safetensors.numpy import save_file

    files = []
    rng = np.random.default_rng(0)
    tensors = {"w": rng.standard_normal((3, 4)).astype(np.float32),
               "b": np.arange(5, dtype=np.int16), "e": np.zeros((0, 2), np.float16),
               "s": np.array(1.5, np.float64), "m": np.ones((2, 2), np.uint8)}
    p = d / "valid.safetensors"
    save_file(tensors, str(p), metadata={"format": "pt", "k\"ey": "vé\U0001f600"})
    files.append(p)
    files.append(_write(d / "empty.safetensors", {}))
    files.append(_write(d / "escapes.safetensors",
                        {"x\ty": {"dtype": "BF16", "shape": [2, 3], "data_offsets": [0, 12],
                                  "extra": [1, {"a": None, "b": [True, False, -1.5e3]}]},
                         "__metadata__": {"k": "v", "é/": "\U0001f600中"}},
                        bytes(12), pad=5))
    ok = {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}
    bad = {
        "short": b"\x05\x00\x00",
        "len_too_big": struct.pack("<Q", 1000) + b"{}",
    }
    for name, raw in bad.items():
        p = d / f"{name}.safetensors"
        p.write_bytes(raw)
        files.append(p)
    for name, hdr, data in [
        ("not_json", "{\"t\": ", bytes(8)),
        ("unknown_dtype", {"t": {"dtype": "Q7", "shape": [2], "data_offsets": [0, 8]}}, bytes(8)),
        ("offsets_past_end", ok, bytes(4)),
        ("size_mismatch", {"t": {"dtype": "F16", "shape": [2], "data_offsets": [0, 8]}}, bytes(8)),
        ("duplicate", '{"t": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}, '
                      '"t": {"dtype": "U8", "shape": [1], "data_offsets": [1, 2]}}', bytes(2)),
        ("trailing", json.dumps(ok) + "x", bytes(8)),
        ("metadata_not_string", {"__metadata__": {"k": 1}, **ok}, bytes(8)),
        ("missing_shape", {"t": {"dtype": "F32", "data_offsets": [0, 8]}}, bytes(8)),
        ("negative_dim", {"t": {"dtype": "F32", "shape": [-2], "data_offsets": [0, 8]}}, bytes(8)),
        ("float_offsets", {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8.0]}}, bytes(8)),
        ("huge_shape", {"t": {"dtype": "F64", "shape": [2 ** 31, 2 ** 31, 8],
                              "data_offsets": [0, 8]}}, bytes(8)),
        ("deep", "[" * 200 + "]" * 200, b""),
        ("lone_surrogate", '{"\\ud800": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}',
         bytes(1)),
        ("lone_low_surrogate", '{"\\udc00": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}',
         bytes(1)),
        ("raw_control_char", '{"a\x01b": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}',
         bytes(1)),
    ]:
        files.append(_write(d / f"{name}.safetensors", hdr, data))
    p = d / "invalid_utf8.safetensors"
    hb = b'{"a\xffb": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}'
    p.write_bytes(struct.pack("<Q", len(hb)) + hb + bytes(1))
    files.append(p)
    return files


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not available")
def test_st_header_parser_under_asan_ubsan(tmp_path):
    exe = tmp_path / "st_header_fuzz"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           str(HARNESS), str(PARSER), "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    files = _corpus(tmp_path)
    env = {"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=1",
           "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1", "PATH": "/usr/bin:/bin"}
    for seed in (1, 2):
        r = subprocess.run([str(exe), "100000", str(seed), *map(str, files)], capture_output=True,
                           text=True, env=env, timeout=600)
        assert r.returncode == 0, (r.stdout, r.stderr[-4000:])
        assert "failures 0" in r.stdout, r.stdout
        # the valid seeds are accepted, the malformed ones are not
        assert "(accepted 3)" in r.stdout, r.stdout
