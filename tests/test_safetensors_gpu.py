"""Safetensors tensors streamed to the GPU vs the oracle: bit-exact for every load and conversion."""
import json

import numpy as np
import pytest
import torch
from safetensors.numpy import save_file

from oracle import st_reader as S

pytestmark = pytest.mark.gpu

_TORCH = {"F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16}
_BITS = {torch.float32: (torch.int32, np.uint32), torch.float16: (torch.int16, np.uint16),
         torch.bfloat16: (torch.int16, np.uint16)}


def _retype(path, names, dtype):
    """Rewrite the header of a file so that the tensors `names` carry `dtype` (numpy has no
    bfloat16: the bf16 patterns are saved as U16 and relabelled; the byte size is unchanged)."""
    raw = path.read_bytes()
    hlen = int.from_bytes(raw[:8], "little")
    head = json.loads(raw[8:8 + hlen])
    for n in names:
        head[n]["dtype"] = dtype
    hb = json.dumps(head, separators=(",", ":")).encode()
    hb += b" " * (-len(hb) % 8)
    path.write_bytes(len(hb).to_bytes(8, "little") + hb + raw[8 + hlen:])


def _bits(t):
    it, npt = _BITS[t.dtype]
    return t.contiguous().view(it).cpu().numpy().view(npt).reshape(-1)


def _float_file(tmp_path):
    """Every 16-bit pattern as F16 and as BF16, and F32 values with ties, subnormals, NaN, inf."""
    rng = np.random.default_rng(3)
    allp = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f32 = np.concatenate([
        (rng.standard_normal(50000) * 10.0 ** rng.integers(-12, 8, 50000)).astype(np.float32),
        ((np.arange(0, 0x7F80, dtype=np.uint32) << 16) | 0x8000).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65520, 2.0 ** -25, 1e-45], np.float32)])
    d = {"f16": allp.view(np.float16).reshape(256, 256), "bf16_bits": allp.reshape(256, 256),
         "f32": f32}
    p = tmp_path / "floats.safetensors"
    save_file(d, str(p))
    _retype(p, ["bf16_bits"], "BF16")
    return p


@pytest.mark.parametrize("src", ["f16", "bf16_bits", "f32"])
@pytest.mark.parametrize("dst", [None, "F32", "F16", "BF16"])
def test_load_and_convert_bit_exact(pkg, dev, tmp_path, src, dst):
    p = _float_file(tmp_path)
    _, tensors, _ = S.read_header(p)
    sdt = tensors[src][0]
    print(f"  st load {src} ({sdt}) -> {dst}", flush=True)
    with pkg.SafetensorsFile(p, dev) as sf:
        got = sf.read_tensor(src, None if dst is None else _TORCH[dst])
        torch.cuda.synchronize()
        assert tuple(got.shape) == tensors[src][1]
        want = S.convert_bits(S.read_raw(p, src), sdt, dst or sdt)
        np.testing.assert_array_equal(_bits(got), want.reshape(-1))
        if dst == "F32":  # readTensorF32 is the same load
            np.testing.assert_array_equal(_bits(sf.read_tensor_f32(src)), want.reshape(-1))


@pytest.mark.parametrize("dst", [None, torch.float32, torch.float16])
def test_multi_chunk_tensor(pkg, dev, tmp_path, dst):
    """A tensor spanning several pinned chunks (16 MiB each) with a ragged tail."""
    rng = np.random.default_rng(4)
    n = 3 * (16 << 20) // 2 + 12345  # bf16 elements: 3 chunks + a partial one
    w = rng.integers(0, 1 << 16, n, dtype=np.uint32).astype(np.uint16)
    w[(w & 0x7F80) == 0x7F80] = 0  # no NaN/inf patterns in this weight-like tensor
    p = tmp_path / "big.safetensors"
    save_file({"pad": np.zeros(3, np.uint8), "w": w}, str(p))
    _retype(p, ["w"], "BF16")
    print(f"  st multi-chunk n={n} -> {dst}", flush=True)
    with pkg.SafetensorsFile(p, dev) as sf:
        got = sf.read_tensor("w", dst)
        torch.cuda.synchronize()
        want = S.convert_bits(S.read_raw(p, "w"), "BF16",
                              {None: "BF16", torch.float32: "F32", torch.float16: "F16"}[dst])
        np.testing.assert_array_equal(_bits(got), want)


def test_raw_types_and_errors(pkg, dev, tmp_path):
    rng = np.random.default_rng(5)
    d = {"i64": rng.integers(-1 << 60, 1 << 60, 1001), "i32": rng.integers(-5, 5, (7, 3)).astype(np.int32),
         "u8": rng.integers(0, 256, 33).astype(np.uint8), "b": rng.integers(0, 2, 9).astype(bool),
         "f64": rng.standard_normal((2, 5)), "i8": rng.integers(-128, 128, 5).astype(np.int8),
         "empty": np.zeros((0, 7), np.float16)}
    p = tmp_path / "raw.safetensors"
    save_file(d, str(p))
    print("  st raw types", flush=True)
    with pkg.SafetensorsFile(p, dev) as sf:
        for name, arr in d.items():
            got = sf.read_tensor(name)
            assert got.is_cuda and tuple(got.shape) == arr.shape
            np.testing.assert_array_equal(got.cpu().numpy(), arr)
            np.testing.assert_array_equal(sf.read_tensor_raw(name).cpu().numpy(), S.read_raw(p, name))
        assert sf.read_tensor("empty", torch.float32).shape == (0, 7)
        # readTensorF32 of a non-float tensor: its bytes as float32 values (weights.ts:178-186)
        np.testing.assert_array_equal(sf.read_tensor_f32("i64").cpu().numpy(),
                                      d["i64"].view(np.float32))
        with pytest.raises(pkg.TscError):
            sf.read_tensor_f32("u8")  # 33 bytes: not a whole number of float32 values
        with pytest.raises(pkg.TscError) as ei:
            sf.read_tensor("i32", torch.float32)
        assert ei.value.status == 2
        with pytest.raises(pkg.TscError):
            sf.read_tensor("missing")


def test_multi_file_loader(pkg, dev, tmp_path):
    a = {"x": np.arange(6, dtype=np.float32).reshape(2, 3)}
    b = {"x": np.full(4, 7, np.int32), "y": np.ones(2, np.float16)}
    save_file(a, str(tmp_path / "a.safetensors"))
    save_file(b, str(tmp_path / "b.safetensors"))
    print("  st multi-file loader", flush=True)
    ld = pkg.MultiFileLoader(dev)
    ld.add_file(tmp_path / "a.safetensors", "enc")
    ld.add_file(tmp_path / "b.safetensors", "dec")
    assert sorted(ld.tensor_to_file) == ["dec:x", "dec:y", "enc:x"]
    np.testing.assert_array_equal(ld.read_tensor("enc:x").cpu().numpy(),
                                  a["x"].view(np.uint8).reshape(-1))
    np.testing.assert_array_equal(ld.read_tensor_as("dec:x").cpu().numpy(), b["x"])
    assert ld.read_tensor_as("dec:y", torch.float32).dtype == torch.float32
    with pytest.raises(pkg.TscError):
        ld.read_tensor("nope:x")
    ld.close_all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_conv_with_weights_from_file(pkg, dev, tmp_path, dtype):
    """A (Co,3,3,3,Ci) bf16 conv weight saved to disk and streamed back drives the conv to the same
    bits as the in-memory weight (converted to dtype the same way)."""
    from safetensors.torch import save_file as save_torch

    rng = np.random.default_rng(6)
    ci, co = 64, 64
    w = torch.from_numpy(pkg.workloads.conv_weight(co, ci, 8)).to(torch.bfloat16)
    bias = torch.from_numpy(rng.standard_normal(co).astype(np.float32)).to(torch.bfloat16)
    p = tmp_path / "conv.safetensors"
    save_torch({"conv.weight": w, "conv.bias": bias}, str(p))
    coords = pkg.workloads.make_coords("conv64_f32")
    feats = torch.from_numpy(rng.standard_normal((len(coords), ci)).astype(np.float32)).to(dtype).to(dev)
    x = pkg.SparseTensor(feats, torch.from_numpy(coords).to(dev))
    print(f"  conv with file weights {dtype}", flush=True)
    with pkg.SafetensorsFile(p, dev) as sf:
        wf = sf.read_tensor("conv.weight", dtype)
        bf = sf.read_tensor("conv.bias", dtype)
    assert torch.equal(wf.cpu(), w.to(dtype)) and torch.equal(bf.cpu(), bias.to(dtype))
    y_file = pkg.SparseConv3d(wf, bf).forward(x)
    y_mem = pkg.SparseConv3d(w.to(dtype).to(dev), bias.to(dtype).to(dev)).forward(x)
    torch.cuda.synchronize()
    assert torch.equal(y_file.feats, y_mem.feats)
