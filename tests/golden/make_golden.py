"""Generate the golden fixtures in this directory.

Fixture format follows the reference's golden harness (src/validation/loader.ts:1-33): one
directory per case with metadata.json ({name, tolerance, inputs[], expected[]}, each entry
{file, shape, dtype}) and raw little-endian row-major .bin files.  "float64" is added as a dtype.

Expected values are computed WITHOUT the CPU oracle under oracle/, from the definitions:
  * neighbor maps by a Python dict brute force over the 27 offsets (conv3d_wgsl.ts:91-124),
    sorted keys by numpy.unique of the packed keys;
  * convolutions by the closed form of README.md:81 — scatter the features to a dense grid per
    batch sample, torch.nn.functional.conv3d in float64 with the weight permuted from
    (Co,Kd,Kh,Kw,Ci) to (Co,Ci,Kd,Kh,Kw), padding = dilation, then gather at the voxels;
  * LayerNorm / SiLU by torch.nn.functional.layer_norm / silu in float64.

Run:  python tests/golden/make_golden.py   (rewrites every case; deterministic)
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent


def brute_map(coords, shape, dil):
    X, Y, Z = shape
    table = {tuple(int(v) for v in c): i for i, c in enumerate(coords)}
    out = np.full((len(coords), 27), -1, np.int32)
    for i, (b, x, y, z) in enumerate(coords):
        for v in range(27):
            kd, kh, kw = v // 9, (v // 3) % 3, v % 3
            n = (int(x) + (kd - 1) * dil[0], int(y) + (kh - 1) * dil[1], int(z) + (kw - 1) * dil[2])
            if 0 <= n[0] < X and 0 <= n[1] < Y and 0 <= n[2] < Z:
                out[i, v] = table.get((int(b), *n), -1)
    return out


def dense_conv(coords, feats, weight, bias, shape, dil, batch):
    """Closed form: dense F.conv3d per sample, gathered back at the voxels (float64)."""
    X, Y, Z = shape
    ci, co = weight.shape[4], weight.shape[0]
    w = torch.from_numpy(weight.astype(np.float64)).permute(0, 4, 1, 2, 3).contiguous()
    out = np.zeros((len(coords), co), np.float64)
    for b in range(batch):
        rows = np.nonzero(coords[:, 0] == b)[0]
        grid = torch.zeros((1, ci, X, Y, Z), dtype=torch.float64)
        c = torch.from_numpy(coords[rows].astype(np.int64))
        grid[0, :, c[:, 1], c[:, 2], c[:, 3]] = torch.from_numpy(feats[rows].astype(np.float64)).T
        y = F.conv3d(grid, w, None, padding=tuple(dil), dilation=tuple(dil))
        out[rows] = y[0, :, c[:, 1], c[:, 2], c[:, 3]].T.numpy()
    if bias is not None:
        out += bias.astype(np.float64)
    return out


def random_voxels(rng, batch, shape, n_per):
    rows = []
    for b in range(batch):
        cells = rng.choice(shape[0] * shape[1] * shape[2], size=n_per, replace=False)
        x, rem = np.divmod(cells, shape[1] * shape[2])
        y, z = np.divmod(rem, shape[2])
        rows.append(np.stack([np.full(n_per, b), x, y, z], 1))
    c = np.concatenate(rows).astype(np.int32)
    return c[rng.permutation(len(c))] if batch == 1 else c


def ball_shell(rng, batch, g):
    """Small 1-2 voxel shells of random balls, rows grouped by batch and shuffled within it."""
    parts = []
    for b in range(batch):
        r = rng.uniform(g * 0.25, g * 0.42)
        c = g / 2 + rng.uniform(-1, 1, 3)
        p = np.argwhere(np.ones((g, g, g), bool)) + 0.5
        d = np.linalg.norm(p - c, axis=1)
        xyz = np.argwhere(np.ones((g, g, g), bool))[(d < r) & (d >= r - 1.6)]
        xyz = xyz[rng.permutation(len(xyz))]
        parts.append(np.concatenate([np.full((len(xyz), 1), b), xyz], 1))
    return np.concatenate(parts).astype(np.int32)


def write_case(name, tol, inputs, expected, meta=None):
    d = HERE / name
    d.mkdir(exist_ok=True)
    entries_in, entries_out = [], []
    for key, arr in inputs.items():
        f = f"input_{key}.bin"
        np.ascontiguousarray(arr).tofile(d / f)
        entries_in.append({"file": f, "shape": list(arr.shape), "dtype": str(arr.dtype)})
    for key, arr in expected.items():
        f = f"expected_{key}.bin"
        np.ascontiguousarray(arr).tofile(d / f)
        entries_out.append({"file": f, "shape": list(arr.shape), "dtype": str(arr.dtype)})
    md = {"name": name, "tolerance": tol, "nondeterministic": False,
          "inputs": entries_in, "expected": entries_out, "metadata": meta or {}}
    (d / "metadata.json").write_text(json.dumps(md, indent=1) + "\n")


def main():
    rng = np.random.default_rng(20261201)

    # 1. two ball shells (B=2) in 14^3, dilation 1: map, sorted keys, fp32 conv 8->32 with bias.
    shape = (14, 14, 14)
    coords = ball_shell(rng, 2, 14)
    nbr = brute_map(coords, shape, (1, 1, 1))
    keys = np.unique(((coords[:, 0].astype(np.int64) * 14 + coords[:, 1]) * 14 + coords[:, 2]) * 14
                     + coords[:, 3])
    assert len(keys) == len(coords)
    feats = rng.standard_normal((len(coords), 8)).astype(np.float32)
    w = (rng.standard_normal((32, 3, 3, 3, 8)) / np.sqrt(27 * 8)).astype(np.float32)
    b = rng.standard_normal(32).astype(np.float32)
    out = dense_conv(coords, feats, w, b, shape, (1, 1, 1), 2)
    write_case("shell_b2", {"rtol": 0, "atol": 0},
               {"coords": coords, "feats": feats, "weight": w, "bias": b},
               {"nbr": nbr, "sorted_keys": keys, "conv_out": out},
               {"batch": "2", "spatial_shape": "14,14,14", "dilation": "1,1,1"})

    # 2. random voxels in a non-cubic 10x12x9 grid, dilation (2,1,3), one sample, shuffled.
    shape = (10, 12, 9)
    coords = random_voxels(rng, 1, shape, 300)
    nbr = brute_map(coords, shape, (2, 1, 3))
    feats = rng.standard_normal((len(coords), 16)).astype(np.float32)
    w = (rng.standard_normal((32, 3, 3, 3, 16)) / np.sqrt(27 * 16)).astype(np.float32)
    out = dense_conv(coords, feats, w, None, shape, (2, 1, 3), 1)
    write_case("random_dil213", {"rtol": 0, "atol": 0},
               {"coords": coords, "feats": feats, "weight": w},
               {"nbr": nbr, "conv_out": out},
               {"batch": "1", "spatial_shape": "10,12,9", "dilation": "2,1,3"})

    # 3. LayerNorm(eps=1e-6) with affine, and LayerNorm -> SiLU, over 96 channels.
    x = (rng.standard_normal((40, 96)) * 3 + 0.5).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 96).astype(np.float32)
    beta = rng.standard_normal(96).astype(np.float32)
    xt = torch.from_numpy(x.astype(np.float64))
    ln = F.layer_norm(xt, (96,), torch.from_numpy(g.astype(np.float64)),
                      torch.from_numpy(beta.astype(np.float64)), eps=1e-6)
    write_case("layernorm_silu", {"rtol": 1e-5, "atol": 1e-7},
               {"x": x, "gamma": g, "beta": beta},
               {"ln": ln.numpy(), "ln_silu": F.silu(ln).numpy()}, {"eps": "1e-6"})
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    sys.exit(main())
