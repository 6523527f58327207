"""PyTorch-CPU restatement of the reference's Python sparse-conv path — TEST INFRASTRUCTURE ONLY.

The reference's Python backend (`SPARSE_CONV_BACKEND=none`) is documented as
  * hashmap_fallback: "GPU-sorted flat_idx hashmap via torch.sort + torch.searchsorted"
    (README.md:111), giving 27 self+neighbor lookups per voxel (README.md:80);
  * conv_none: "Pure-PyTorch submanifold sparse conv ... Weight layout (Co,Kd,Kh,Kw,Ci)"
    (README.md:109), i.e. gather + GEMM + bias (src/sparse/ops/conv3d.ts:1-6).
The original files are not in the checkout (empty submodule), so this module restates that
description with the same torch primitives.  It is the timed CPU baseline of bench.py and a
second, independent implementation the C oracle is checked against.
"""
from __future__ import annotations

import torch

OFFSETS = [(kd - 1, kh - 1, kw - 1) for kd in range(3) for kh in range(3) for kw in range(3)]


def flat_idx(coords: torch.Tensor, shape) -> torch.Tensor:
    X, Y, Z = shape
    c = coords.to(torch.int64)
    return ((c[:, 0] * X + c[:, 1]) * Y + c[:, 2]) * Z + c[:, 3]


def hashmap_fallback(coords: torch.Tensor, shape, dilation=(1, 1, 1)):
    """(sorted_keys int64, perm int64, nbr (N,27) int32) via torch.sort + torch.searchsorted."""
    X, Y, Z = shape
    key = flat_idx(coords, shape)
    sorted_keys, perm = torch.sort(key)
    n = coords.shape[0]
    nbr = torch.full((n, 27), -1, dtype=torch.int32)
    c = coords.to(torch.int64)
    for v, (dx, dy, dz) in enumerate(OFFSETS):
        nx = c[:, 1] + dx * dilation[0]
        ny = c[:, 2] + dy * dilation[1]
        nz = c[:, 3] + dz * dilation[2]
        ok = (nx >= 0) & (nx < X) & (ny >= 0) & (ny < Y) & (nz >= 0) & (nz < Z)
        nk = ((c[:, 0] * X + nx) * Y + ny) * Z + nz
        pos = torch.searchsorted(sorted_keys, nk).clamp_(max=max(n - 1, 0))
        hit = ok & (sorted_keys[pos] == nk)
        nbr[:, v] = torch.where(hit, perm[pos], torch.full_like(pos, -1)).to(torch.int32)
    return sorted_keys, perm, nbr


def conv_none(feats: torch.Tensor, weight: torch.Tensor, bias, nbr: torch.Tensor,
              acc_dtype=torch.float32) -> torch.Tensor:
    """out = bias + sum_v feats[nbr[:,v]] @ W[:,v,:]^T over valid taps, accumulated in acc_dtype."""
    co, ci = weight.shape[0], weight.shape[-1]
    w = weight.reshape(co, 27, ci).to(acc_dtype)
    out = torch.zeros(nbr.shape[0], co, dtype=acc_dtype, device=feats.device)
    f = feats.to(acc_dtype)
    for v in range(27):
        idx = nbr[:, v].to(torch.int64)
        m = idx >= 0
        if not bool(m.any()):
            continue
        rows = torch.nonzero(m, as_tuple=True)[0]
        out.index_add_(0, rows, torch.index_select(f, 0, idx[rows]) @ w[:, v, :].T)
    if bias is not None:
        out += bias.to(acc_dtype)
    return out
