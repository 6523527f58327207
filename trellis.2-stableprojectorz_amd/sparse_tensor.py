"""SparseTensor: the operand type of the sparse conv path.

Mirrors src/sparse/sparse_tensor.ts:18-121 (and, through it, trellis2.modules.sparse.SparseTensor):
  coords        (N,4) int32 rows [batch, x, y, z]
  feats         (N,C) features
  spatial_shape [X,Y,Z] = per-axis max coordinate + 1 unless given (sparse_tensor.ts:44-60; the
                reference returns [0,0,0] for GPU coords, here it is computed on either device)
  scale         per-axis scale fraction; the spatial cache is keyed by it (sparse_tensor.ts:77-88)
  replace()     new feats, same coords / shape / scale / layout / cache (sparse_tensor.ts:112-121),
                so a neighbor map built once is reused by every later conv on the same voxels
  layout        per-batch [start, stop) row ranges, rows grouped by batch, batch size taken from
                the last row (sparse_tensor.ts:216-237)
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Fraction:
    num: int = 1
    den: int = 1


@dataclass(frozen=True)
class Scale:
    x: Fraction = Fraction()
    y: Fraction = Fraction()
    z: Fraction = Fraction()

    def key(self) -> str:
        """Cache key string, the format of scaleToString (src/sparse/types.ts:41-43)."""
        return f"{self.x.num}/{self.x.den},{self.y.num}/{self.y.den},{self.z.num}/{self.z.den}"


SCALE_IDENTITY = Scale()


def compute_layout(coords: torch.Tensor) -> list[tuple[int, int]]:
    """Per-batch (start, stop) ranges; batch size = coords[-1, 0] + 1 (sparse_tensor.ts:216-237)."""
    n = coords.shape[0]
    if n == 0:
        return [(0, 0)]
    b = coords[:, 0].to(torch.int64)
    batch = int(b[-1].item()) + 1
    counts = torch.bincount(b, minlength=batch)[:batch].tolist()
    layout, start = [], 0
    for c in counts:
        layout.append((start, start + int(c)))
        start += int(c)
    return layout


class SparseTensor:
    """spatial_shape / batch_size may be given by the caller (host ints, e.g. the model's grid
    resolution): the conv path then never reads device values back, so SparseConv3d.forward only
    enqueues work.  Otherwise they are computed from the coordinates on first use (one
    device-to-host read each, cached), as are the per-batch row ranges (`layout`)."""

    def __init__(self, feats: torch.Tensor, coords: torch.Tensor, shape=None,
                 scale: Scale | None = None, cache: dict | None = None, layout=None,
                 spatial_shape=None, batch_size: int | None = None):
        if coords.dim() != 2 or coords.shape[1] != 4:
            raise ValueError("coords must be (N,4) [batch,x,y,z]")
        if feats.shape[0] != coords.shape[0]:
            raise ValueError("feats and coords must have the same number of rows")
        self.feats = feats
        self.coords = coords
        self._shape = list(shape) if shape is not None else None
        self._scale = scale or SCALE_IDENTITY
        self._spatial_cache = cache if cache is not None else {}
        self._layout = layout
        self._batch_size = int(batch_size) if batch_size is not None else None
        if spatial_shape is not None:
            self.register_spatial_cache("shape", [int(v) for v in spatial_shape])

    # ---- properties ---------------------------------------------------------------------
    @property
    def device(self) -> torch.device:
        return self.feats.device

    @property
    def dtype(self) -> torch.dtype:
        return self.feats.dtype

    @property
    def layout(self) -> list[tuple[int, int]]:
        """Per-batch (start, stop) row ranges, computed on first use (sparse_tensor.ts:216-237)."""
        if self._layout is None:
            self._layout = compute_layout(self.coords)
        return self._layout

    @property
    def batch_size(self) -> int:
        if self._batch_size is None:
            self._batch_size = len(self.layout)
        return self._batch_size

    @property
    def shape(self) -> list[int]:
        """[batch, *channel dims]."""
        if self._shape is None:
            self._shape = [self.batch_size, *self.feats.shape[1:]]
        return self._shape

    @property
    def scale(self) -> Scale:
        return self._scale

    @property
    def spatial_shape(self) -> list[int]:
        cached = self.get_spatial_cache("shape")
        if cached is not None:
            return cached
        if self.coords.shape[0] == 0:
            shape = [0, 0, 0]
        else:
            shape = [int(v) + 1 for v in self.coords[:, 1:].amax(dim=0).tolist()]
        self.register_spatial_cache("shape", shape)
        return shape

    # ---- spatial cache (sparse_tensor.ts:77-107) ----------------------------------------
    def get_spatial_cache(self, key: str):
        return self._spatial_cache.get(self._scale.key(), {}).get(key)

    def register_spatial_cache(self, key: str, value) -> None:
        self._spatial_cache.setdefault(self._scale.key(), {})[key] = value

    def clear_spatial_cache(self) -> None:
        """Drops every cached entry (and with it the device buffers of neighbor maps)."""
        for d in self._spatial_cache.values():
            d.clear()

    # ---- replace (sparse_tensor.ts:112-121) ---------------------------------------------
    def replace(self, feats: torch.Tensor, coords: torch.Tensor | None = None) -> "SparseTensor":
        """New feats (and optionally coords) with this tensor's shape, scale, spatial cache and
        layout, as the reference's replace (sparse_tensor.ts:112-121)."""
        return SparseTensor(feats, self.coords if coords is None else coords, self._shape,
                            self._scale, self._spatial_cache, self._layout,
                            batch_size=self._batch_size)

    def to(self, device) -> "SparseTensor":
        return SparseTensor(self.feats.to(device), self.coords.to(device), self._shape,
                            self._scale, self._spatial_cache, self._layout,
                            batch_size=self._batch_size)

    @staticmethod
    def from_feats_and_coords(feats_list, coords_list) -> "SparseTensor":
        """Concatenate per-sample (N_b,C) feats and (N_b,4) coords, rewriting the batch column
        to the sample index (sparse_tensor.ts:159-205)."""
        feats = torch.cat(list(feats_list), dim=0)
        cs = []
        for b, c in enumerate(coords_list):
            c = c.clone()
            c[:, 0] = b
            cs.append(c)
        return SparseTensor(feats, torch.cat(cs, dim=0))

    def __repr__(self) -> str:
        return (f"SparseTensor(voxels={self.feats.shape[0]}, feats={self.shape}, "
                f"spatial={self.spatial_shape}, dtype={self.dtype})")
