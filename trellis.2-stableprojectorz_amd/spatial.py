"""SparseSubdivide: the sparse decoder's upsample step (each voxel -> its 2x2x2 children).

Caller in the reference: the level transition of the SLat decoder,
src/models/sparse_unet_vae_decoder.ts:155-175 ("Subdivide 1 voxel -> 8 child voxels"), where the
TS port only doubles the spatial shape and keeps the parent coordinates.  Here the children are
generated on the GPU (tsc_subdivide): coordinates [b, 2x+dx, 2y+dy, 2z+dz] in parent-major order,
children c = dx*4 + dy*2 + dz in increasing order, features copied from the parent, optionally
only the children a per-parent keep mask selects (the decoder's predicted subdivision, kept as
`guideSubs` in the TS port).  The result has twice the spatial shape and scale; it shares the
input's spatial cache dict, whose entries are keyed by scale, so the neighbor map of the children
is built on their first conv.
"""
from __future__ import annotations

from math import gcd

import torch

from . import ops
from .sparse_tensor import Fraction, Scale, SparseTensor


def _double(f: Fraction) -> Fraction:
    num, den = 2 * f.num, f.den
    g = gcd(num, den)
    return Fraction(num // g, den // g)


class SparseSubdivide:
    def forward(self, x: SparseTensor, keep: torch.Tensor | None = None) -> SparseTensor:
        coords, feats = ops.sparse_subdivide(x.coords, x.feats, keep)
        scale = Scale(_double(x.scale.x), _double(x.scale.y), _double(x.scale.z))
        out = SparseTensor(feats, coords, scale=scale, cache=x._spatial_cache)
        out.register_spatial_cache("shape", [2 * s for s in x.spatial_shape])
        return out

    __call__ = forward
