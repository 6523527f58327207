"""MI355X-native submanifold sparse conv3d for TRELLIS.2 (host side over libtrellis_sparse.so).

Importable under the alias `trellis2_amd` (see __graft_entry__.load_package); the directory name
is not a Python identifier.

  SparseTensor, SparseConv3d, SparseResBlock3d   operator API of src/sparse (conv3d.ts:18-222)
  build_neighbor_map, sparse_conv3d,             functional entry points, one C-ABI call each
  layer_norm, silu, add, sparse_resblock
  SparseSubdivide, sparse_subdivide              decoder upsample (sparse_unet_vae_decoder.ts:155-175)
  SparseLinear, SparseConvNeXtBlock3d,           decoder blocks (linear.ts:9-29,
  sparse_linear                                  sparse_unet_vae_decoder.ts:48-78)
  sparse_attention,                              varlen attention (sparse/ops/attention.ts:24-79,
  scaled_dot_product_attention                   dense/ops/attention.ts:36-110)
  SafetensorsFile, MultiFileLoader               weight files -> device tensors (weights.ts:58-237)
  workloads                                      seeded synthetic voxel shells
"""
from ._lib import TscError, load_library, header_symbols, LIB_PATH  # noqa: F401
from .sparse_tensor import SparseTensor, Scale, Fraction, SCALE_IDENTITY, compute_layout  # noqa: F401
from .conv3d import SparseConv3d, SparseResBlock3d, get_neighbor_map, neighbor_cache_key  # noqa: F401
from .ops import (NeighborMap, build_neighbor_map, map_conv_order, map_gather_plan,  # noqa: F401
                  sparse_conv3d,
                  layer_norm, silu, add, sparse_resblock, sparse_subdivide, subdivide_count,
                  sparse_linear, sparse_attention, scaled_dot_product_attention)
from .spatial import SparseSubdivide  # noqa: F401
from .blocks import SparseLinear, SparseConvNeXtBlock3d  # noqa: F401
from .weights import SafetensorsFile, SafetensorsHeader, TensorEntry, MultiFileLoader  # noqa: F401
from . import workloads  # noqa: F401

__all__ = [
    "TscError", "SparseTensor", "SparseConv3d", "SparseResBlock3d", "NeighborMap",
    "build_neighbor_map", "map_conv_order", "map_gather_plan", "sparse_conv3d", "layer_norm", "silu", "add", "sparse_resblock",
    "sparse_subdivide", "subdivide_count", "SparseSubdivide", "sparse_linear", "SparseLinear",
    "SparseConvNeXtBlock3d", "sparse_attention", "scaled_dot_product_attention", "SafetensorsFile", "SafetensorsHeader", "TensorEntry", "MultiFileLoader",
    "get_neighbor_map", "neighbor_cache_key", "workloads",
]
