"""SparseConv3d — submanifold sparse 3D convolution, drop-in for the reference operator.

Mirrors src/sparse/ops/conv3d.ts:18-222:
  SparseConv3d(weight (Co,Kd,Kh,Kw,Ci), bias (Co)|None, kernel_size=(3,3,3), dilation=(1,1,1))
  .V                 Kd*Kh*Kw                                          (conv3d.ts:37-39)
  .forward(x)        Ci = weight.shape[4], Co = weight.shape[0]        (conv3d.ts:47-49)
                     neighbor map from x's spatial cache under
                     "conv_neighbors_{Kw}x{Kh}x{Kd}_dil{W}x{H}x{D}", built on a miss  (:62-152)
                     gather-GEMM-bias                                  (:154-208)
                     returns x.replace(out): same coords, shape, scale, cache  (:210-221)
Differences: the neighbor map carries the batch index (the WGSL grid has none) and the grid is
not materialised (an occupancy bitmap or a radix sort replaces it); accumulation is fp32 for
every storage dtype (the WGSL path accumulates in the storage type, conv3d_wgsl.ts:177).
"""
from __future__ import annotations

import torch

from . import ops
from ._lib import TSC_ERR_UNSUPPORTED, TscError
from .sparse_tensor import SparseTensor


def neighbor_cache_key(kernel_size, dilation) -> str:
    kd, kh, kw = kernel_size
    dd, dh, dw = dilation
    return f"conv_neighbors_{kw}x{kh}x{kd}_dil{dw}x{dh}x{dd}"


def get_neighbor_map(x: SparseTensor, kernel_size=(3, 3, 3), dilation=(1, 1, 1),
                     method: str = "auto", validate: bool = False) -> ops.NeighborMap:
    """The cached neighbor map of x's voxels, built on first use.  The build is only enqueued
    (the status word is not read back unless validate=True; NeighborMap.check() reads it), so with
    x's spatial shape and batch size known on the host the conv path never synchronizes."""
    key = neighbor_cache_key(kernel_size, dilation)
    nmap = x.get_spatial_cache(key)
    if nmap is None:
        nmap = ops.build_neighbor_map(x.coords, x.spatial_shape, x.batch_size, dilation,
                                      kernel_size, method, validate=validate)
        x.register_spatial_cache(key, nmap)
    return nmap


class SparseConv3d:
    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None = None,
                 kernel_size=(3, 3, 3), dilation=(1, 1, 1)):
        if tuple(kernel_size) != (3, 3, 3):
            raise TscError(TSC_ERR_UNSUPPORTED, f"kernel {tuple(kernel_size)}: only 3x3x3 is supported")
        if weight.dim() != 5 or tuple(weight.shape[1:4]) != tuple(kernel_size):
            raise ValueError(f"weight must be (Co,Kd,Kh,Kw,Ci), got {tuple(weight.shape)}")
        self.weight = weight.contiguous()
        self.bias = None if bias is None else bias.contiguous()
        self.kernel_size = tuple(kernel_size)
        self.dilation = tuple(dilation)

    @property
    def V(self) -> int:
        return self.kernel_size[0] * self.kernel_size[1] * self.kernel_size[2]

    @property
    def in_channels(self) -> int:
        return self.weight.shape[4]

    @property
    def out_channels(self) -> int:
        return self.weight.shape[0]

    def forward(self, x: SparseTensor) -> SparseTensor:
        if not x.feats.is_cuda:
            raise TscError(1, "SparseConv3d requires GPU input")  # conv3d.ts:42
        nmap = get_neighbor_map(x, self.kernel_size, self.dilation)
        out = ops.sparse_conv3d(x.feats.contiguous(), self.weight, self.bias, nmap)
        return x.replace(out)

    __call__ = forward


class SparseResBlock3d:
    """x + conv2(silu(LN(conv1(x)))) with LN(eps) over channels, C -> C.

    The block of the resblock workload: conv3x3x3 -> LayerNorm -> SiLU -> conv3x3x3 -> +x.  The
    reference's decoder blocks compose the same ops (src/models/sparse_unet_vae_decoder.ts:48-78,
    src/models/sparse_structure_decoder.ts:43-70); the conv1 epilogue adds bias, LayerNorm and
    SiLU run as one row pass, and the conv2 epilogue adds bias and the residual.
    """

    def __init__(self, w1, b1, w2, b2, ln_weight=None, ln_bias=None, eps: float = 1e-6):
        self.conv1 = SparseConv3d(w1, b1)
        self.conv2 = SparseConv3d(w2, b2)
        self.ln_weight, self.ln_bias, self.eps = ln_weight, ln_bias, eps

    def forward(self, x: SparseTensor) -> SparseTensor:
        nmap = get_neighbor_map(x)
        out = ops.sparse_resblock(x.feats.contiguous(), nmap, self.conv1.weight, self.conv1.bias,
                                  self.conv2.weight, self.conv2.bias, self.ln_weight, self.ln_bias,
                                  self.eps)
        return x.replace(out)

    __call__ = forward
