"""Sparse decoder blocks around the conv: SparseLinear and the ConvNeXt block.

  SparseLinear            src/sparse/ops/linear.ts:9-29 (nn.Linear per voxel; the TS port
                          multiplies by the (out,in) weight untransposed)
  SparseConvNeXtBlock3d   src/models/sparse_unet_vae_decoder.ts:48-78 and its use at :119-134:
                          h = conv(x); h = LN(h); h = h W0^T + b0; h = silu(LN(h)); out = x + h W2^T + b2
                          (LayerNorm without affine, eps 1e-6, as the TS block calls it)

Each step is one C-ABI call: the conv (tsc_conv, map cached on x), tsc_layernorm (SiLU fused into
the second one), and tsc_linear (hipBLASLt GEMM with the bias epilogue; the second linear takes
the block input as its residual operand, so the skip add costs no extra pass).
"""
from __future__ import annotations

import torch

from . import ops
from .conv3d import SparseConv3d
from .sparse_tensor import SparseTensor


class SparseLinear:
    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None = None):
        if weight.dim() != 2:
            raise ValueError("weight must be (out_channels, in_channels)")
        self.weight = weight.contiguous()
        self.bias = None if bias is None else bias.contiguous()

    def forward(self, x: SparseTensor) -> SparseTensor:
        return x.replace(ops.sparse_linear(x.feats, self.weight, self.bias))

    __call__ = forward


class SparseConvNeXtBlock3d:
    def __init__(self, conv_weight: torch.Tensor, conv_bias: torch.Tensor | None,
                 linear0_weight: torch.Tensor, linear0_bias: torch.Tensor | None,
                 linear2_weight: torch.Tensor, linear2_bias: torch.Tensor | None,
                 eps: float = 1e-6):
        self.conv = SparseConv3d(conv_weight, conv_bias)
        self.linear0 = SparseLinear(linear0_weight, linear0_bias)
        self.linear2 = SparseLinear(linear2_weight, linear2_bias)
        self.eps = eps

    def forward(self, x: SparseTensor) -> SparseTensor:
        h = self.conv.forward(x).feats
        ops.layer_norm(h, eps=self.eps, out=h)
        h = ops.sparse_linear(h, self.linear0.weight, self.linear0.bias)
        ops.layer_norm(h, eps=self.eps, silu=True, out=h)
        out = ops.sparse_linear(h, self.linear2.weight, self.linear2.bias, residual=x.feats)
        return x.replace(out)

    __call__ = forward
