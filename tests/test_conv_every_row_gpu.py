"""Every output row of the narrow and wide convs at their full stated sizes, against the
reference's conv_none restated in PyTorch (oracle/torch_path.py: per tap index_select of the valid
neighbor rows, mm with W[:,v,:]^T, index_add) computed in fp32 on the GPU from the same rounded
inputs.  (test_conv_gpu.py checks the same convs against the fp64 oracle on sampled rows.)

  narrow512 fp16: 1.5 M voxels of a 1-voxel shell in 512^3, Ci = 32 -> Co = 32 and 32 -> 64, as
                  sparse_conv3d runs them (the planned kernel on the map's gather plan)
  wide128 bf16:   4 x ~61 k voxels of 2-voxel shells in 128^3, 512 -> 512 (the 256x256 tile
                  kernel in the map's conv row order)

Tolerance: (i) norm-wise relative error <= 2e-2 and (ii) per-element allclose with
atol = rtol * rms(r), rtol = 2e-2 (tests/_tol.py); both are printed.
"""
import numpy as np
import pytest
import torch

from oracle import torch_path
from tests import _tol

pytestmark = pytest.mark.gpu

CASES = [("narrow512_f16", 32, 32, torch.float16), ("narrow512_f16", 32, 64, torch.float16),
         ("wide128_bf16", 512, 512, torch.bfloat16)]


@pytest.mark.parametrize("workload,ci,co,dtype", CASES)
def test_conv_every_row_vs_conv_none_fp32(pkg, dev, workload, ci, co, dtype):
    wl = pkg.workloads
    coords = wl.make_coords(workload)
    n = len(coords)
    batch = int(coords[:, 0].max()) + 1
    print(f"  every row {workload} N={n} {ci}->{co} {dtype}", flush=True)
    m = pkg.build_neighbor_map(torch.from_numpy(coords).to(dev), wl.grid_shape(workload), batch)
    f = torch.from_numpy(wl.features(n, ci, 11)).to(dev).to(dtype)
    w = torch.from_numpy(wl.conv_weight(co, ci, 12)).to(dev).to(dtype)
    b = (torch.from_numpy(np.random.default_rng(13).standard_normal(co).astype(np.float32)) * 0.1
         ).to(dev).to(dtype)
    got = pkg.sparse_conv3d(f, w, b, m)
    ref = torch_path.conv_none(f.float(), w.float(), b.float(), m.nbr, acc_dtype=torch.float32)
    torch.cuda.synchronize()
    _tol.check(got.float(), ref, 2e-2, f"{workload} {ci}->{co}")
