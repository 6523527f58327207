"""Per-voxel linear layer and the sparse ConvNeXt block on the GPU vs the fp64 oracle.

Tolerance (norm-wise relative, max|y - r| / max|r|, r in fp64 from the same rounded inputs):
fp32 <= 1e-4, fp16 / bf16 <= 2e-2.
"""
import numpy as np
import pytest
import torch

import oracle
from tests import _tol

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _rounded(a, dtype, dev):
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(dtype)
    return t, t.float().cpu().numpy().astype(np.float64)


def rel_err(got, ref):
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n,cin,cout", [(5000, 256, 1024), (777, 96, 40)])
def test_linear_matches_oracle(pkg, dev, dtype, n, cin, cout):
    rng = np.random.default_rng(cin)
    x, x64 = _rounded(rng.standard_normal((n, cin)), dtype, dev)
    w, w64 = _rounded(rng.standard_normal((cout, cin)) / np.sqrt(cin), dtype, dev)
    b, b64 = _rounded(rng.standard_normal(cout) * 0.1, dtype, dev)
    r, r64 = _rounded(rng.standard_normal((n, cout)), dtype, dev)
    print(f"  linear N={n} {cin}->{cout} {dtype}", flush=True)
    got = pkg.sparse_linear(x, w, b).float().cpu().numpy()
    assert rel_err(got, oracle.linear(x64, w64, b64)) <= TOL[dtype]
    got = pkg.sparse_linear(x, w).float().cpu().numpy()
    assert rel_err(got, oracle.linear(x64, w64)) <= TOL[dtype]
    r2 = r.clone()
    pkg.sparse_linear(x, w, b, residual=r2, out=r2)  # in place on the residual
    assert rel_err(r2.float().cpu().numpy(), oracle.linear(x64, w64, b64, r64)) <= TOL[dtype]


def test_linear_rejects_bad_arguments(pkg, dev):
    x = torch.zeros((4, 8), device=dev)
    with pytest.raises(pkg.TscError):
        pkg.sparse_linear(x, torch.zeros((3, 7), device=dev))
    with pytest.raises(pkg.TscError):
        pkg.sparse_linear(x, torch.zeros((3, 8), device=dev), torch.zeros(4, device=dev))
    with pytest.raises(pkg.TscError):
        pkg.sparse_linear(x, torch.zeros((3, 8), device=dev, dtype=torch.float16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_convnext_block_matches_oracle(pkg, dev, dtype):
    coords = pkg.workloads.make_coords("resblock64_bf16")
    n = len(coords)
    c, hid = 128, 512
    rng = np.random.default_rng(11)
    x, x64 = _rounded(rng.standard_normal((n, c)), dtype, dev)
    cw, cw64 = _rounded(pkg.workloads.conv_weight(c, c, 12), dtype, dev)
    cb, cb64 = _rounded(rng.standard_normal(c) * 0.1, dtype, dev)
    w0, w064 = _rounded(rng.standard_normal((hid, c)) / np.sqrt(c), dtype, dev)
    b0, b064 = _rounded(rng.standard_normal(hid) * 0.1, dtype, dev)
    w2, w264 = _rounded(rng.standard_normal((c, hid)) / np.sqrt(hid), dtype, dev)
    b2, b264 = _rounded(rng.standard_normal(c) * 0.1, dtype, dev)
    st = pkg.SparseTensor(x, torch.from_numpy(coords).to(dev))
    blk = pkg.SparseConvNeXtBlock3d(cw, cb, w0, b0, w2, b2, eps=1e-6)
    print(f"  convnext N={n} C={c} hidden={hid} {dtype}", flush=True)
    out = blk(st)
    assert out.coords is st.coords and out.feats.shape == (n, c)
    nbr = pkg.get_neighbor_map(st).nbr.cpu().numpy()
    rows = np.sort(rng.choice(n, 1500, replace=False))
    got = out.feats.float().cpu().numpy()[rows]
    if dtype == torch.float32:
        ref = oracle.convnext_block(x64, nbr, cw64, cb64, w064, b064, w264, b264, 1e-6, rows=rows)
        assert rel_err(got, ref) <= 1e-4
        return
    # The block stores each step's tensor in bf16, as the TS block does: the oracle rounds its
    # fp64 intermediates to bf16 at the same five points (round to nearest even), and the block
    # must match it within the bf16 tolerance.  Against the unrounded fp64 block the five
    # roundings add up to more (printed; bounded at 5e-2).
    def to_bf16(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).double().numpy()
    ref_r = oracle.convnext_block(x64, nbr, cw64, cb64, w064, b064, w264, b264, 1e-6, rows=rows,
                                  store=to_bf16)
    ref_u = oracle.convnext_block(x64, nbr, cw64, cb64, w064, b064, w264, b264, 1e-6, rows=rows)
    e_r = _tol.check(got, ref_r, 2e-2, "convnext bf16 vs bf16-rounded oracle")
    e_u = rel_err(got, ref_u)
    print(f"  convnext bf16 vs unrounded fp64 oracle: norm-wise {e_u:.3e}", flush=True)
    assert e_u <= 5e-2, e_u
