"""Subdivision (the decoder's upsample step) on the GPU vs the oracle: bit-exact."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _run(pkg, dev, coords, feats=None, keep=None):
    c = torch.from_numpy(np.ascontiguousarray(coords, np.int32)).to(dev)
    f = None if feats is None else torch.from_numpy(np.ascontiguousarray(feats)).to(dev)
    k = None if keep is None else torch.from_numpy(np.ascontiguousarray(keep, np.uint8)).to(dev)
    print(f"  subdivide N={len(coords)} feats={None if feats is None else feats.shape} "
          f"keep={keep is not None}", flush=True)
    co, fo = pkg.sparse_subdivide(c, f, k)
    torch.cuda.synchronize()
    return co.cpu().numpy(), None if fo is None else fo.cpu()


def _features(rng, n, c, dtype):
    return torch.from_numpy(rng.standard_normal((n, c)).astype(np.float32)).to(dtype)


@pytest.mark.parametrize("dtype,c", [(torch.float16, 32), (torch.bfloat16, 512), (torch.float32, 3),
                                     (torch.bfloat16, 5)])
@pytest.mark.parametrize("masked", [False, True])
def test_subdivide_matches_oracle(pkg, dev, dtype, c, masked):
    rng = np.random.default_rng(c)
    coords = pkg.workloads.make_coords("resblock64_bf16")[:20000]
    n = len(coords)
    f = _features(rng, n, c, dtype)
    keep = rng.integers(0, 256, size=n).astype(np.uint8) if masked else None
    print(f"  subdivide N={n} C={c} {dtype} keep={masked}", flush=True)
    ct = torch.from_numpy(coords).to(dev)
    kt = None if keep is None else torch.from_numpy(keep).to(dev)
    co, fo = pkg.sparse_subdivide(ct, f.to(dev), kt)
    want_c, want_f = oracle.subdivide(coords, f.float().numpy(), keep)
    np.testing.assert_array_equal(co.cpu().numpy(), want_c)
    # features are copies: compare the bit patterns
    idx = np.repeat(np.arange(n), 8)
    if keep is not None:
        idx = idx[np.unpackbits(keep[:, None], axis=1, bitorder="little").astype(bool).reshape(-1)]
    assert torch.equal(fo.cpu(), f[torch.from_numpy(idx)])
    assert want_f.shape == tuple(fo.shape)


def test_subdivide_edge_cases(pkg, dev):
    # empty input, a single voxel, coordinates only, an all-zero mask, batch > 1
    co, fo = pkg.sparse_subdivide(torch.zeros((0, 4), dtype=torch.int32, device=dev))
    assert co.shape == (0, 4) and fo is None
    one = np.array([[0, 0, 0, 0]], np.int32)
    got, _ = _run(pkg, dev, one)
    np.testing.assert_array_equal(got, oracle.subdivide(one)[0])
    rng = np.random.default_rng(1)
    coords = np.concatenate([pkg.workloads.make_coords("conv64_f32")[:3000] + np.array([b, 0, 0, 0], np.int32)
                             for b in range(3)])
    got, _ = _run(pkg, dev, coords)
    np.testing.assert_array_equal(got, oracle.subdivide(coords)[0])
    got, _ = _run(pkg, dev, coords, keep=np.zeros(len(coords), np.uint8))
    assert got.shape == (0, 4)
    keep = rng.integers(0, 256, size=len(coords)).astype(np.uint8)
    got, _ = _run(pkg, dev, coords, keep=keep)
    np.testing.assert_array_equal(got, oracle.subdivide(coords, None, keep)[0])
    assert pkg.subdivide_count(torch.from_numpy(keep).to(dev)) == int(
        np.unpackbits(keep).sum())


def test_subdivide_rejects_bad_arguments(pkg, dev):
    c = torch.zeros((4, 4), dtype=torch.int32, device=dev)
    with pytest.raises(pkg.TscError):
        pkg.sparse_subdivide(c[:, :3].contiguous())
    with pytest.raises(pkg.TscError):
        pkg.sparse_subdivide(c, torch.zeros((3, 8), device=dev))
    with pytest.raises(pkg.TscError):
        pkg.sparse_subdivide(c, None, torch.zeros(4, dtype=torch.int32, device=dev))


def test_subdivide_module_then_conv(pkg, dev):
    """SparseSubdivide output: doubled shape and scale, and a conv on it uses the children's own
    neighbor map (bit-exact against the oracle's map of the children)."""
    coords = pkg.workloads.make_coords("conv64_f32")
    n = len(coords)
    rng = np.random.default_rng(2)
    f = torch.from_numpy(rng.standard_normal((n, 16)).astype(np.float32)).to(dev)
    x = pkg.SparseTensor(f, torch.from_numpy(coords).to(dev))
    sp = x.spatial_shape
    y = pkg.SparseSubdivide()(x)
    assert y.spatial_shape == [2 * s for s in sp]
    assert y.scale.key() == "2/1,2/1,2/1" and y._spatial_cache is x._spatial_cache
    assert y.feats.shape == (8 * n, 16) and y.batch_size == x.batch_size
    w = torch.from_numpy(pkg.workloads.conv_weight(32, 16, 7)).to(dev)
    print(f"  subdivide -> conv N={8 * n}", flush=True)
    out = pkg.SparseConv3d(w).forward(y)
    nmap = pkg.get_neighbor_map(y)
    kids = y.coords.cpu().numpy()
    st, _, _, nbr = oracle.map_sorted(kids, 1, tuple(y.spatial_shape))
    assert st == 0
    np.testing.assert_array_equal(nmap.nbr.cpu().numpy(), nbr)
    sel = np.sort(rng.choice(8 * n, 2000, replace=False))
    ref = oracle.conv(y.feats.cpu().numpy().astype(np.float64), w.cpu().numpy().astype(np.float64),
                      None, nbr[sel])
    err = np.abs(out.feats.cpu().numpy()[sel] - ref).max() / np.abs(ref).max()
    assert err <= 1e-4, err
