"""The operator path only enqueues work (the reference's forward enqueues and returns without
awaiting, src/sparse/ops/conv3d.ts:41-222): with the spatial shape and batch size given on the host,
SparseConv3d / SparseResBlock3d forward passes, including the neighbor-map build and the conv row
order on first use, make no device-to-host read.  torch's sync debug mode turns any such read
(.item(), .tolist(), .cpu(), ...) into an error.  Results equal the same calls made without the
debug mode, bit for bit; NeighborMap.check() reads the status word afterwards.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _tensor(pkg, dev, coords, feats):
    return pkg.SparseTensor(feats, coords, spatial_shape=(64, 64, 64), batch_size=2)


def test_conv_and_resblock_forward_enqueue_only(pkg, dev):
    wl = pkg.workloads
    coords = torch.from_numpy(wl.make_coords("resblock64_bf16")).to(dev)
    n = coords.shape[0]
    dt = torch.bfloat16
    feats = torch.from_numpy(wl.features(n, 128, 3)).to(dev).to(dt)
    conv = pkg.SparseConv3d(torch.from_numpy(wl.conv_weight(128, 128, 4)).to(dev).to(dt),
                            torch.linspace(-1, 1, 128, device=dev).to(dt))
    blk = pkg.SparseResBlock3d(torch.from_numpy(wl.conv_weight(128, 128, 5)).to(dev).to(dt), None,
                               torch.from_numpy(wl.conv_weight(128, 128, 6)).to(dev).to(dt), None)
    narrow = pkg.SparseConv3d(torch.from_numpy(wl.conv_weight(32, 128, 7)).to(dev).to(dt))
    print(f"  enqueue-only N={n}", flush=True)
    # reference run (also grows the context workspaces, which synchronizes once)
    x0 = _tensor(pkg, dev, coords, feats)
    want = narrow(blk(conv(x0))).feats.clone()
    torch.cuda.synchronize()
    x1 = _tensor(pkg, dev, coords, feats)  # fresh spatial cache: the map is built again
    torch.cuda.set_sync_debug_mode("error")
    try:
        got = narrow(blk(conv(x1))).feats
    finally:
        torch.cuda.set_sync_debug_mode(0)
    assert torch.equal(got, want)
    nmap = x1.get_spatial_cache(pkg.neighbor_cache_key((3, 3, 3), (1, 1, 1)))
    nmap.check()  # valid coordinates: no error


def test_neighbor_map_check_reports_lazily(pkg, dev):
    """A map built through the operator path is not validated until check()."""
    coords = torch.tensor([[0, 1, 1, 1], [0, 1, 1, 1], [0, 2, 2, 2]], dtype=torch.int32, device=dev)
    x = pkg.SparseTensor(torch.zeros((3, 32), device=dev), coords, spatial_shape=(4, 4, 4),
                         batch_size=1)
    nmap = pkg.get_neighbor_map(x)  # enqueue only: no error yet
    with pytest.raises(pkg.TscError, match="duplicate"):
        nmap.check()
    with pytest.raises(pkg.TscError, match="duplicate"):
        pkg.build_neighbor_map(coords, (4, 4, 4), 1)  # the direct call validates by default
