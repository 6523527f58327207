"""Neighbor-map build on the GPU vs the oracle / golden fixtures: bit-exact."""
import numpy as np
import pytest
import torch

import oracle
from tests import _golden

pytestmark = pytest.mark.gpu

METHODS = ["bitmap", "radix"]


def _build(pkg, dev, coords, batch, shape, dil=(1, 1, 1), method="auto"):
    print(f"  map_build N={len(coords)} B={batch} shape={shape} dil={dil} method={method}", flush=True)
    c = torch.from_numpy(np.ascontiguousarray(coords, np.int32)).to(dev)
    m = pkg.build_neighbor_map(c, shape, batch, dil, method=method)
    torch.cuda.synchronize()
    return m


def _check(m, coords, batch, shape, dil):
    st, keys, perm, nbr = oracle.map_sorted(coords, batch, shape, dil)
    assert st == 0
    np.testing.assert_array_equal(m.nbr.cpu().numpy(), nbr)
    np.testing.assert_array_equal(m.keys.cpu().numpy().astype(np.int64), keys)
    np.testing.assert_array_equal(m.perm.cpu().numpy(), perm)


@pytest.mark.parametrize("method", METHODS)
@pytest.mark.parametrize("case", ["shell_b2", "random_dil213"])
def test_map_golden(pkg, dev, case, method):
    md, a = _golden.load(case)
    coords = a[("in", "coords")]
    batch = int(md["metadata"]["batch"])
    shape = _golden.meta_tuple(md, "spatial_shape")
    dil = _golden.meta_tuple(md, "dilation")
    m = _build(pkg, dev, coords, batch, shape, dil, method)
    np.testing.assert_array_equal(m.nbr.cpu().numpy(), a[("exp", "nbr")])
    if ("exp", "sorted_keys") in a:
        np.testing.assert_array_equal(m.keys.cpu().numpy().astype(np.int64), a[("exp", "sorted_keys")])


@pytest.mark.parametrize("method", METHODS)
@pytest.mark.parametrize("workload", ["conv64_f32", "wide128_bf16", "resblock64_bf16", "map512"])
def test_map_workloads_bit_exact(pkg, dev, workload, method):
    coords = pkg.workloads.make_coords(workload)
    batch = int(coords[:, 0].max()) + 1
    shape = pkg.workloads.grid_shape(workload)
    m = _build(pkg, dev, coords, batch, shape, method=method)
    _check(m, coords, batch, shape, (1, 1, 1))


@pytest.mark.parametrize("method", METHODS)
def test_map_edge_cases(pkg, dev, method):
    # single voxel at the grid corner
    one = np.array([[0, 0, 0, 0]], np.int32)
    m = _build(pkg, dev, one, 1, (1, 1, 1), method=method)
    _check(m, one, 1, (1, 1, 1), (1, 1, 1))
    # full 3x3x3 block, shuffled, and a full 5x4x6 grid with dilation 2
    rng = np.random.default_rng(0)
    block = np.array([[0, x, y, z] for x in range(3) for y in range(3) for z in range(3)], np.int32)
    block = block[rng.permutation(27)]
    m = _build(pkg, dev, block, 1, (3, 3, 3), method=method)
    _check(m, block, 1, (3, 3, 3), (1, 1, 1))
    full = np.array([[b, x, y, z] for b in range(2) for x in range(5) for y in range(4)
                     for z in range(6)], np.int32)
    m = _build(pkg, dev, full, 2, (5, 4, 6), (2, 1, 2), method)
    _check(m, full, 2, (5, 4, 6), (2, 1, 2))
    # many samples, non-cubic grid, voxels on every face
    coords = np.concatenate([
        np.array([[b, x, y, z] for x in (0, 6) for y in (0, 2, 8) for z in (0, 4)], np.int32)
        for b in range(7)])
    m = _build(pkg, dev, coords, 7, (7, 9, 5), method=method)
    _check(m, coords, 7, (7, 9, 5), (1, 1, 1))
    # key space above 2^31 cells -> int64 keys
    big = np.array([[2, 1020, 1023, 699], [2, 1021, 1023, 699], [0, 0, 0, 0], [1, 5, 5, 5]], np.int32)
    m = _build(pkg, dev, big, 3, (1024, 1024, 700), method=method)
    assert m.keys.dtype == torch.int64
    _check(m, big, 3, (1024, 1024, 700), (1, 1, 1))


@pytest.mark.parametrize("method", METHODS)
def test_map_dense_and_sparse_extremes(pkg, dev, method):
    rng = np.random.default_rng(5)
    # two dense 64x256 slabs in 256^3: key buckets of 16384 voxels (more than one sorting tile)
    slab = np.array([[0, x, y, z] for x in (10, 11) for y in range(64) for z in range(256)], np.int32)
    slab = np.concatenate([slab, np.array([[0, 200, 3, 4], [0, 12, 63, 255]], np.int32)])
    slab = slab[rng.permutation(len(slab))]
    m = _build(pkg, dev, slab, 1, (256, 256, 256), method=method)
    _check(m, slab, 1, (256, 256, 256), (1, 1, 1))
    # full columns of 100 voxels: long binary searches inside the fill windows
    cols = np.array([[b, x, y, z] for b in range(2) for x in range(4) for y in range(5)
                     for z in range(100)], np.int32)
    cols = cols[rng.permutation(len(cols))]
    m = _build(pkg, dev, cols, 2, (4, 5, 100), method=method)
    _check(m, cols, 2, (4, 5, 100), (1, 1, 1))
    # sparse random voxels in 512^3: consecutive sorted voxels far apart
    flat = rng.choice(512 ** 3, size=20000, replace=False)
    sparse = np.stack([np.zeros_like(flat), flat // (512 * 512), (flat // 512) % 512, flat % 512],
                      axis=1).astype(np.int32)
    m = _build(pkg, dev, sparse, 1, (512, 512, 512), method=method)
    _check(m, sparse, 1, (512, 512, 512), (1, 1, 1))
    # a repeated key inside a 2^18-cell grid is still reported after the bucket sort
    dup = np.concatenate([cols[:500, 1:], cols[:1, 1:]])
    dup = np.concatenate([np.zeros((len(dup), 1), np.int32), dup], axis=1)
    with pytest.raises(pkg.TscError, match="duplicate"):
        _build(pkg, dev, dup, 1, (64, 64, 64), method=method)


@pytest.mark.parametrize("method", METHODS)
def test_map_bucket_over_65536(pkg, dev, method):
    """A dense 256x512 half slice of 512^3 is one 2^17-cell key bucket of 131072 voxels: past the
    bitmap rank's 16-bit prefixes, so the radix path sorts it by LSD passes."""
    yz = np.stack(np.meshgrid(np.arange(256), np.arange(512), indexing="ij"), -1).reshape(-1, 2)
    c = np.concatenate([np.zeros((len(yz), 1), np.int64), np.full((len(yz), 1), 7), yz], 1)
    c = np.concatenate([c, [[0, 6, 3, 3], [0, 8, 255, 511], [0, 400, 1, 2]]]).astype(np.int32)
    c = c[np.random.default_rng(8).permutation(len(c))]
    m = _build(pkg, dev, c, 1, (512, 512, 512), method=method)
    _check(m, c, 1, (512, 512, 512), (1, 1, 1))


@pytest.mark.parametrize("xs", [256, 257])
def test_map_dense_box_at_the_sort_limit(pkg, dev, xs):
    """Dense xs x 256 x 256 boxes, shuffled: 2048 sorting tiles of 8192 voxels (xs = 256, the most
    the gathering sort takes: every bucket thread holds eight runs) and 2056 tiles (xs = 257, the
    four-launch sort).  16.8 M voxels are too many for the oracle; a dense box fixes the answer:
    the sorted keys are 0..N-1, perm inverts the shuffle, and neighbor v of a row is the row of the
    in-box cell at offset v, else -1."""
    X, Y, Z = 260, 256, 256
    n = xs * Y * Z
    print(f"  dense box {xs}x{Y}x{Z} N={n}", flush=True)
    key_of_row = torch.randperm(n, generator=torch.Generator().manual_seed(11)).to(dev)
    x, y, z = key_of_row // (Y * Z), (key_of_row // Z) % Y, key_of_row % Z
    coords = torch.stack([torch.zeros_like(x), x, y, z], 1).int()
    m = pkg.build_neighbor_map(coords, (X, Y, Z), 1, method="radix")
    torch.cuda.synchronize()
    assert torch.equal(m.keys.long(), torch.arange(n, device=dev))
    row_of_key = torch.empty_like(key_of_row)
    row_of_key[key_of_row] = torch.arange(n, device=dev)
    assert torch.equal(m.perm.long(), row_of_key)
    for v in range(27):
        nx, ny, nz = x + (v // 9 - 1), y + ((v // 3) % 3 - 1), z + (v % 3 - 1)
        inside = (nx >= 0) & (nx < xs) & (ny >= 0) & (ny < Y) & (nz >= 0) & (nz < Z)
        nkey = ((nx * Y + ny) * Z + nz).clamp(0, n - 1)
        want = torch.where(inside, row_of_key[nkey], torch.full_like(nkey, -1))
        assert torch.equal(m.nbr[:, v].long(), want), f"tap {v}"
    del m


def test_map_empty(pkg, dev):
    c = torch.zeros((0, 4), dtype=torch.int32, device=dev)
    m = pkg.build_neighbor_map(c, (4, 4, 4), 1)
    assert m.nbr.shape == (0, 27)


@pytest.mark.parametrize("method", METHODS)
def test_map_rejects_duplicates_and_out_of_range(pkg, dev, method):
    dup = np.array([[0, 1, 1, 1], [0, 2, 2, 2], [0, 1, 1, 1]], np.int32)
    with pytest.raises(pkg.TscError, match="duplicate"):
        _build(pkg, dev, dup, 1, (4, 4, 4), method=method)
    oob = np.array([[0, 1, 1, 1], [0, 4, 0, 0]], np.int32)
    with pytest.raises(pkg.TscError, match="outside"):
        _build(pkg, dev, oob, 1, (4, 4, 4), method=method)
    neg = np.array([[0, 1, -1, 1]], np.int32)
    with pytest.raises(pkg.TscError, match="outside"):
        _build(pkg, dev, neg, 1, (4, 4, 4), method=method)
    # a valid build after the failures still works (status word is cleared per call)
    ok = np.array([[0, 1, 1, 1], [0, 1, 1, 2]], np.int32)
    m = _build(pkg, dev, ok, 1, (4, 4, 4), method=method)
    _check(m, ok, 1, (4, 4, 4), (1, 1, 1))


def test_map_rejects_bad_arguments(pkg, dev):
    c = torch.zeros((2, 4), dtype=torch.int32, device=dev)
    with pytest.raises(pkg.TscError):
        pkg.build_neighbor_map(c, (4, 4, 4), 1, kernel_size=(5, 5, 5))
    with pytest.raises(pkg.TscError):
        pkg.build_neighbor_map(c, (4, 4, 4), 1, dilation=(0, 1, 1))
    with pytest.raises(pkg.TscError):
        pkg.build_neighbor_map(c[:, 1:].contiguous(), (4, 4, 4), 1)


@pytest.mark.parametrize("n", [1, 111, 113, 100003])
def test_write_floor_writes_the_fill_pattern(pkg, dev, n):
    """tsc_map_write_floor (the measurement kernel bench.py times beside the fill): every row
    rows[i] comes out as (-1, row, -1) x 9, through a permutation and with rows NULL (i); rows of
    the table it is not given stay untouched."""
    import ctypes

    ctx = pkg._lib.context(dev.index)
    perm = torch.randperm(n, generator=torch.Generator().manual_seed(n)).to(torch.int32).to(dev)
    want = torch.tensor([-1, 0, -1] * 9, dtype=torch.int32).repeat(n, 1)
    want[:, 1::3] = torch.arange(n, dtype=torch.int32)[:, None]
    print(f"  write floor n={n}", flush=True)
    for rows in (perm, None):
        out = torch.full((n + 1, 27), 7, dtype=torch.int32, device=dev)  # one row past the table
        st = ctx.lib.tsc_map_write_floor(ctx.bind(), None if rows is None else
                                         ctypes.c_void_p(rows.data_ptr()), n,
                                         ctypes.c_void_p(out.data_ptr()))
        assert st == 0, ctx.lib.tsc_last_error()
        got = out.cpu()
        assert torch.equal(got[:n], want)
        assert (got[n] == 7).all()
