"""Gather plan (tsc_map_gather_plan) and the planned narrow conv (tsc_conv_planned) on the GPU.

The plan is checked against its definition on the CPU: rows are a permutation sorted by the
Morton code of the coordinates, every (row, tap) slot names the neighbor the map gives, slots
follow the stated order (own rows first, then first use in (tap, row) order; a split tile —
more distinct rows than the LDS staging holds, but each 32-row half fewer — orders them as rows
only the first half uses, rows both use, rows only the second half uses, and stores the second
half's slots minus the first group's size), and the tap masks are the OR of presence.  The
planned conv must equal the unplanned kernels bit for bit, including split tiles and tiles that
take its fallback path (more distinct rows than the staging holds even per half).
"""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

TILE, SLOTS, TBL = 64, 256, 16 * 28 * 4
STAGE = 208  # LDS row slots per wave in the planned kernel (tiles or halves with fewer are staged)
SPLIT = 1 << 30  # count flag of a split tile: d | sA << 8 | aonly << 16 | SPLIT


def _align(v):
    return (v + 255) // 256 * 256


def _decode(plan, n):
    t = (n + TILE - 1) // TILE
    b = plan.cpu().numpy()
    off = 0
    rows = b[off:off + t * TILE * 4].view(np.int32)
    off = _align(off + t * TILE * 4)
    count = b[off:off + t * 4].view(np.int32)
    off = _align(off + t * 4)
    rbm = b[off:off + t * 16].view(np.uint32).reshape(t, 4)
    off = _align(off + t * 16)
    lst = b[off:off + t * SLOTS * 4].view(np.int32).reshape(t, SLOTS)
    off = _align(off + t * SLOTS * 4)
    slots = b[off:off + t * TBL].reshape(t, 16, 28, 4)
    off = _align(off + t * TBL)
    assert off == len(b)
    return rows, count, rbm, lst, slots


def _morton(c, bits):
    k = np.zeros(len(c), np.uint64)
    for i in range(bits):
        for a, ax in enumerate((3, 2, 1)):  # z lowest, then y, then x
            k |= ((c[:, ax].astype(np.uint64) >> np.uint64(i)) & np.uint64(1)) << np.uint64(3 * i + a)
    return k | (c[:, 0].astype(np.uint64) << np.uint64(3 * bits))


def _check_plan(pkg, dev, coords, batch, shape, dil=(1, 1, 1)):
    m = pkg.build_neighbor_map(torch.from_numpy(coords).to(dev), shape, batch, dil)
    plan = m.gather_plan()
    torch.cuda.synchronize()
    n = len(coords)
    nbr = m.nbr.cpu().numpy()
    rows, count, rbm, lst, slots = _decode(plan, n)
    t = len(count)
    assert np.array_equal(np.sort(rows[:n]), np.arange(n)) and (rows[n:] == -1).all()
    bits = max(int(max(shape) - 1).bit_length(), 0)
    key = _morton(coords, bits)[rows[:n]]
    assert (key[1:] >= key[:-1]).all()
    for ti in range(t):
        r = rows[ti * TILE:(ti + 1) * TILE]
        nb = np.where(r[:, None] >= 0, nbr[np.maximum(r, 0)], -1)  # (64, 27)
        pres = nb >= 0
        assert np.array_equal(rbm[ti], [int((pres[16 * k:16 * k + 16].any(0) << np.arange(27)).sum())
                                        for k in range(4)])
        distinct = np.unique(nb[pres])
        if count[ti] < 0:
            assert len(distinct) > SLOTS - 1
            continue
        used_a, used_b = set(nb[:32][pres[:32]].tolist()), set(nb[32:][pres[32:]].tolist())
        split = count[ti] >= SPLIT
        d = int(count[ti]) & 0xff if split else int(count[ti])
        assert d == len(distinct)
        # split exactly when the tile exceeds the staging and each half fits it
        assert split == (d >= STAGE and len(used_a) < STAGE and len(used_b) < STAGE)
        # expected slot order: own rows, then by first (tap, row) use
        seen, order = set(), []
        for i in range(TILE):
            if r[i] >= 0:
                seen.add(r[i]); order.append(r[i])
        for v in range(27):
            for i in range(TILE):
                e = nb[i, v]
                if v != 13 and e >= 0 and e not in seen:
                    seen.add(e); order.append(e)
        base = np.zeros(TILE, np.int64)
        if split:
            sa, aonly = (int(count[ti]) >> 8) & 0xff, (int(count[ti]) >> 16) & 0xff
            assert sa == len(used_a) and aonly == len(used_a - used_b)
            order = ([e for e in order if e in used_a and e not in used_b] +
                     [e for e in order if e in used_a and e in used_b] +
                     [e for e in order if e in used_b and e not in used_a])
            base[32:] = aonly  # the second half's table stores slot - aonly
        assert np.array_equal(lst[ti, :len(order)], order)
        s = slots[ti].transpose(2, 0, 1).reshape(TILE, 28)[:, :27].astype(np.int64)  # [row][tap]
        got = np.where(s > 0, lst[ti][np.maximum(s + base[:, None] - 1, 0)], -1)
        assert np.array_equal(got, nb)
    return m, count


def test_plan_shell(pkg, dev):
    spec = pkg.workloads.ShellSpec(128, 40.0, 48.0, 1, 0.3, (6, 5))
    coords = pkg.workloads.shell_coords(spec, 3, batch=2)
    print(f"  gather plan shell N={len(coords)} batch 2", flush=True)
    _, count = _check_plan(pkg, dev, coords, 2, (128, 128, 128))
    assert (count >= 0).all() and count.max() < STAGE


def test_plan_dense_blocks_and_ragged_tail(pkg, dev):
    """A dense 12^3 block: interior 4^3 Morton tiles have 216 distinct neighbors (> the staging);
    with dilation 2, 512 (> the list capacity: count -1).  N = 1728 + 37 is not a tile multiple."""
    g = np.stack(np.meshgrid(*[np.arange(12)] * 3, indexing="ij"), -1).reshape(-1, 3) + 8
    extra = np.random.default_rng(1).choice(32 ** 3, 400, replace=False)
    e = np.stack(np.unravel_index(extra, (32, 32, 32)), -1)
    e = e[(e < 8).any(1) | (e >= 20).any(1)][:37]
    xyz = np.concatenate([g, e])
    coords = np.concatenate([np.zeros((len(xyz), 1), np.int64), xyz], 1).astype(np.int32)
    coords = coords[np.random.default_rng(2).permutation(len(coords))]
    print(f"  gather plan dense N={len(coords)}", flush=True)
    _, c1 = _check_plan(pkg, dev, coords, 1, (32, 32, 32))
    assert (c1 >= SPLIT).any()
    _, c2 = _check_plan(pkg, dev, coords, 1, (32, 32, 32), (2, 2, 2))
    assert (c2 < 0).any()


def test_plan_large_morton_buckets(pkg, dev):
    """A dense 32x64x8 block in 512^3 fills one 10-bit Morton prefix (a 32x64x64 cell region)
    with 16384 voxels: four chunks of the bucket kernel's bitmap rank."""
    g = np.stack(np.meshgrid(np.arange(32) + 32, np.arange(64) + 64, np.arange(8) + 128,
                             indexing="ij"), -1).reshape(-1, 3)
    xyz = np.concatenate([g, [[0, 0, 0], [511, 511, 511], [40, 100, 200]]])
    coords = np.concatenate([np.zeros((len(xyz), 1), np.int64), xyz], 1).astype(np.int32)
    coords = coords[np.random.default_rng(6).permutation(len(coords))]
    print(f"  gather plan dense slab in 512^3 N={len(coords)}", flush=True)
    _check_plan(pkg, dev, coords, 1, (512, 512, 512))


def _pair(pkg, dev, coords, batch, shape, ci, co, dtype, epilogue, dil=(1, 1, 1), seed=0):
    m = pkg.build_neighbor_map(torch.from_numpy(coords).to(dev), shape, batch, dil)
    n = len(coords)
    rng = np.random.default_rng(seed)
    f = torch.from_numpy(rng.standard_normal((n, ci)).astype(np.float32)).to(dev).to(dtype)
    w = torch.from_numpy((rng.standard_normal((co, 3, 3, 3, ci)) / np.sqrt(27 * ci)).astype(np.float32)).to(dev).to(dtype)
    b = torch.from_numpy(rng.standard_normal(co).astype(np.float32) * 0.1).to(dev).to(dtype)
    res = torch.from_numpy(rng.standard_normal((n, co)).astype(np.float32)).to(dev).to(dtype)
    kw = dict(epilogue=epilogue, residual=res if epilogue == "residual" else None)
    planned = pkg.sparse_conv3d(f, w, b, m, **kw)                       # through the plan
    direct = pkg.sparse_conv3d(f, w, b, m, order=m.conv_order(), **kw)  # the unplanned kernels
    torch.cuda.synchronize()
    return m, f, w, b, res, planned, direct


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("co", [32, 64])
@pytest.mark.parametrize("epilogue", ["bias", "residual", "ln_silu"])
def test_planned_equals_direct_map512(pkg, dev, dtype, co, epilogue):
    coords = pkg.workloads.make_coords("map512")
    print(f"  planned conv map512 N={len(coords)} 32->{co} {dtype} {epilogue}", flush=True)
    *_, planned, direct = _pair(pkg, dev, coords, 1, (512, 512, 512), 32, co, dtype, epilogue)
    assert torch.equal(planned, direct)


@pytest.mark.parametrize("dil", [(1, 1, 1), (2, 2, 2)])
def test_planned_fallback_tiles_match(pkg, dev, dil):
    """Dense block: tiles over the staging run as two 32-row halves (dilation 1), tiles over the
    list (dilation 2) take the neighbor-map path inside the planned kernel; results still equal
    the direct kernels and the fp64 oracle."""
    g = np.stack(np.meshgrid(*[np.arange(12)] * 3, indexing="ij"), -1).reshape(-1, 3) + 4
    coords = np.concatenate([np.zeros((len(g), 1), np.int64), g], 1).astype(np.int32)
    coords = coords[np.random.default_rng(4).permutation(len(coords))]
    print(f"  planned conv dense block dil={dil}", flush=True)
    m, f, w, b, res, planned, direct = _pair(pkg, dev, coords, 1, (24, 24, 24), 32, 64,
                                             torch.bfloat16, "residual", dil)
    assert torch.equal(planned, direct)
    ref = oracle.conv(f.double().cpu().numpy(), w.double().cpu().numpy(), b.double().cpu().numpy(),
                      m.nbr.cpu().numpy()) + res.double().cpu().numpy()
    err = np.abs(planned.double().cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= 2e-2, err


@pytest.mark.parametrize("n", [1, 63, 64, 65, 1000])
def test_planned_small_and_ragged(pkg, dev, n):
    rng = np.random.default_rng(n)
    flat = rng.choice(16 ** 3 * 2, n, replace=False)
    b, rest = np.divmod(flat, 16 ** 3)
    xyz = np.stack(np.unravel_index(rest, (16, 16, 16)), -1)
    coords = np.concatenate([b[:, None], xyz], 1).astype(np.int32)
    print(f"  planned conv small N={n}", flush=True)
    m, f, w, bias, res, planned, direct = _pair(pkg, dev, coords, 2, (16, 16, 16), 32, 32,
                                                torch.float16, "bias", seed=n)
    assert torch.equal(planned, direct)
    ref = oracle.conv(f.double().cpu().numpy(), w.double().cpu().numpy(),
                      bias.double().cpu().numpy(), m.nbr.cpu().numpy())
    err = np.abs(planned.double().cpu().numpy() - ref).max() / max(np.abs(ref).max(), 1e-30)
    assert err <= 2e-2, err


def test_plan_other_shapes_use_plan_order(pkg, dev):
    """tsc_conv_planned on a shape the planned kernel does not cover (fp32, Ci = 64) runs the
    direct kernels in the plan's row order: same results as the default order."""
    import ctypes
    coords = pkg.workloads.make_coords("conv64_f32")
    m = pkg.build_neighbor_map(torch.from_numpy(coords).to(dev), pkg.workloads.grid_shape("conv64_f32"), 1)
    n = len(coords)
    rng = np.random.default_rng(9)
    f = torch.from_numpy(rng.standard_normal((n, 64)).astype(np.float32)).to(dev)
    w = torch.from_numpy(rng.standard_normal((64, 3, 3, 3, 64)).astype(np.float32) * 0.02).to(dev)
    ref = pkg.sparse_conv3d(f, w, None, m)
    out = torch.empty_like(ref)
    plan = m.gather_plan()
    ctx = pkg._lib.context(dev.index)
    print(f"  planned entry, fp32 64->64 N={n}", flush=True)
    pkg._lib.check(ctx.lib.tsc_conv_planned(ctx.bind(), 0, f.data_ptr(), w.data_ptr(), None,
                                            m.nbr.data_ptr(), plan.data_ptr(), n, 64, 64, 0, None,
                                            None, None, ctypes.c_float(0.0), out.data_ptr()))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_plan_64bit_morton_keys(pkg, dev):
    """A 2048^3 grid with two samples: 34-bit Morton keys take the 64-bit sort."""
    g = np.stack(np.meshgrid(*[np.arange(10)] * 3, indexing="ij"), -1).reshape(-1, 3)
    xyz = np.concatenate([g + 1500, g + 37, g * 3 + 900])
    b = np.repeat([0, 1, 1], len(g))[:, None]
    coords = np.concatenate([b, xyz], 1).astype(np.int32)
    coords = coords[np.random.default_rng(5).permutation(len(coords))]
    print(f"  gather plan 2048^3 x2 N={len(coords)}", flush=True)
    _check_plan(pkg, dev, coords, 2, (2048, 2048, 2048))
    *_, planned, direct = _pair(pkg, dev, coords, 2, (2048, 2048, 2048), 32, 32, torch.float16,
                                "bias")
    assert torch.equal(planned, direct)


@pytest.mark.parametrize("co", [32, 64])
def test_planned_two_voxel_shell_split_tiles(pkg, dev, co):
    """A 2-voxel shell (what subdividing a 1-voxel shell gives): ~6 % of its Morton tiles exceed
    the staging and run as split tiles, a few exceed it per half too.  Planned = direct, bit for
    bit, and the plan marks both kinds."""
    spec = pkg.workloads.ShellSpec(128, 50.0, 62.0, 2, 0.35, (10, 8))
    coords = pkg.workloads.shell_coords(spec, 21, 1)
    print(f"  planned conv 2-voxel shell N={len(coords)} 32->{co}", flush=True)
    m, *_, planned, direct = _pair(pkg, dev, coords, 1, (128, 128, 128), 32, co, torch.float16,
                                   "residual", seed=co)
    assert torch.equal(planned, direct)
    _, count, *_ = _decode(m.gather_plan(), len(coords))
    assert (count >= SPLIT).sum() > 10


@pytest.mark.parametrize("co", [32, 64])
def test_planned_residual_in_place(pkg, dev, co):
    """The planned kernel's epilogue exchanges columns between lanes before its row stores, so an
    output that aliases the residual is read and written by different lanes: in place (out is the
    residual) must give the bits of the separate output, split tiles included."""
    spec = pkg.workloads.ShellSpec(128, 50.0, 62.0, 2, 0.35, (10, 8))
    coords = pkg.workloads.shell_coords(spec, 23, 1)
    print(f"  planned conv in place N={len(coords)} 32->{co}", flush=True)
    m, f, w, b, res, planned, _ = _pair(pkg, dev, coords, 1, (128, 128, 128), 32, co,
                                        torch.bfloat16, "residual", seed=5 + co)
    r2 = res.clone()
    out = pkg.sparse_conv3d(f, w, b, m, epilogue="residual", residual=r2, out=r2)
    torch.cuda.synchronize()
    assert out.data_ptr() == r2.data_ptr()
    assert torch.equal(r2, planned)


def test_plan_two_voxel_shell_layout(pkg, dev):
    """The plan of a small 2-voxel shell against its definition, split tiles included."""
    spec = pkg.workloads.ShellSpec(64, 24.0, 30.0, 2, 0.35, (10, 8))
    coords = pkg.workloads.shell_coords(spec, 22, 1)
    print(f"  gather plan 2-voxel shell N={len(coords)}", flush=True)
    _, count = _check_plan(pkg, dev, coords, 1, (64, 64, 64))
    assert (count >= SPLIT).any()
