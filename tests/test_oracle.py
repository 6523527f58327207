"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the HIP path.

Every oracle function is checked against something that does not share its code:
  * map build: brute force (dict), the dense-grid restatement, the torch.sort+searchsorted
    restatement, numpy.unique for sorted keys, symmetry / self-tap invariants, known patterns;
  * conv: the dense torch F.conv3d closed form (README.md:81) and exact special cases;
  * LayerNorm / SiLU: torch.nn.functional in float64;
  * all of them: the committed golden fixtures (generated without oracle/).
Planted-mistake checks at the end confirm these tests can fail.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import brute, torch_path
from tests import _golden

torch.set_num_threads(4)


def _random_coords(rng, batch, shape, n_per):
    rows = []
    for b in range(batch):
        cells = rng.choice(shape[0] * shape[1] * shape[2], size=n_per, replace=False)
        x, rem = np.divmod(cells, shape[1] * shape[2])
        y, z = np.divmod(rem, shape[2])
        rows.append(np.stack([np.full(n_per, b), x, y, z], 1))
    c = np.concatenate(rows).astype(np.int32)
    return c[rng.permutation(len(c))]


def _dense_conv(coords, feats, weight, bias, shape, dil, batch):
    X, Y, Z = shape
    ci, co = weight.shape[4], weight.shape[0]
    w = torch.from_numpy(np.asarray(weight, np.float64)).permute(0, 4, 1, 2, 3).contiguous()
    out = np.zeros((len(coords), co))
    for b in range(batch):
        rows = np.nonzero(coords[:, 0] == b)[0]
        grid = torch.zeros((1, ci, X, Y, Z), dtype=torch.float64)
        c = torch.from_numpy(coords[rows].astype(np.int64))
        grid[0, :, c[:, 1], c[:, 2], c[:, 3]] = torch.from_numpy(np.asarray(feats[rows], np.float64)).T
        y = F.conv3d(grid, w, None, padding=tuple(dil), dilation=tuple(dil))
        out[rows] = y[0, :, c[:, 1], c[:, 2], c[:, 3]].T.numpy()
    return out if bias is None else out + np.asarray(bias, np.float64)


@pytest.mark.parametrize("seed,batch,shape,n_per,dil", [
    (0, 1, (6, 6, 6), 80, (1, 1, 1)),
    (1, 2, (7, 5, 9), 120, (1, 1, 1)),
    (2, 3, (8, 8, 8), 200, (2, 1, 3)),
    (3, 1, (4, 4, 4), 64, (1, 1, 1)),      # completely full grid
    (4, 2, (9, 3, 11), 90, (3, 2, 1)),
])
def test_map_three_ways_agree(seed, batch, shape, n_per, dil):
    rng = np.random.default_rng(seed)
    coords = _random_coords(rng, batch, shape, n_per)
    st, keys, perm, nbr = oracle.map_sorted(coords, batch, shape, dil)
    st2, nbr_grid = oracle.map_grid(coords, batch, shape, dil)
    assert st == 0 and st2 == 0
    expect = np.array(brute.neighbor_map(coords.tolist(), shape, dil), np.int32)
    np.testing.assert_array_equal(nbr, expect)
    np.testing.assert_array_equal(nbr_grid, expect)
    packed = oracle.pack_keys(coords, shape)
    np.testing.assert_array_equal(keys, np.unique(packed))
    np.testing.assert_array_equal(packed[perm], keys)
    _, tperm, tnbr = torch_path.hashmap_fallback(torch.from_numpy(coords), shape, dil)
    np.testing.assert_array_equal(tnbr.numpy(), expect)


def test_map_invariants_on_shell(pkg):
    coords = pkg.workloads.make_coords("conv64_f32")
    shape = pkg.workloads.grid_shape("conv64_f32")
    st, keys, perm, nbr = oracle.map_sorted(coords, 1, shape)
    assert st == 0
    n = len(coords)
    np.testing.assert_array_equal(nbr[:, 13], np.arange(n))
    rows, taps = np.nonzero(nbr >= 0)
    # symmetry: nbr[n,v] = m  <=>  nbr[m,26-v] = n
    np.testing.assert_array_equal(nbr[nbr[rows, taps], 26 - taps], rows)
    _, nbr_grid = oracle.map_grid(coords, 1, shape)
    np.testing.assert_array_equal(nbr, nbr_grid)
    _, _, tnbr = torch_path.hashmap_fallback(torch.from_numpy(coords), shape)
    np.testing.assert_array_equal(nbr, tnbr.numpy())
    p = (nbr >= 0).sum()
    assert 14 * n < p < 20 * n  # a 2-voxel shell has ~16-17 neighbors per voxel


def test_map_known_patterns():
    one = np.array([[0, 2, 2, 2]], np.int32)
    _, _, _, nbr = oracle.map_sorted(one, 1, (5, 5, 5))
    assert nbr[0, 13] == 0 and (np.delete(nbr[0], 13) == -1).all()
    block = np.array([[0, x, y, z] for x in range(3) for y in range(3) for z in range(3)], np.int32)
    _, _, _, nbr = oracle.map_sorted(block, 1, (3, 3, 3))
    centre = 13  # row of (1,1,1)
    np.testing.assert_array_equal(nbr[centre], np.arange(27))
    assert (nbr[0] >= 0).sum() == 8  # corner (0,0,0): only the +1 octant
    assert nbr[0, 26] == 13 and nbr[0, 0] == -1  # (0,0,0)+(1,1,1) is row 13; -1 offset is outside
    assert nbr[26, 0] == 13 and nbr[26, 26] == -1
    # batch separation: same xyz in two samples never see each other
    two = np.array([[0, 1, 1, 1], [1, 1, 1, 2]], np.int32)
    _, _, _, nbr = oracle.map_sorted(two, 2, (3, 3, 3))
    assert (nbr[:, [v for v in range(27) if v != 13]] == -1).all()


def test_map_status_bits():
    dup = np.array([[0, 1, 1, 1], [0, 2, 2, 2], [0, 1, 1, 1]], np.int32)
    assert oracle.map_sorted(dup, 1, (4, 4, 4))[0] & oracle.STATUS_DUPLICATE
    assert oracle.map_grid(dup, 1, (4, 4, 4))[0] & oracle.STATUS_DUPLICATE
    oob = np.array([[0, 1, 1, 1], [0, 4, 0, 0], [1, 0, 0, 0], [0, -1, 0, 0]], np.int32)
    assert oracle.map_sorted(oob, 1, (4, 4, 4))[0] == oracle.STATUS_OUT_OF_RANGE
    assert oracle.map_grid(oob, 1, (4, 4, 4))[0] == oracle.STATUS_OUT_OF_RANGE


@pytest.mark.parametrize("seed,batch,shape,n_per,ci,co,dil,bias", [
    (0, 2, (8, 8, 8), 150, 8, 16, (1, 1, 1), True),
    (1, 1, (9, 7, 10), 250, 5, 3, (2, 1, 3), False),
    (2, 3, (6, 6, 6), 100, 16, 8, (1, 2, 1), True),
])
def test_conv_matches_dense_conv3d(seed, batch, shape, n_per, ci, co, dil, bias):
    rng = np.random.default_rng(seed)
    coords = _random_coords(rng, batch, shape, n_per)
    feats = rng.standard_normal((len(coords), ci))
    w = rng.standard_normal((co, 3, 3, 3, ci))
    b = rng.standard_normal(co) if bias else None
    _, _, _, nbr = oracle.map_sorted(coords, batch, shape, dil)
    got = oracle.conv(feats, w, b, nbr)
    want = _dense_conv(coords, feats, w, b, shape, dil, batch)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    tp = torch_path.conv_none(torch.from_numpy(feats), torch.from_numpy(w),
                              None if b is None else torch.from_numpy(b), torch.from_numpy(nbr),
                              acc_dtype=torch.float64)
    np.testing.assert_allclose(tp.numpy(), want, rtol=1e-12, atol=1e-12)


def test_conv_special_cases(pkg):
    coords = pkg.workloads.make_coords("conv64_f32")[:3000]
    _, _, _, nbr = oracle.map_sorted(coords, 1, (64, 64, 64))
    n = len(coords)
    # all-ones weight, Ci=Co=1, ones input: the output is the neighbor count, exactly.
    out = oracle.conv(np.ones((n, 1)), np.ones((1, 27, 1)), None, nbr)
    np.testing.assert_array_equal(out[:, 0], (nbr >= 0).sum(1))
    # one-hot weight at tap v: out[n] = feats[nbr[n,v]] (or 0): a shift.
    rng = np.random.default_rng(7)
    f = rng.standard_normal((n, 4))
    for v in (0, 13, 22):
        w = np.zeros((4, 27, 4))
        w[:, v, :] = np.eye(4)
        out = oracle.conv(f, w, None, nbr)
        want = np.where(nbr[:, v:v + 1] >= 0, f[np.maximum(nbr[:, v], 0)], 0.0)
        np.testing.assert_array_equal(out, want)
    # zero weight: bias only.
    b = rng.standard_normal(4)
    np.testing.assert_array_equal(oracle.conv(f, np.zeros((4, 27, 4)), b, nbr), np.tile(b, (n, 1)))


def test_layernorm_and_silu_vs_torch():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((50, 130)) * 2 + 1
    g, b = rng.uniform(0.5, 2, 130), rng.standard_normal(130)
    xt = torch.from_numpy(x)
    want = F.layer_norm(xt, (130,), torch.from_numpy(g), torch.from_numpy(b), eps=1e-6)
    np.testing.assert_allclose(oracle.layernorm(x, g, b, 1e-6), want.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.layernorm(x, g, b, 1e-6, silu=True), F.silu(want).numpy(),
                               rtol=1e-12, atol=1e-12)
    want0 = F.layer_norm(xt, (130,), eps=1e-6)
    np.testing.assert_allclose(oracle.layernorm(x, eps=1e-6), want0.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.silu(x), F.silu(xt).numpy(), rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("case", ["shell_b2", "random_dil213"])
def test_oracle_matches_golden_maps_and_convs(case):
    md, a = _golden.load(case)
    coords = a[("in", "coords")]
    batch = int(md["metadata"]["batch"])
    shape = _golden.meta_tuple(md, "spatial_shape")
    dil = _golden.meta_tuple(md, "dilation")
    st, keys, perm, nbr = oracle.map_sorted(coords, batch, shape, dil)
    assert st == 0
    np.testing.assert_array_equal(nbr, a[("exp", "nbr")])
    if ("exp", "sorted_keys") in a:
        np.testing.assert_array_equal(keys, a[("exp", "sorted_keys")])
    bias = a.get(("in", "bias"))
    out = oracle.conv(a[("in", "feats")], a[("in", "weight")], bias, nbr)
    np.testing.assert_allclose(out, a[("exp", "conv_out")], rtol=1e-10, atol=1e-10)


def test_oracle_matches_golden_layernorm():
    md, a = _golden.load("layernorm_silu")
    x, g, b = a[("in", "x")], a[("in", "gamma")], a[("in", "beta")]
    np.testing.assert_allclose(oracle.layernorm(x, g, b, 1e-6), a[("exp", "ln")], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.layernorm(x, g, b, 1e-6, silu=True), a[("exp", "ln_silu")],
                               rtol=1e-12, atol=1e-12)


def test_planted_mistakes_are_caught():
    """A transposed tap order, a wrong sign of the offset or a dropped bias must fail the checks
    above; plant each in a copy of the oracle's output and confirm the comparisons notice."""
    md, a = _golden.load("shell_b2")
    coords, expect = a[("in", "coords")], a[("exp", "nbr")]
    _, _, _, nbr = oracle.map_sorted(coords, 2, (14, 14, 14))
    assert not np.array_equal(nbr[:, ::-1], expect)                      # offset sign flipped
    swapped = nbr.reshape(-1, 3, 3, 3).transpose(0, 3, 2, 1).reshape(-1, 27)
    assert not np.array_equal(swapped, expect)                           # kd/kw transposed
    out = oracle.conv(a[("in", "feats")], a[("in", "weight")], None, nbr)
    assert not np.allclose(out, a[("exp", "conv_out")], rtol=1e-6, atol=1e-6)  # bias dropped
    w_t = a[("in", "weight")].transpose(0, 3, 2, 1, 4)
    out_t = oracle.conv(a[("in", "feats")], w_t, a[("in", "bias")], nbr)
    assert not np.allclose(out_t, a[("exp", "conv_out")], rtol=1e-6, atol=1e-6)  # kernel transposed


# ---- subdivision (decoder upsample) ---------------------------------------------------------

def _unique_coords(rng, n, batch, shape):
    cells = rng.choice(batch * shape[0] * shape[1] * shape[2], size=n, replace=False)
    b, r = np.divmod(cells, shape[0] * shape[1] * shape[2])
    x, r = np.divmod(r, shape[1] * shape[2])
    y, z = np.divmod(r, shape[2])
    return np.stack([b, x, y, z], axis=1).astype(np.int32)


def test_subdivide_parent_and_child_index_of_every_row():
    rng = np.random.default_rng(3)
    c = _unique_coords(rng, 300, 3, (9, 7, 11))
    f = rng.standard_normal((300, 5)).astype(np.float32)
    kids, kf = oracle.subdivide(c, f)
    assert kids.shape == (2400, 4)
    rows = np.arange(2400)
    par = c[rows // 8]
    np.testing.assert_array_equal(kids[:, 0], par[:, 0])
    np.testing.assert_array_equal(kids[:, 1:] // 2, par[:, 1:])
    child = (kids[:, 1] & 1) * 4 + (kids[:, 2] & 1) * 2 + (kids[:, 3] & 1)
    np.testing.assert_array_equal(child, rows % 8)
    np.testing.assert_array_equal(kf, f[rows // 8])


def test_subdivide_children_are_the_doubled_cells_inside_parents():
    """Brute force over every cell of the doubled grid."""
    rng = np.random.default_rng(4)
    shape = (3, 4, 2)
    c = _unique_coords(rng, 7, 2, shape)
    parents = {tuple(r) for r in c.tolist()}
    want = {(b, x, y, z) for b in range(2) for x in range(6) for y in range(8) for z in range(4)
            if (b, x // 2, y // 2, z // 2) in parents}
    kids, _ = oracle.subdivide(c)
    got = [tuple(r) for r in kids.tolist()]
    assert len(got) == len(set(got)) == 8 * len(c)
    assert set(got) == want


def test_subdivide_dense_block_and_keep_masks():
    block = np.array([[0, x, y, z] for x in range(2) for y in range(2) for z in range(2)], np.int32)
    kids, _ = oracle.subdivide(block)
    assert {tuple(r) for r in kids.tolist()} == {(0, x, y, z) for x in range(4) for y in range(4)
                                                 for z in range(4)}
    rng = np.random.default_rng(5)
    c = _unique_coords(rng, 50, 1, (6, 6, 6))
    f = rng.standard_normal((50, 3)).astype(np.float32)
    full, ff = oracle.subdivide(c, f)
    # eight single-child masks interleave back into the full subdivision
    singles = [oracle.subdivide(c, f, np.full(50, 1 << ch, np.uint8)) for ch in range(8)]
    inter = np.stack([s[0] for s in singles], axis=1).reshape(-1, 4)
    np.testing.assert_array_equal(inter, full)
    np.testing.assert_array_equal(np.stack([s[1] for s in singles], axis=1).reshape(-1, 3), ff)
    # a random mask keeps exactly its set bits, in parent-major order
    keep = rng.integers(0, 256, size=50).astype(np.uint8)
    kk, kf = oracle.subdivide(c, f, keep)
    bits = np.unpackbits(keep[:, None], axis=1, bitorder="little").astype(bool).reshape(-1)
    np.testing.assert_array_equal(kk, full[bits])
    np.testing.assert_array_equal(kf, ff[bits])
    assert oracle.subdivide(c, None, np.zeros(50, np.uint8))[0].shape == (0, 4)


def test_linear_vs_torch_functional():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((40, 24))
    w = rng.standard_normal((12, 24))
    b = rng.standard_normal(12)
    r = rng.standard_normal((40, 12))
    want = F.linear(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b)).numpy()
    np.testing.assert_allclose(oracle.linear(x, w, b), want, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.linear(x, w, b, r), want + r, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.linear(x, w), x @ w.T, rtol=1e-12, atol=1e-12)
    # a transposed weight is caught
    assert not np.allclose(oracle.linear(x[:, :12], w[:, :12].T.copy()), x[:, :12] @ w[:, :12].T)


def test_convnext_block_composition_and_store_rounding():
    """oracle.convnext_block against the same five steps composed from torch.nn.functional (fp64;
    the conv from oracle.conv, pinned above by the dense closed form), and its `store` rounding:
    identity changes nothing, bf16 rounding leaves bf16-representable outputs within a few bf16
    ulps of the unrounded block, and a planted step order (linear before the first LayerNorm) is
    caught."""
    rng = np.random.default_rng(19)
    coords = np.unique(rng.integers(0, 6, (120, 3)), axis=0)
    coords = np.concatenate([np.zeros((len(coords), 1), np.int64), coords], 1).astype(np.int32)
    _, _, _, nbr = oracle.map_sorted(coords, 1, (6, 6, 6))
    n, c, hid = len(coords), 8, 16
    x = rng.standard_normal((n, c))
    cw = rng.standard_normal((c, 3, 3, 3, c)) / np.sqrt(27 * c)
    cb, w0, b0 = rng.standard_normal(c), rng.standard_normal((hid, c)), rng.standard_normal(hid)
    w2, b2 = rng.standard_normal((c, hid)), rng.standard_normal(c)
    T = torch.from_numpy
    h = T(oracle.conv(x, cw, cb, nbr))
    h = F.layer_norm(h, (c,), eps=1e-6)
    h = F.linear(h, T(w0), T(b0))
    h = F.silu(F.layer_norm(h, (hid,), eps=1e-6))
    want = (T(x) + F.linear(h, T(w2), T(b2))).numpy()
    got = oracle.convnext_block(x, nbr, cw, cb, w0, b0, w2, b2, 1e-6)
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10)
    assert np.array_equal(oracle.convnext_block(x, nbr, cw, cb, w0, b0, w2, b2, 1e-6,
                                                store=lambda a: a), got)

    def to_bf16(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).double().numpy()
    rounded = oracle.convnext_block(x, nbr, cw, cb, w0, b0, w2, b2, 1e-6, store=to_bf16)
    assert np.array_equal(to_bf16(rounded), rounded)
    err = np.abs(rounded - got).max() / np.abs(got).max()
    assert 0 < err < 5e-2, err
    rows = np.array([3, 7, 50])
    assert np.array_equal(oracle.convnext_block(x, nbr, cw, cb, w0, b0, w2, b2, 1e-6, rows=rows,
                                                store=to_bf16), rounded[rows])
    # planted: the first linear before the first LayerNorm
    hp = F.linear(T(oracle.conv(x, cw, cb, nbr)), T(w0), T(b0))
    hp = F.silu(F.layer_norm(hp, (hid,), eps=1e-6))
    planted = (T(x) + F.linear(hp, T(w2), T(b2))).numpy()
    assert not np.allclose(planted, got, rtol=1e-3, atol=1e-3)
