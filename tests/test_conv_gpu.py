"""Sparse conv on the GPU vs the fp64 oracle.

Tolerance (norm-wise relative, max|y - r| / max|r|, r computed in fp64 from the same rounded
inputs and weights): fp32 <= 1e-4, fp16 / bf16 <= 2e-2.  The workload convs also assert the
per-element allclose with atol = rtol * rms(r) (tests/_tol.py) and print both.
"""
import numpy as np
import pytest
import torch

import oracle
from tests import _golden, _tol

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def _rounded(a, dtype, dev):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dtype)
    return t, t.float().cpu().numpy().astype(np.float64)


def _map(pkg, dev, coords, batch, shape, dil=(1, 1, 1)):
    return pkg.build_neighbor_map(torch.from_numpy(coords).to(dev), shape, batch, dil)


@pytest.mark.parametrize("case", ["shell_b2", "random_dil213"])
def test_conv_golden_fp32(pkg, dev, case):
    md, a = _golden.load(case)
    coords = a[("in", "coords")]
    m = _map(pkg, dev, coords, int(md["metadata"]["batch"]), _golden.meta_tuple(md, "spatial_shape"),
             _golden.meta_tuple(md, "dilation"))
    f = torch.from_numpy(a[("in", "feats")]).to(dev)
    w = torch.from_numpy(a[("in", "weight")]).to(dev)
    b = a.get(("in", "bias"))
    b = None if b is None else torch.from_numpy(b).to(dev)
    print(f"  conv golden {case} N={len(coords)} Ci={f.shape[1]} Co={w.shape[0]}", flush=True)
    out = pkg.sparse_conv3d(f, w, b, m)
    err = rel_err(out.cpu().numpy(), a[("exp", "conv_out")])
    assert err <= 1e-4, err


def _workload_conv(pkg, dev, workload, ci, co, dtype, sample_rows=None, seed=0, bias=True):
    coords = pkg.workloads.make_coords(workload)
    batch = int(coords[:, 0].max()) + 1
    shape = pkg.workloads.grid_shape(workload)
    n = len(coords)
    print(f"  conv {workload} N={n} {ci}->{co} {dtype}", flush=True)
    m = _map(pkg, dev, coords, batch, shape)
    f, f64 = _rounded(pkg.workloads.features(n, ci, seed), dtype, dev)
    w, w64 = _rounded(pkg.workloads.conv_weight(co, ci, seed + 1), dtype, dev)
    bnp = np.random.default_rng(seed + 2).standard_normal(co).astype(np.float32) * 0.1
    b, b64 = _rounded(bnp, dtype, dev) if bias else (None, None)
    out = pkg.sparse_conv3d(f, w, b, m).float().cpu().numpy()
    nbr = m.nbr.cpu().numpy()
    rows = np.arange(n)
    if sample_rows is not None and sample_rows < n:
        rows = np.sort(np.random.default_rng(seed + 3).choice(n, sample_rows, replace=False))
    ref = oracle.conv(f64, w64, b64, nbr[rows])
    # both halves of the tolerance definition: norm-wise (returned, asserted by the caller) and
    # per-element allclose with atol = rtol * rms(r) (asserted here, printed beside it)
    _tol.check(out[rows], ref, TOL[dtype], f"{workload} {ci}->{co} {dtype}")
    return rel_err(out[rows], ref), m, (f, w, b), out


def test_conv_fp32_64_full(pkg, dev):
    err, *_ = _workload_conv(pkg, dev, "conv64_f32", 64, 64, torch.float32)
    assert err <= TOL[torch.float32], err


@pytest.mark.parametrize("ci,co", [(32, 32), (32, 64)])
def test_conv_fp16_narrow_full_size(pkg, dev, ci, co):
    err, *_ = _workload_conv(pkg, dev, "narrow512_f16", ci, co, torch.float16, sample_rows=20000)
    assert err <= TOL[torch.float16], err


@pytest.mark.parametrize("ci,co", [(32, 32), (32, 64)])
def test_conv_fp32_narrow_full_size(pkg, dev, ci, co):
    """fp32 32->32 runs the wave-tile kernel on v_mfma_f32_16x16x4f32; 32->64 the tile path."""
    err, *_ = _workload_conv(pkg, dev, "narrow512_f16", ci, co, torch.float32, sample_rows=20000)
    assert err <= TOL[torch.float32], err


def test_conv_fp32_narrow_residual_in_place(pkg, dev):
    """fp32 narrow kernel epilogue: bias + residual, out aliasing the residual (16-byte stores)."""
    coords = pkg.workloads.make_coords("conv64_f32")
    n = len(coords)
    m = _map(pkg, dev, coords, int(coords[:, 0].max()) + 1, pkg.workloads.grid_shape("conv64_f32"))
    nbr = m.nbr.cpu().numpy()
    dt = torch.float32
    f, f64 = _rounded(pkg.workloads.features(n, 32, 4), dt, dev)
    w, w64 = _rounded(pkg.workloads.conv_weight(32, 32, 5), dt, dev)
    b, b64 = _rounded(np.linspace(-1, 1, 32).astype(np.float32), dt, dev)
    r, r64 = _rounded(pkg.workloads.features(n, 32, 6), dt, dev)
    print(f"  conv fp32 narrow residual N={n}", flush=True)
    base = oracle.conv(f64, w64, b64, nbr)
    r2 = r.clone()
    pkg.sparse_conv3d(f, w, b, m, epilogue="residual", residual=r2, out=r2)
    assert rel_err(r2.cpu().numpy(), base + r64) <= 1e-4
    out = pkg.sparse_conv3d(f, w, None, m)
    assert rel_err(out.cpu().numpy(), oracle.conv(f64, w64, None, nbr)) <= 1e-4


def test_conv_bf16_wide_full_size(pkg, dev):
    err, *_ = _workload_conv(pkg, dev, "wide128_bf16", 512, 512, torch.bfloat16, sample_rows=600)
    assert err <= TOL[torch.bfloat16], err


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("ci,co", [(16, 32), (64, 128), (96, 96), (128, 256), (256, 64)])
def test_conv_dtypes_and_shapes(pkg, dev, dtype, ci, co):
    err, *_ = _workload_conv(pkg, dev, "resblock64_bf16", ci, co, dtype, sample_rows=800)
    assert err <= TOL[dtype], err


@pytest.mark.parametrize("ci,co,rows", [(64, 768, None), (64, 256, 100), (128, 512, 2000)])
def test_conv_wide_tile_schedule(pkg, dev, ci, co, rows):
    """256x256 tiles go through the longest-first schedule: three column tiles per row tile,
    fewer row tiles than XCDs (empty schedule slots), and a partial last tile."""
    coords = pkg.workloads.make_coords("resblock64_bf16")
    if rows is not None:
        coords = coords[coords[:, 0] == 0][:rows]
    n = len(coords)
    batch = int(coords[:, 0].max()) + 1
    print(f"  conv schedule N={n} {ci}->{co}", flush=True)
    m = _map(pkg, dev, coords, batch, (64, 64, 64))
    dt = torch.bfloat16
    f, f64 = _rounded(pkg.workloads.features(n, ci, 4), dt, dev)
    w, w64 = _rounded(pkg.workloads.conv_weight(co, ci, 5), dt, dev)
    out = pkg.sparse_conv3d(f, w, None, m).float().cpu().numpy()
    nbr = m.nbr.cpu().numpy()
    sel = np.sort(np.random.default_rng(6).choice(n, min(n, 700), replace=False))
    ref = oracle.conv(f64, w64, None, nbr[sel])
    assert rel_err(out[sel], ref) <= TOL[dt]
    again = pkg.sparse_conv3d(f, w, None, m.nbr, order=m.perm)
    assert torch.equal(again.float().cpu(), torch.from_numpy(out))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_conv_order_invariance_bit_exact(pkg, dev, dtype):
    coords = pkg.workloads.make_coords("conv64_f32")
    n = len(coords)
    m = _map(pkg, dev, coords, 1, (64, 64, 64))
    f = torch.from_numpy(pkg.workloads.features(n, 64, 5)).to(dev).to(dtype)
    w = torch.from_numpy(pkg.workloads.conv_weight(128, 64, 6)).to(dev).to(dtype)
    ident = pkg.sparse_conv3d(f, w, None, m.nbr)
    sorted_ = pkg.sparse_conv3d(f, w, None, m)
    rnd = torch.from_numpy(np.random.default_rng(1).permutation(n).astype(np.int32)).to(dev)
    shuffled = pkg.sparse_conv3d(f, w, None, m.nbr, order=rnd)
    keyorder = pkg.sparse_conv3d(f, w, None, m.nbr, order=m.perm)
    assert torch.equal(ident, sorted_) and torch.equal(ident, shuffled)
    assert torch.equal(ident, keyorder)


def _order_model(present, perm):
    """CPU model of tsc_map_conv_order: (order, Gray rank of every row's mask, sorted order)."""
    n = len(present)
    # taps by the number of offset coordinates that are not 0 (3 = corner, 2 = edge, 1 = face)
    cls = [sum(c != 1 for c in (v // 9, v // 3 % 3, v % 3)) for v in range(27)]
    taps = sorted((v for v in range(27) if v != 13), key=lambda v: (-cls[v], v))
    assert taps[:8] == [0, 2, 6, 8, 18, 20, 24, 26] and len(taps) == 26
    m26 = np.zeros(n, np.int64)
    for v in taps:
        m26 = (m26 << 1) | present[:, v]
    # rank of m26 read as a reflected binary (Gray) code: bit i of the rank is the XOR of bits
    # i..25 of the code
    rank = np.zeros(n, np.int64)
    for i in range(26):
        rank |= (np.bitwise_xor.reduce([(m26 >> j) & 1 for j in range(i, 26)], axis=0)) << i
    assert rank[m26 == 0].max(initial=0) == 0
    srt = np.empty(n, np.int64)
    win = 262144
    for w0 in range(0, n, win):
        rows = perm[w0:w0 + win]
        srt[w0:w0 + win] = rows[np.argsort(rank[rows], kind="stable")]
    return _greedy_tiles(srt, rank[srt]), rank, srt


@pytest.mark.parametrize("workload", ["map512", "wide128_bf16", "conv64_f32"])
def test_map_conv_order(pkg, dev, workload):
    """The conv order: inside each window of 262144 consecutive key-sorted rows, rows sorted by the
    Gray-sequence rank of their 26-bit mask of present neighbors (corner taps in the top bits, then
    edges, then faces, each class in tap order; tap 13 left out), ties in key order; then inside
    each chunk of 4096 sorted rows, 256-row tiles regrouped greedily (_greedy_tiles).  Exact
    match, and the regrouping never raises the taps the 256-row tiles process."""
    coords = pkg.workloads.make_coords(workload)
    batch = int(coords[:, 0].max()) + 1
    m = _map(pkg, dev, coords, batch, pkg.workloads.grid_shape(workload))
    print(f"  conv order {workload} N={len(coords)}", flush=True)
    order = m.conv_order().cpu().numpy()
    n = len(coords)
    want, rank, srt = _order_model(m.nbr.cpu().numpy() >= 0, m.perm.cpu().numpy())
    np.testing.assert_array_equal(order, want)
    assert np.array_equal(np.sort(order), np.arange(n))
    mask = (rank ^ (rank >> 1))[order], (rank ^ (rank >> 1))[srt]  # neighbor masks (ranks -> codes)
    taps = [_tile_taps(x, 256) for x in mask]
    assert taps[0] <= taps[1], taps


@pytest.mark.parametrize("rows", [200, None])
def test_map_conv_order_without_perm(pkg, dev, rows):
    """perm = NULL orders rows 0..N-1 as given (the same as passing the identity), on ragged
    sizes: a 200-row map (every kernel's only block partial) and the conv64 set (25 k rows, no
    multiple of the 256-, 4096- or 16384-row tiles)."""
    coords = pkg.workloads.make_coords("conv64_f32")
    if rows is not None:
        coords = coords[:rows]
    m = _map(pkg, dev, coords, 1, pkg.workloads.grid_shape("conv64_f32"))
    n = len(coords)
    print(f"  conv order without perm N={n}", flush=True)
    got = pkg.map_conv_order(m.nbr, None).cpu().numpy()
    ident = torch.arange(n, dtype=torch.int32, device=dev)
    np.testing.assert_array_equal(got, pkg.map_conv_order(m.nbr, ident).cpu().numpy())
    want, _, _ = _order_model(m.nbr.cpu().numpy() >= 0, np.arange(n))
    np.testing.assert_array_equal(got, want)


def _popcount(a):
    a = np.asarray(a, np.int64)
    c = np.zeros_like(a)
    for b in range(26):
        c += (a >> b) & 1
    return c


def _tile_taps(masks, tile):
    """Taps processed by `tile`-row tiles: popcount of each tile's OR, times the tile's rows."""
    t = (len(masks) + tile - 1) // tile
    pad = np.zeros(t * tile, np.int64)
    pad[:len(masks)] = masks
    return int((_popcount(np.bitwise_or.reduce(pad.reshape(t, tile), axis=1)) * tile).sum())


def _greedy_tiles(srt, rank, chunk=4096, tile=256):
    """Greedy 256-row tiles inside each chunk of the sorted rows `srt` (Gray ranks `rank`): entries
    = runs of equal rank, ordered by run length capped at 255 (descending), then rank; a tile starts from the
    first entry with rows left (OR = its mask) and takes, in entry order, the rows of every entry
    whose mask lies inside OR; while rows are missing, OR gains the entry mask that adds the fewest
    taps (lowest entry on ties).  Rows of an entry are taken in their sorted order."""
    out = np.empty_like(srt)
    for c0 in range(0, len(srt), chunk):
        rows, rk = srt[c0:c0 + chunk], rank[c0:c0 + chunk]
        nc = len(rows)
        heads = np.flatnonzero(np.r_[True, rk[1:] != rk[:-1]])
        cnt = np.diff(np.r_[heads, nc])
        o = np.lexsort((rk[heads], -np.minimum(cnt, 255)))
        mask = rk[heads][o] ^ (rk[heads][o] >> 1)
        pos, left = heads[o].copy(), cnt[o].copy()
        ptr = 0
        for t0 in range(0, nc, tile):
            need = min(tile, nc - t0)
            src = []
            while left[ptr] == 0:
                ptr += 1
            orm = int(mask[ptr])
            while True:
                for i in np.flatnonzero((left > 0) & ((mask & ~orm) == 0)):
                    take = int(min(left[i], need))
                    src.extend(range(pos[i], pos[i] + take))
                    pos[i] += take
                    left[i] -= take
                    need -= take
                    if need == 0:
                        break
                if need == 0:
                    break
                alive = np.flatnonzero(left > 0)
                orm |= int(mask[alive[np.argmin(_popcount(mask[alive] & ~orm))]])
            out[c0 + t0:c0 + t0 + len(src)] = rows[np.asarray(src)]
    return out


def test_conv_properties(pkg, dev):
    """Exact identities: one-hot weights give a gather; scaling by 2 commutes; zero W = bias."""
    coords = pkg.workloads.make_coords("conv64_f32")
    n = len(coords)
    m = _map(pkg, dev, coords, 1, (64, 64, 64))
    nbr = m.nbr.cpu().numpy()
    f = torch.from_numpy(pkg.workloads.features(n, 32, 9)).to(dev).to(torch.bfloat16)
    for v in (0, 13, 26):
        w = torch.zeros((32, 27, 32))
        w[:, v, :] = torch.eye(32)
        out = pkg.sparse_conv3d(f, w.reshape(32, 3, 3, 3, 32).to(dev).to(torch.bfloat16), None, m)
        idx = torch.from_numpy(np.maximum(nbr[:, v], 0)).to(dev).long()
        want = torch.where(torch.from_numpy(nbr[:, v:v + 1] >= 0).to(dev), f[idx], torch.zeros_like(f[idx]))
        assert torch.equal(out, want), v
    w = torch.from_numpy(pkg.workloads.conv_weight(64, 32, 3)).to(dev).to(torch.bfloat16)
    a = pkg.sparse_conv3d(f, w, None, m)
    b2 = pkg.sparse_conv3d(f * 2, w, None, m)
    assert torch.equal(a.float() * 2, b2.float())
    bias = torch.randn(64, device=dev).to(torch.bfloat16)
    z = pkg.sparse_conv3d(f, torch.zeros_like(w), bias, m)
    assert torch.equal(z, bias.expand(n, 64))


def test_conv_epilogues(pkg, dev):
    coords = pkg.workloads.make_coords("resblock64_bf16")[:4000]
    coords = coords[coords[:, 0] == 0]
    n = len(coords)
    m = _map(pkg, dev, coords, 1, (64, 64, 64))
    nbr = m.nbr.cpu().numpy()
    dt = torch.bfloat16
    f, f64 = _rounded(pkg.workloads.features(n, 256, 1), dt, dev)
    w, w64 = _rounded(pkg.workloads.conv_weight(256, 256, 2), dt, dev)
    b, b64 = _rounded(np.linspace(-1, 1, 256).astype(np.float32), dt, dev)
    r, r64 = _rounded(pkg.workloads.features(n, 256, 3), dt, dev)
    g, g64 = _rounded(np.linspace(0.5, 1.5, 256).astype(np.float32), dt, dev)
    be, be64 = _rounded(np.linspace(-0.2, 0.3, 256).astype(np.float32), dt, dev)
    base = oracle.conv(f64, w64, b64, nbr)
    out = pkg.sparse_conv3d(f, w, b, m, epilogue="residual", residual=r)
    assert rel_err(out.float().cpu().numpy(), base + r64) <= 2e-2
    out = pkg.sparse_conv3d(f, w, b, m, epilogue="ln_silu", ln_weight=g, ln_bias=be, eps=1e-6)
    ref = oracle.layernorm(base, g64, be64, 1e-6, silu=True)
    assert rel_err(out.float().cpu().numpy(), ref) <= 2e-2
    # in place: out aliases the residual
    r2 = r.clone()
    pkg.sparse_conv3d(f, w, b, m, epilogue="residual", residual=r2, out=r2)
    assert rel_err(r2.float().cpu().numpy(), base + r64) <= 2e-2


def _small_map(pkg, dev, n_keep=3000):
    coords = pkg.workloads.make_coords("conv64_f32")[:n_keep]
    return coords, _map(pkg, dev, coords, 1, (64, 64, 64))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("ci,co", [(1, 1), (3, 7), (13, 48), (40, 72), (8, 32), (32, 48),
                                   (24, 100)])
def test_conv_any_channels(pkg, dev, dtype, ci, co):
    """Channel counts the tuned kernels do not take (rows not a multiple of 32 bytes, Co not a
    multiple of 32) run the generic kernel: zero-padded K tail, masked Co tail.  The reference
    shader accepts any Ci and Co (conv3d_wgsl.ts:174-196)."""
    coords, m = _small_map(pkg, dev)
    n = len(coords)
    nbr = m.nbr.cpu().numpy()
    print(f"  conv any channels N={n} {ci}->{co} {dtype}", flush=True)
    f, f64 = _rounded(pkg.workloads.features(n, ci, ci), dtype, dev)
    w, w64 = _rounded(pkg.workloads.conv_weight(co, ci, co), dtype, dev)
    b, b64 = _rounded(np.linspace(-0.5, 0.5, co).astype(np.float32), dtype, dev)
    out = pkg.sparse_conv3d(f, w, b, m).float().cpu().numpy()
    assert rel_err(out, oracle.conv(f64, w64, b64, nbr)) <= TOL[dtype]
    r, r64 = _rounded(pkg.workloads.features(n, co, 7), dtype, dev)
    out = pkg.sparse_conv3d(f, w, None, m, epilogue="residual", residual=r).float().cpu().numpy()
    assert rel_err(out, oracle.conv(f64, w64, None, nbr) + r64) <= TOL[dtype]
    g, g64 = _rounded(np.linspace(0.5, 1.5, co).astype(np.float32), dtype, dev)
    out = pkg.sparse_conv3d(f, w, b, m, epilogue="ln_silu", ln_weight=g, eps=1e-6)
    ref = oracle.layernorm(oracle.conv(f64, w64, b64, nbr), g64, None, 1e-6, silu=True)
    assert rel_err(out.float().cpu().numpy(), ref) <= TOL[dtype] * (2 if co < 8 else 1)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("ci,co,fused", [(64, 64, True), (48, 64, True), (128, 128, True),
                                         (256, 256, True), (48, 128, False), (64, 512, False)])
def test_conv_ln_silu_epilogue_in_kernel(pkg, dev, dtype, ci, co, fused):
    """Where the conv kernel owns whole output rows (16-bit rows wider than 64 bytes; Co = 64, or
    Co = 128 / 256 with 64-byte K chunks) LayerNorm + SiLU run in its epilogue and no row pass is
    launched; elsewhere the row pass runs.  Either way the result equals the conv followed by the
    LayerNorm row pass bit for bit (with and without gamma / beta), and the fp64 oracle within
    2e-2."""
    coords, m = _small_map(pkg, dev, 5000)
    n = len(coords)
    nbr = m.nbr.cpu().numpy()
    print(f"  conv LN epilogue N={n} {ci}->{co} {dtype}", flush=True)
    f, f64 = _rounded(pkg.workloads.features(n, ci, ci), dtype, dev)
    w, w64 = _rounded(pkg.workloads.conv_weight(co, ci, co), dtype, dev)
    b, b64 = _rounded(np.linspace(-0.5, 0.5, co).astype(np.float32), dtype, dev)
    g, g64 = _rounded(np.linspace(0.5, 1.5, co).astype(np.float32), dtype, dev)
    be, be64 = _rounded(np.linspace(-0.2, 0.3, co).astype(np.float32), dtype, dev)
    ctx = pkg._lib.context(dev.index)
    m.conv_order()
    torch.cuda.synchronize()
    ctx.profile_reset()
    ctx.profile(True)
    out = pkg.sparse_conv3d(f, w, b, m, epilogue="ln_silu", ln_weight=g, ln_bias=be, eps=1e-6)
    ctx.profile(False)
    names = list(ctx.profile_results())
    ctx.profile_reset()
    assert any(",ln>" in k for k in names) == fused, names
    assert any(k.startswith("layernorm") for k in names) == (not fused), names
    plain = pkg.sparse_conv3d(f, w, b, m)
    assert torch.equal(out, pkg.layer_norm(plain, g, be, eps=1e-6, silu=True))
    out2 = pkg.sparse_conv3d(f, w, b, m, epilogue="ln_silu", eps=1e-5)
    assert torch.equal(out2, pkg.layer_norm(plain, None, None, eps=1e-5, silu=True))
    ref = oracle.layernorm(oracle.conv(f64, w64, b64, nbr), g64, be64, 1e-6, silu=True)
    assert rel_err(out.float().cpu().numpy(), ref) <= 2e-2


def _offset(t: torch.Tensor) -> torch.Tensor:
    """A contiguous copy of t whose data pointer is one element past a 256-byte boundary."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    v = buf[1:].view(t.shape)
    v.copy_(t)
    assert v.data_ptr() % 16 != 0
    return v


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_conv_misaligned_buffers_take_generic_kernel(pkg, dev, dtype):
    """Buffers aligned only to their element size run the generic kernel (element stores), with
    the same bits as the tuned kernels on aligned buffers: both accumulate every row's taps in
    ascending order and each tap's channels in the same MFMA K groups."""
    coords, m = _small_map(pkg, dev)
    n = len(coords)
    f = torch.from_numpy(pkg.workloads.features(n, 64, 3)).to(dev).to(dtype)
    w = torch.from_numpy(pkg.workloads.conv_weight(64, 64, 4)).to(dev).to(dtype)
    b = torch.linspace(-1, 1, 64, device=dev).to(dtype)
    r = torch.from_numpy(pkg.workloads.features(n, 64, 5)).to(dev).to(dtype)
    print(f"  conv misaligned N={n} {dtype}", flush=True)
    want = pkg.sparse_conv3d(f, w, b, m.nbr, epilogue="residual", residual=r)
    fo, wo, bo, ro = _offset(f), _offset(w), _offset(b), _offset(r)
    out = _offset(torch.zeros_like(want))
    pkg.sparse_conv3d(fo, wo, bo, m.nbr, epilogue="residual", residual=ro, out=out)
    assert torch.equal(out, want)
    nbr = m.nbr.cpu().numpy()
    ref = oracle.conv(f.float().cpu().numpy(), w.float().cpu().numpy(), b.float().cpu().numpy(), nbr)
    assert rel_err(out.float().cpu().numpy(), ref + r.float().cpu().numpy()) <= TOL[dtype]


def test_conv_rejects_invalid(pkg, dev):
    coords = np.array([[0, 1, 1, 1]], np.int32)
    m = _map(pkg, dev, coords, 1, (3, 3, 3))
    f = torch.zeros((1, 32), device=dev, dtype=torch.float16)
    w = torch.zeros((48, 3, 3, 3, 32), device=dev, dtype=torch.float16)
    with pytest.raises(pkg.TscError):
        pkg.sparse_conv3d(f.cpu(), w.cpu(), None, m)  # no CPU path
    with pytest.raises(pkg.TscError):
        pkg.sparse_conv3d(f, w.float(), None, m)  # dtype mismatch
    with pytest.raises(pkg.TscError, match="residual"):
        pkg.sparse_conv3d(f, w, None, m, epilogue="residual")
    # odd byte addresses are not aligned to the 2-byte element: rejected by the C ABI
    lib = pkg._lib.context(dev.index)
    raw = torch.zeros(64, dtype=torch.uint8, device=dev)
    st = lib.lib.tsc_conv(lib.bind(), pkg._lib.TSC_F16, raw.data_ptr() + 1, w.data_ptr(), None,
                          m.nbr.data_ptr(), None, 1, 32, 48, raw.data_ptr() + 2)
    assert st == pkg._lib.TSC_ERR_INVALID
