"""LayerNorm / SiLU / add and the ResBlock chain on the GPU vs fp64 references."""
import numpy as np
import pytest
import torch

import oracle
from tests import _golden

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def _r(a, dtype, dev):
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(dtype)
    return t, t.float().cpu().numpy().astype(np.float64)


def test_layernorm_golden(pkg, dev):
    md, a = _golden.load("layernorm_silu")
    x = torch.from_numpy(a[("in", "x")]).to(dev)
    g = torch.from_numpy(a[("in", "gamma")]).to(dev)
    b = torch.from_numpy(a[("in", "beta")]).to(dev)
    ln = pkg.layer_norm(x, g, b, 1e-6).cpu().numpy()
    np.testing.assert_allclose(ln, a[("exp", "ln")], rtol=1e-5, atol=1e-5)
    lns = pkg.layer_norm(x, g, b, 1e-6, silu=True).cpu().numpy()
    np.testing.assert_allclose(lns, a[("exp", "ln_silu")], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n,c", [(1000, 1024), (333, 96), (50, 4100), (7, 40), (64, 5000)])
@pytest.mark.parametrize("affine", [False, True])
def test_layernorm_silu_shapes(pkg, dev, dtype, n, c, affine):
    rng = np.random.default_rng(n + c)
    x, x64 = _r(rng.standard_normal((n, c)) * 2 + 0.3, dtype, dev)
    g = b = g64 = b64 = None
    if affine:
        g, g64 = _r(rng.uniform(0.5, 1.5, c), dtype, dev)
        b, b64 = _r(rng.standard_normal(c) * 0.1, dtype, dev)
    for silu in (False, True):
        y = pkg.layer_norm(x, g, b, 1e-6, silu=silu).float().cpu().numpy()
        ref = oracle.layernorm(x64, g64, b64, 1e-6, silu=silu)
        assert rel_err(y, ref) <= TOL[dtype] * 4, (silu, rel_err(y, ref))
    # in place (the reference's layerNorm mutates its input, layer_norm.ts:63)
    x2 = x.clone()
    pkg.layer_norm(x2, g, b, 1e-6, out=x2)
    assert rel_err(x2.float().cpu().numpy(), oracle.layernorm(x64, g64, b64, 1e-6)) <= TOL[dtype] * 4


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_layernorm_row_groups(pkg, dev, dtype):
    """Rows of 1..33 16-byte vectors around every lane-group size of the grouped pass (several
    rows per wave for <= 32 vectors, one row per wave above), a row count that leaves the last
    wave partly empty, affine and plain, against the fp64 layer norm; in-place as well."""
    per = 4 if dtype == torch.float32 else 8  # elements per 16-byte vector
    rng = np.random.default_rng(5)
    for nvec in (1, 2, 3, 5, 8, 16, 17, 32, 33):
        c = nvec * per
        n = 3 * (64 // min(64, 1 << (nvec - 1).bit_length())) * 4 + 5
        x, x64 = _r(rng.standard_normal((n, c)) * 1.5 - 0.2, dtype, dev)
        g, g64 = _r(rng.uniform(0.5, 1.5, c), dtype, dev)
        b, b64 = _r(rng.standard_normal(c) * 0.1, dtype, dev)
        for affine in (False, True):
            gg, bb = (g, b) if affine else (None, None)
            gr, br = (g64, b64) if affine else (None, None)
            y = pkg.layer_norm(x, gg, bb, 1e-6, silu=True).float().cpu().numpy()
            err = rel_err(y, oracle.layernorm(x64, gr, br, 1e-6, silu=True))
            assert err <= TOL[dtype] * 4, (nvec, affine, err)
        x2 = x.clone()
        pkg.layer_norm(x2, None, None, 1e-6, out=x2)
        assert rel_err(x2.float().cpu().numpy(), oracle.layernorm(x64, None, None, 1e-6)) <= TOL[dtype] * 4


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_silu_add(pkg, dev, dtype):
    rng = np.random.default_rng(1)
    x, x64 = _r(rng.standard_normal(100003) * 4, dtype, dev)
    y, y64 = _r(rng.standard_normal(100003), dtype, dev)
    s = pkg.silu(x).float().cpu().numpy()
    assert rel_err(s, oracle.silu(x64)) <= TOL[dtype]
    a = pkg.add(x, y).float().cpu().numpy()
    assert rel_err(a, x64 + y64) <= TOL[dtype]
    pkg.add(x, y, out=x)
    assert rel_err(x.float().cpu().numpy(), x64 + y64) <= TOL[dtype]


@pytest.mark.parametrize("c,nvox", [(256, 1500), (1024, 500)])
def test_resblock_vs_oracle(pkg, dev, c, nvox):
    coords = pkg.workloads.make_coords("resblock64_bf16")
    coords = coords[coords[:, 0] == 1][:nvox].copy()
    coords[:, 0] = 0
    n = len(coords)
    print(f"  resblock C={c} N={n}", flush=True)
    m = pkg.build_neighbor_map(torch.from_numpy(coords).to(dev), (64, 64, 64), 1)
    nbr = m.nbr.cpu().numpy()
    dt = torch.bfloat16
    x, x64 = _r(pkg.workloads.features(n, c, 1), dt, dev)
    w1, w164 = _r(pkg.workloads.conv_weight(c, c, 2), dt, dev)
    w2, w264 = _r(pkg.workloads.conv_weight(c, c, 3), dt, dev)
    b1, b164 = _r(np.linspace(-0.1, 0.1, c), dt, dev)
    b2, b264 = _r(np.linspace(0.1, -0.1, c), dt, dev)
    out = pkg.sparse_resblock(x, m, w1, b1, w2, b2, eps=1e-6).float().cpu().numpy()
    ref = oracle.resblock(x64, nbr, w164, b164, w264, b264, eps=1e-6)
    err = rel_err(out, ref)
    assert err <= 2e-2, err


def test_resblock_module_chain(pkg, dev):
    """Four SparseResBlock3d through the operator API share one cached neighbor map."""
    coords = pkg.workloads.make_coords("resblock64_bf16")[:3000]
    coords = coords[coords[:, 0] == 0]
    n = len(coords)
    dt = torch.bfloat16
    c = 128
    x = pkg.SparseTensor(torch.from_numpy(pkg.workloads.features(n, c, 0)).to(dev).to(dt),
                         torch.from_numpy(coords).to(dev))
    blocks, ws = [], []
    for i in range(4):
        w1 = torch.from_numpy(pkg.workloads.conv_weight(c, c, 10 + i)).to(dev).to(dt)
        w2 = torch.from_numpy(pkg.workloads.conv_weight(c, c, 20 + i)).to(dev).to(dt)
        blocks.append(pkg.SparseResBlock3d(w1, None, w2, None))
        ws.append((w1.float().cpu().numpy(), w2.float().cpu().numpy()))
    h = x
    for blk in blocks:
        h = blk(h)
    key = pkg.neighbor_cache_key((3, 3, 3), (1, 1, 1))
    assert h.get_spatial_cache(key) is x.get_spatial_cache(key)
    nbr = x.get_spatial_cache(key).nbr.cpu().numpy()
    ref = x.feats.float().cpu().numpy().astype(np.float64)
    for w1, w2 in ws:
        ref = oracle.resblock(ref, nbr, w1, None, w2, None, eps=1e-6)
    assert rel_err(h.feats.float().cpu().numpy(), ref) <= 2e-2
