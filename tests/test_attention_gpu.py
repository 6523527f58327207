"""Varlen attention on the GPU vs the fp64 oracle.

Tolerance: norm-wise relative error max|y - r| / max|r| <= 1e-4 for fp32 and <= 2e-2 for
bf16/fp16, the reference computed in fp64 from the same rounded inputs."""
import ctypes

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _inputs(rng, tq, tkv, h, d, dtype, q_scale=1.5):
    q = torch.from_numpy(rng.standard_normal((tq, h, d)) * q_scale).to(dtype)
    k = torch.from_numpy(rng.standard_normal((tkv, h, d))).to(dtype)
    v = torch.from_numpy(rng.standard_normal((tkv, h, d))).to(dtype)
    return q, k, v


def _check(got, q, k, v, cu_q, cu_kv, dtype, scale=None, rows=None):
    ref = oracle.attention(q.double().numpy(), k.double().numpy(), v.double().numpy(), cu_q, cu_kv,
                           scale, rows)
    g = got.float().cpu().numpy().astype(np.float64)
    if rows is not None:
        g, ref = g[rows], ref[rows]
    err = np.abs(g - ref).max() / max(np.abs(ref).max(), 1e-30)
    assert err <= TOL[dtype], err
    return err


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("d", [64, 128])
def test_ragged_self_attention(pkg, dev, dtype, d):
    rng = np.random.default_rng(d)
    cu = [0, 1, 33, 33, 200, 457, 713]  # a 1-row sequence, an empty one, non-multiples of 32/64/128
    h = 3
    q, k, v = _inputs(rng, cu[-1], cu[-1], h, d, dtype)
    print(f"  attention self {dtype} D={d} cu={cu}", flush=True)
    out = pkg.sparse_attention(q.to(dev), k.to(dev), v.to(dev), cu)
    torch.cuda.synchronize()
    _check(out, q, k, v, cu, cu, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_cross_attention_and_empty_keys(pkg, dev, dtype):
    rng = np.random.default_rng(7)
    cu_q, cu_kv = [0, 70, 70, 300, 301], [0, 0, 129, 129 + 1000, 129 + 1000 + 5]
    h, d = 2, 128
    q, k, v = _inputs(rng, cu_q[-1], cu_kv[-1], h, d, dtype)
    print(f"  attention cross {dtype}", flush=True)
    out = pkg.sparse_attention(q.to(dev), k.to(dev), v.to(dev), cu_q, cu_kv, scale=0.05)
    torch.cuda.synchronize()
    assert not out[:70].any()  # sequence 0 has no keys: zeros
    _check(out, q, k, v, cu_q, cu_kv, dtype, scale=0.05)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_running_max_rescales(pkg, dev, dtype):
    """Scores that grow along the keys (every block raises the max, by small and by large steps)
    and one late key far above the rest: the lazily raised running max must stay exact."""
    rng = np.random.default_rng(3)
    n, h, d = 1500, 2, 64
    base = rng.standard_normal((1, h, d))
    base /= np.linalg.norm(base, axis=-1, keepdims=True)
    q = np.repeat(base * 4.0, n, 0) + 0.1 * rng.standard_normal((n, h, d))
    ramp = np.linspace(0.0, 60.0, n)[:, None, None]  # the scaled max climbs ~43 log2 units
    k = base * ramp + 0.1 * rng.standard_normal((n, h, d))
    k[1400] = base[0] * 150.0  # one jump of far more than the 2^8 headroom
    v = rng.standard_normal((n, h, d))
    qt, kt, vt = (torch.from_numpy(x).to(dtype) for x in (q, k, v))
    print(f"  attention running max {dtype}", flush=True)
    out = pkg.sparse_attention(qt.to(dev), kt.to(dev), vt.to(dev), [0, n])
    torch.cuda.synchronize()
    _check(out, qt, kt, vt, [0, n], [0, n], dtype)


def test_dense_entry_and_grid_cover(pkg, dev):
    """scaledDotProductAttention over B equal sequences equals the varlen call; a max_seqlen_q
    below the real length still covers every query (the kernel's tile loop)."""
    rng = np.random.default_rng(4)
    b, s, h, d = 3, 300, 4, 128
    q, k, v = (x.to(dev) for x in _inputs(rng, b * s, b * s, h, d, torch.bfloat16))
    print("  attention dense entry / grid cover", flush=True)
    dense = pkg.scaled_dot_product_attention(q.view(b, s, h, d), k.view(b, s, h, d),
                                             v.view(b, s, h, d), h, batch_size=b)
    cu = torch.tensor([0, s, 2 * s, 3 * s], dtype=torch.int32, device=dev)
    var = pkg.sparse_attention(q, k, v, cu)
    assert torch.equal(dense.view(-1, h, d), var)
    out = torch.empty_like(q)
    ctx = pkg._lib.context(dev.index)
    pkg._lib.check(ctx.lib.tsc_attention(ctx.bind(), 2, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                         cu.data_ptr(), cu.data_ptr(), b, b * s, b * s, h, d,
                                         ctypes.c_float(0.0), 1, out.data_ptr()))
    torch.cuda.synchronize()
    assert torch.equal(out, var)


def test_key_permutation_invariance(pkg, dev):
    rng = np.random.default_rng(5)
    n, h, d = 777, 2, 128
    q, k, v = (x.to(dev) for x in _inputs(rng, n, n, h, d, torch.float32))
    perm = torch.from_numpy(rng.permutation(n)).to(dev)
    print("  attention key permutation", flush=True)
    a = pkg.sparse_attention(q, k, v, [0, n])
    b = pkg.sparse_attention(q, k[perm].contiguous(), v[perm].contiguous(), [0, n])
    torch.cuda.synchronize()
    assert (a - b).abs().max().item() <= 1e-5 * a.abs().max().item()


def test_slat_sized_bf16_sampled_rows(pkg, dev):
    """Two ragged sequences of SLat-flow size (12 heads x 128) in bf16, checked on sampled rows."""
    rng = np.random.default_rng(6)
    cu = [0, 9000, 9000 + 6143]
    h, d = 12, 128
    q, k, v = _inputs(rng, cu[-1], cu[-1], h, d, torch.bfloat16, q_scale=1.0)
    print(f"  attention SLat-sized bf16 cu={cu}", flush=True)
    out = pkg.sparse_attention(q.to(dev), k.to(dev), v.to(dev), cu)
    torch.cuda.synchronize()
    rows = np.sort(rng.choice(cu[-1], 300, replace=False))
    _check(out, q, k, v, cu, cu, torch.bfloat16, rows=rows)


def test_rows_outside_every_sequence_are_zero(pkg, dev):
    """cu_seqlens need not cover every row: rows before cu[0] and after cu[B] come out zero, as the
    reference's zero-initialised output (attention.ts:49) leaves them."""
    rng = np.random.default_rng(8)
    cu = [5, 40, 90]
    q, k, v = _inputs(rng, 100, 100, 2, 64, torch.bfloat16)
    print("  attention partial coverage", flush=True)
    out = pkg.sparse_attention(q.to(dev), k.to(dev), v.to(dev), cu, cu)
    torch.cuda.synchronize()
    assert not out[:5].any() and not out[90:].any()
    _check(out, q, k, v, cu, cu, torch.bfloat16)


def test_attention_rejects_bad_arguments(pkg, dev):
    x = torch.zeros(10, 2, 64, device=dev, dtype=torch.bfloat16)
    with pytest.raises(pkg.TscError):
        pkg.sparse_attention(x, x, x, [0, 5, 4, 10])      # decreasing offsets
    with pytest.raises(pkg.TscError):
        pkg.sparse_attention(x, x, x, [0, 11])            # past the end
    y = torch.zeros(10, 2, 96, device=dev, dtype=torch.bfloat16)
    with pytest.raises(pkg.TscError):
        pkg.sparse_attention(y, y, y, [0, 10])            # head_dim 96
    with pytest.raises(pkg.TscError):
        pkg.sparse_attention(x, x.float(), x, [0, 10])    # mixed dtypes


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_device_cu_seqlens_make_no_host_read(pkg, dev, dtype):
    """Device cu_seqlens go to the kernel as given: under torch's sync debug mode "error" (any
    device-to-host read raises) the call succeeds, and the result equals the call with host
    offsets bit for bit.  The sequences are unbalanced (one 6x the mean), so the default grid size
    (twice the mean length) leaves the longest one to the kernel's tile loop; empty and 1-row
    sequences included.  Rows outside every sequence come out zero."""
    rng = np.random.default_rng(21)
    cu = [3, 3, 4, 130, 3130, 3200, 3456]
    tq, h, d = 3470, 4, 128
    q, k, v = _inputs(rng, tq, tq, h, d, dtype)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    cu_dev = torch.tensor(cu, dtype=torch.int32, device=dev)
    print(f"  attention device cu_seqlens {dtype}", flush=True)
    want = pkg.sparse_attention(qd, kd, vd, cu)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        got = pkg.sparse_attention(qd, kd, vd, cu_dev)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert not got[:3].any() and not got[3456:].any()
    _check(got, q, k, v, cu, cu, dtype)
