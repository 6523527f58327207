"""tsc_conv_fused_noalloc (the conv entry point that allocates nothing) against tsc_conv_fused,
through the C ABI: the same kernels run with the tile schedule in the static per-device scratch
instead of the context's workspace, so the outputs must be equal bit for bit.  Each case makes two
calls in a row, the second on a smaller input (the scratch keeps the first call's contents), and
compares both with tsc_conv_fused on the same inputs.
"""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
_EPI = {"bias": 0, "residual": 1, "ln_silu": 2}


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _run(pkg, entry, f, w, b, nbr, order, epi, res, gamma, out):
    ctx = pkg._lib.context(f.device.index)
    fn = getattr(ctx.lib, entry)
    n, ci = f.shape
    co = w.shape[0]
    st = fn(ctx.bind(), _CODES[f.dtype], _p(f), _p(w), _p(b), _p(nbr), _p(order), n, ci, co,
            _EPI[epi], _p(res), _p(gamma), None, ctypes.c_float(1e-6), _p(out))
    if st:
        raise pkg.TscError(st, ctx.lib.tsc_last_error().decode())
    return out


def _inputs(pkg, dev, coords, ci, co, dtype, seed):
    batch = int(coords[:, 0].max()) + 1
    m = pkg.build_neighbor_map(torch.from_numpy(coords).to(dev), (64, 64, 64), batch)
    n = len(coords)
    f = torch.from_numpy(pkg.workloads.features(n, ci, seed)).to(dev).to(dtype)
    w = torch.from_numpy(pkg.workloads.conv_weight(co, ci, seed + 1)).to(dev).to(dtype)
    b = torch.linspace(-0.3, 0.3, co, device=dev).to(dtype)
    r = torch.from_numpy(pkg.workloads.features(n, co, seed + 2)).to(dev).to(dtype)
    g = torch.linspace(0.5, 1.5, co, device=dev).to(dtype)
    return m, f, w, b, r, g


@pytest.mark.parametrize("dtype,ci,co,epi", [
    (torch.bfloat16, 256, 256, "bias"),       # 256x256 tiles with the longest-first schedule
    (torch.bfloat16, 512, 512, "residual"),
    (torch.bfloat16, 1024, 1024, "ln_silu"),
    (torch.float16, 32, 64, "bias"),          # narrow kernel (no schedule)
    (torch.float32, 64, 64, "residual"),
    (torch.bfloat16, 13, 48, "ln_silu"),      # generic kernel
])
def test_noalloc_matches_conv_fused(pkg, dev, dtype, ci, co, epi):
    full = pkg.workloads.make_coords("resblock64_bf16")
    small = full[full[:, 0] == 1][:7000].copy()
    small[:, 0] = 0
    for coords, seed in ((full, 1), (small, 5)):  # second call: a smaller input
        m, f, w, b, r, g = _inputs(pkg, dev, coords, ci, co, dtype, seed)
        order = m.conv_order()
        print(f"  noalloc {dtype} {ci}->{co} {epi} N={len(coords)}", flush=True)
        res = r if epi == "residual" else None
        gamma = g if epi == "ln_silu" else None
        want = _run(pkg, "tsc_conv_fused", f, w, b, m.nbr, order, epi, res, gamma,
                    torch.empty((len(coords), co), dtype=dtype, device=dev))
        got = _run(pkg, "tsc_conv_fused_noalloc", f, w, b, m.nbr, order, epi, res, gamma,
                   torch.full((len(coords), co), float("nan"), dtype=dtype, device=dev))
        assert torch.equal(got, want)
        # the same call again (scratch holding this shape's schedule) and in place on the residual
        if epi == "residual":
            r2 = r.clone()
            _run(pkg, "tsc_conv_fused_noalloc", f, w, b, m.nbr, order, epi, r2, None, r2)
            assert torch.equal(r2, want)


def test_noalloc_first_call_on_fresh_context_under_graph_capture(pkg, dev):
    """'Allocates nothing', checked by behaviour: the first call on a new context, whose
    workspaces are all empty, is captured into a CUDA (HIP) graph.  During a capture any
    hipMalloc, hipFree or stream synchronization (what growing a workspace does) fails the call and
    the capture, so a path that reached for the context's workspace would not pass.  The graph is
    replayed three times with eager calls on other inputs in between; every replay must equal
    tsc_conv_fused bit for bit.  The captured kernels write no memset node (the schedule is built
    by kernels).  bf16 256->256 uses the 256-row tiles and their longest-first schedule."""
    coords = pkg.workloads.make_coords("resblock64_bf16")
    m, f, w, b, r, g = _inputs(pkg, dev, coords, 256, 256, torch.bfloat16, 3)
    order = m.conv_order()
    n = len(coords)
    want = _run(pkg, "tsc_conv_fused", f, w, b, m.nbr, order, "bias", None, None,
                torch.empty((n, 256), dtype=torch.bfloat16, device=dev))
    # The device's scratch address is looked up once per device; do it outside the capture, on
    # the shared context (not the fresh one).
    _run(pkg, "tsc_conv_fused_noalloc", f, w, b, m.nbr, order, "bias", None, None,
         torch.empty((n, 256), dtype=torch.bfloat16, device=dev))
    torch.cuda.synchronize()
    side = torch.cuda.Stream(dev)
    with torch.cuda.stream(side):
        fresh = pkg._lib.Context(dev.index)  # bound to the capture stream from the start
    out = torch.full((n, 256), float("nan"), dtype=torch.bfloat16, device=dev)
    graph = torch.cuda.CUDAGraph()
    print(f"  noalloc under graph capture N={n}", flush=True)
    with torch.cuda.graph(graph, stream=side):
        st = fresh.lib.tsc_conv_fused_noalloc(
            fresh.bind(), _CODES[torch.bfloat16], _p(f), _p(w), _p(b), _p(m.nbr), _p(order), n,
            256, 256, _EPI["bias"], None, None, None, ctypes.c_float(1e-6), _p(out))
    assert st == 0, fresh.lib.tsc_last_error().decode()
    try:
        small = coords[coords[:, 0] == 0][:5000].copy()
        for i in range(3):
            out.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, want), f"replay {i}"
            # eager work in between: another shape through the shared context
            m2, f2, w2, b2, _, _ = _inputs(pkg, dev, small, 256, 256, torch.bfloat16, 10 + i)
            _run(pkg, "tsc_conv_fused_noalloc", f2, w2, b2, m2.nbr, m2.conv_order(), "bias", None,
                 None, torch.empty((len(small), 256), dtype=torch.bfloat16, device=dev))
            torch.cuda.synchronize()
    finally:
        del graph
        fresh.lib.tsc_ctx_destroy(fresh.handle)


def test_noalloc_rejects_rows_beyond_scratch(pkg, dev):
    """N above 65536 tiles of 256 rows is refused before any launch (small dummy buffers)."""
    ctx = pkg._lib.context(dev.index)
    buf = torch.zeros(64, dtype=torch.int32, device=dev)
    limit = 65536 * 256
    st = ctx.lib.tsc_conv_fused_noalloc(ctx.bind(), 2, _p(buf), _p(buf), None, _p(buf), None,
                                        limit + 1, 256, 256, 0, None, None, None,
                                        ctypes.c_float(1e-6), _p(buf))
    assert st == pkg._lib.TSC_ERR_INVALID
    assert b"scratch" in ctx.lib.tsc_last_error()
    # N = 0 is a no-op
    st = ctx.lib.tsc_conv_fused_noalloc(ctx.bind(), 2, None, None, None, None, None, 0, 256, 256,
                                        0, None, None, None, ctypes.c_float(1e-6), None)
    assert st == 0
