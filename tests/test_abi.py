"""C-ABI library checks that need no GPU: it loads, exports every declared symbol, and rejects
bad arguments with a status code and a message instead of touching device memory."""
import ctypes

import pytest


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.load_library()
    declared = pkg.header_symbols()
    assert len(declared) >= 18
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    assert lib.tsc_version() == 5


def test_null_context_and_bad_arguments_fail_cleanly(pkg):
    lib = pkg.load_library()
    P = ctypes.c_void_p
    st = lib.tsc_conv(None, 0, P(16), P(16), None, P(16), None, 10, 64, 64, P(16))
    assert st == 1 and b"null context" in lib.tsc_last_error()
    st = lib.tsc_sync(None)
    assert st == 1
    assert lib.tsc_map_key_bytes(1, 512, 512, 512) == 4
    assert lib.tsc_map_key_bytes(2, 1024, 1024, 1023) == 4
    assert lib.tsc_map_key_bytes(2, 1024, 1024, 1024) == 8  # 2^31 cells
    assert lib.tsc_map_key_bytes(0, 4, 4, 4) == 0
    out = P()
    st = lib.tsc_ctx_create(-1, None, ctypes.byref(out))
    assert st != 0 and lib.tsc_last_error()
    assert lib.tsc_ctx_destroy(None) == 0


def test_gather_plan_bytes(pkg):
    """Plan size = five 256-byte aligned arrays over T = ceil(N/64) tiles: rows (T*64 int32),
    counts (T int32), tap masks (T*4 uint32), distinct-row lists (T*256 int32), slot tables
    (T*1792 bytes); -1 for N out of range."""
    lib = pkg.load_library()
    lib.tsc_map_gather_plan_bytes.restype = ctypes.c_int64
    lib.tsc_map_gather_plan_bytes.argtypes = [ctypes.c_int64]
    al = lambda v: (v + 255) // 256 * 256
    for n in (0, 1, 64, 65, 1514003):
        t = (n + 63) // 64
        want = al(t * 256) + al(t * 4) + al(t * 16) + al(t * 1024) + al(t * 1792)
        assert lib.tsc_map_gather_plan_bytes(n) == want
    assert lib.tsc_map_gather_plan_bytes(-1) == -1
    assert lib.tsc_map_gather_plan_bytes(2 ** 31) == -1
    P = ctypes.c_void_p
    st = lib.tsc_map_gather_plan(None, P(16), P(16), 10, 1, 8, 8, 8, P(256))
    assert st == 1 and b"null context" in lib.tsc_last_error()


def test_ops_refuse_cpu_tensors(pkg):
    import torch

    x = torch.zeros((4, 32))
    with pytest.raises(pkg.TscError, match="not on a GPU"):
        pkg.layer_norm(x)
    with pytest.raises(pkg.TscError, match="not on a GPU"):
        pkg.build_neighbor_map(torch.zeros((1, 4), dtype=torch.int32), (2, 2, 2), 1)


def test_sparse_tensor_host_logic(pkg):
    import torch

    coords = torch.tensor([[0, 1, 2, 3], [0, 4, 0, 1], [1, 0, 5, 0], [1, 2, 2, 2], [1, 1, 1, 1]],
                          dtype=torch.int32)
    x = pkg.SparseTensor(torch.zeros((5, 8)), coords)
    assert x.spatial_shape == [5, 6, 4]
    assert x.layout == [(0, 2), (2, 5)] and x.batch_size == 2 and x.shape == [2, 8]
    y = x.replace(torch.ones((5, 16)))
    x.register_spatial_cache("k", 1)
    assert y.get_spatial_cache("k") == 1 and y.coords is x.coords
    assert pkg.neighbor_cache_key((3, 3, 3), (1, 2, 3)) == "conv_neighbors_3x3x3_dil3x2x1"
    s = pkg.SparseTensor.from_feats_and_coords([torch.zeros((2, 4)), torch.zeros((1, 4))],
                                               [coords[:2], coords[:1]])
    assert s.coords[:, 0].tolist() == [0, 0, 1]
    with pytest.raises(pkg.TscError):
        pkg.SparseConv3d(torch.zeros((32, 5, 5, 5, 32)), None, (5, 5, 5))


def test_workloads_are_seeded_and_sized(pkg):
    wl = pkg.workloads
    a = wl.make_coords("conv64_f32")
    b = wl.make_coords("conv64_f32")
    assert (a == b).all()
    assert 18000 < len(a) < 30000
    c = wl.make_coords("resblock64_bf16")
    assert int(c[:, 0].max()) == 1 and 25000 < (c[:, 0] == 0).sum() < 36000
    w = wl.conv_weight(64, 32, 0)
    assert w.shape == (64, 3, 3, 3, 32)
    assert abs(w.std() - 1 / (27 * 32) ** 0.5) < 0.01
