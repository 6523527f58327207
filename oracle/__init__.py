"""CPU oracle for the submanifold sparse conv3d path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker or the timed CPU baseline; the product library never calls it.

Contents
  oracle.c          plain-C restatement (map build two ways, fp64 conv, LayerNorm, SiLU);
                    built into liboracle.so by build() with gcc -O2 -fopenmp
  torch_path.py     PyTorch-CPU restatement of the reference's Python path
                    (hashmap_fallback: torch.sort + torch.searchsorted; conv_none: per-tap
                    index_select + mm), used as the timed CPU baseline
  brute.py          pure-Python brute force for tiny inputs

  subdivide()        numpy restatement of the decoder's upsample step (each voxel -> its 2x2x2
                    children, optional keep mask)
  linear(), convnext_block()
                    fp64 numpy restatements of nn.Linear per voxel and the sparse ConvNeXt block
  attention()       fp64 numpy restatement of varlen scaled-dot-product attention
  st_reader.py      numpy restatement of the reference's safetensors reader and its float
                    conversions (pinned in its own docstring and tests/test_safetensors.py)

Pinning (see tests/test_oracle.py): the map builds are checked against each other and against
brute force, sorted keys against numpy.unique, the conv against a dense torch F.conv3d closed
form in fp64, LayerNorm/SiLU against torch.nn.functional in fp64, and all of them against the
fixtures in tests/golden/ that were generated without this package.  subdivide() is pinned by
what its definition fixes: every output row's parent is (b, x//2, y//2, z//2) with child index
from the low bits, the children of a full subdivision are exactly the 8N cells of the doubled
grid that lie inside parent cells, a dense 2^3 block maps onto a dense 4^3 block, and one
subdivision equals the union of eight single-child keep masks.  The reference holds no tests or
fixtures for it (its TS port does not generate children: sparse_unet_vae_decoder.ts:155-175);
the child order follows torch.nonzero over a 2x2x2 cube (dx slowest, dz fastest), the order of
trellis2's SparseSubdivide, which is not in this container: that convention is parity unpinned.
attention() is pinned against torch.nn.functional.scaled_dot_product_attention in fp64 per
sequence, and by closed forms: constant V rows give that row, zero queries give the mean of V,
one key gives its V row, a key permutation leaves the output unchanged, and a sequence without
keys gives zeros (attention.ts:57).
linear() is pinned against torch.nn.functional.linear in fp64; convnext_block() is the
composition of the pinned conv, layernorm and linear (the block's step order is the TS port's,
sparse_unet_vae_decoder.ts:48-78).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
STATUS_DUPLICATE = 1
STATUS_OUT_OF_RANGE = 2

_lib = None


def build(force: bool = True) -> Path:
    """Compile oracle.c into liboracle.so (gcc, OpenMP)."""
    src = HERE / "oracle.c"
    if not force and LIB.exists() and LIB.stat().st_mtime >= src.stat().st_mtime:
        return LIB
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-fopenmp", "-shared", "-fPIC", "-o", str(tmp), str(src), "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB.exists():
        build()
    lib = ctypes.CDLL(str(LIB))
    P = ctypes.c_void_p
    i64, i32, u32, f64 = ctypes.c_int64, ctypes.c_int32, ctypes.c_uint32, ctypes.c_double
    lib.oracle_pack_key.restype = i64
    lib.oracle_pack_key.argtypes = [i32] * 7
    lib.oracle_map_sorted.restype = u32
    lib.oracle_map_sorted.argtypes = [P, i64, i32, i32, i32, i32, P, P, P, P]
    lib.oracle_map_grid.restype = u32
    lib.oracle_map_grid.argtypes = [P, i64, i32, i32, i32, i32, P, P]
    lib.oracle_conv.restype = None
    lib.oracle_conv.argtypes = [P, P, P, P, i64, i32, i32, P]
    lib.oracle_layernorm.restype = None
    lib.oracle_layernorm.argtypes = [P, i64, i32, P, P, f64, i32, P]
    lib.oracle_silu.restype = None
    lib.oracle_silu.argtypes = [P, i64, P]
    _lib = lib
    return lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _coords(coords):
    c = np.ascontiguousarray(coords, dtype=np.int32)
    assert c.ndim == 2 and c.shape[1] == 4
    return c


def pack_keys(coords, shape) -> np.ndarray:
    """key = ((b*X+x)*Y+y)*Z+z as int64 (the packing both sides use)."""
    c = _coords(coords).astype(np.int64)
    X, Y, Z = shape
    return ((c[:, 0] * X + c[:, 1]) * Y + c[:, 2]) * Z + c[:, 3]


def map_sorted(coords, batch, shape, dilation=(1, 1, 1)):
    """hashmap_fallback restatement.  Returns (status, sorted_keys int64, perm int32, nbr (N,27))."""
    lib = _load()
    c = _coords(coords)
    n = c.shape[0]
    keys = np.empty(n, np.int64)
    perm = np.empty(n, np.int32)
    nbr = np.empty((n, 27), np.int32)
    dil = np.asarray(dilation, np.int32)
    st = lib.oracle_map_sorted(_ptr(c), n, batch, *shape, _ptr(dil), _ptr(keys), _ptr(perm), _ptr(nbr))
    return int(st), keys, perm, nbr


def map_grid(coords, batch, shape, dilation=(1, 1, 1)):
    """Dense-grid (WGSL pass0/pass1) restatement.  Returns (status, nbr (N,27))."""
    lib = _load()
    c = _coords(coords)
    n = c.shape[0]
    nbr = np.empty((n, 27), np.int32)
    dil = np.asarray(dilation, np.int32)
    st = lib.oracle_map_grid(_ptr(c), n, batch, *shape, _ptr(dil), _ptr(nbr))
    return int(st), nbr


def conv(feats, weight, bias, nbr) -> np.ndarray:
    """fp64 gather-GEMM-bias.  weight (Co,3,3,3,Ci) or (Co,27,Ci); bias (Co,) or None."""
    lib = _load()
    f = np.ascontiguousarray(feats, dtype=np.float64)
    w = np.ascontiguousarray(weight, dtype=np.float64)
    co = w.shape[0]
    ci = w.shape[-1]
    w = w.reshape(co, 27, ci)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float64)
    nb = np.ascontiguousarray(nbr, dtype=np.int32)
    n = nb.shape[0]
    assert f.shape == (f.shape[0], ci) and nb.shape == (n, 27)
    assert n == 0 or (nb.max() < f.shape[0])
    out = np.empty((n, co), np.float64)
    lib.oracle_conv(_ptr(f), _ptr(w), _ptr(b), _ptr(nb), n, ci, co, _ptr(out))
    return out


def layernorm(x, gamma=None, beta=None, eps=1e-6, silu=False) -> np.ndarray:
    lib = _load()
    a = np.ascontiguousarray(x, dtype=np.float64)
    n, c = a.shape
    g = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.float64)
    b = None if beta is None else np.ascontiguousarray(beta, dtype=np.float64)
    y = np.empty_like(a)
    lib.oracle_layernorm(_ptr(a), n, c, _ptr(g), _ptr(b), float(eps), int(bool(silu)), _ptr(y))
    return y


def silu(x) -> np.ndarray:
    lib = _load()
    a = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty_like(a)
    lib.oracle_silu(_ptr(a), a.size, _ptr(y))
    return y


def resblock(x, nbr, w1, b1, w2, b2, gamma=None, beta=None, eps=1e-6) -> np.ndarray:
    """x + conv2(silu(LN(conv1(x)+b1)))+b2 in fp64 (config-5 block, stated literally)."""
    h = conv(x, w1, b1, nbr)
    h = layernorm(h, gamma, beta, eps, silu=True)
    return np.asarray(x, np.float64) + conv(h, w2, b2, nbr)


def subdivide(coords, feats=None, keep=None):
    """Children at twice the resolution (the decoder's upsample step, caller
    src/models/sparse_unet_vae_decoder.ts:155-175): parent [b,x,y,z] -> [b, 2x+dx, 2y+dy, 2z+dz]
    with c = dx*4 + dy*2 + dz, rows parent-major and c increasing, features copied from the
    parent; keep (uint8 per parent, bit c) selects children.  Returns (coords, feats or None)."""
    coords = np.asarray(coords, np.int64).reshape(-1, 4)
    n = coords.shape[0]
    c = np.arange(8)
    off = np.stack([np.zeros(8, np.int64), c >> 2, (c >> 1) & 1, c & 1], axis=1)
    base = coords * np.array([1, 2, 2, 2], np.int64)
    kids = (base[:, None, :] + off[None, :, :]).reshape(-1, 4)
    sel = np.ones(8 * n, bool) if keep is None else \
        ((np.asarray(keep, np.uint8)[:, None] >> c[None, :]) & 1).astype(bool).reshape(-1)
    out_f = None
    if feats is not None:
        f = np.asarray(feats)
        out_f = np.repeat(f, 8, axis=0)[sel]
    return kids[sel].astype(np.int32), out_f


def linear(x, weight, bias=None, residual=None) -> np.ndarray:
    """x (N,Cin) @ weight(Cout,Cin)^T + bias (+ residual), fp64 (nn.Linear per voxel,
    src/sparse/ops/linear.ts:9-29)."""
    y = np.asarray(x, np.float64) @ np.asarray(weight, np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    if residual is not None:
        y = y + np.asarray(residual, np.float64)
    return y


def convnext_block(feats, nbr, conv_w, conv_b, w0, b0, w2, b2, eps=1e-6, rows=None, store=None):
    """Sparse ConvNeXt block (src/models/sparse_unet_vae_decoder.ts:48-78), fp64:
    h = conv(x); h = LN(h); h = h W0^T + b0; h = silu(LN(h)); out = x + h W2^T + b2.
    rows: optional subset of output rows (the conv reads neighbors from all of feats).
    store: optional rounding (fp64 array -> fp64 array of representable values) applied where the
    TS block stores a step's tensor in its storage type: after the conv, the first LayerNorm, the
    first linear, the LayerNorm + SiLU and the output."""
    st = (lambda a: a) if store is None else store
    f = np.asarray(feats, np.float64)
    nb = np.asarray(nbr) if rows is None else np.asarray(nbr)[rows]
    h = st(conv(f, conv_w, conv_b, nb))
    h = st(layernorm(h, None, None, eps))
    h = st(linear(h, w0, b0))
    h = st(layernorm(h, None, None, eps, silu=True))
    skip = f if rows is None else f[rows]
    return st(linear(h, w2, b2, skip))


def attention(q, k, v, cu_q, cu_kv, scale=None, rows=None) -> np.ndarray:
    """Varlen scaled-dot-product attention in fp64 (src/sparse/ops/attention.ts:24-79: per
    sequence b, softmax(Q_b K_b^T * scale) V_b per head; a sequence without keys stays zero,
    :57).  q (total_q, H, D), k / v (total_kv, H, D); `rows` restricts the output to those query
    rows (the others are zero)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    d = q.shape[-1]
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    out = np.zeros(q.shape, np.float64)
    want = None if rows is None else np.zeros(q.shape[0], bool)
    if want is not None:
        want[np.asarray(rows)] = True
    for b in range(len(cu_q) - 1):
        q0, q1, k0, k1 = int(cu_q[b]), int(cu_q[b + 1]), int(cu_kv[b]), int(cu_kv[b + 1])
        if q1 <= q0 or k1 <= k0:
            continue
        idx = np.arange(q0, q1) if want is None else np.nonzero(want[q0:q1])[0] + q0
        if idx.size == 0:
            continue
        s = np.einsum("nhd,mhd->hnm", q[idx], k[k0:k1]) * scale
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[idx] = np.einsum("hnm,mhd->nhd", p, v[k0:k1])
    return out
