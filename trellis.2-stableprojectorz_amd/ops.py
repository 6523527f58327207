"""Functional ops over torch device tensors, each one C-ABI call into libtrellis_sparse.so.

torch is used for device memory and the current stream only; all compute is in the HIP library.
Inputs must be contiguous tensors on a HIP device (there is no CPU path).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import TscError, check

_DTYPES = {torch.float32: _lib.TSC_F32, torch.float16: _lib.TSC_F16, torch.bfloat16: _lib.TSC_BF16}


def _code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TscError(_lib.TSC_ERR_INVALID, f"unsupported dtype {t.dtype}") from None


def _dev(*ts) -> int:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise TscError(_lib.TSC_ERR_INVALID, "tensor is not on a GPU; this path has no CPU fallback")
        if not t.is_contiguous():
            raise TscError(_lib.TSC_ERR_INVALID, "tensor must be contiguous")
        if dev is None:
            dev = t.device.index
        elif t.device.index != dev:
            raise TscError(_lib.TSC_ERR_INVALID, "tensors live on different devices")
    return dev


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


@dataclass
class NeighborMap:
    """Result of the map build: the (N,27) table plus the sorted keys and their rows."""

    nbr: torch.Tensor          # (N,27) int32, original row of each neighbor or -1
    keys: torch.Tensor         # (N,) int32/int64 sorted unique packed keys
    perm: torch.Tensor         # (N,) int32, perm[i] = row of keys[i]  (spatially sorted order)
    spatial_shape: tuple
    batch_size: int
    dilation: tuple
    coords: torch.Tensor | None = None  # the (N,4) input, kept for the gather plan
    status: torch.Tensor | None = None  # device int32 (1): TSC_MAP_* bits, 0 = valid
    _conv_order: torch.Tensor | None = None
    _gather_plan: torch.Tensor | None = None

    def check(self) -> None:
        """Reads the build's status word (one 4-byte device-to-host copy, which waits for the
        build) and raises on duplicate or out-of-range coordinates, whose outputs are undefined."""
        if self.status is not None:
            _raise_status(int(self.status.item()), self.batch_size, self.spatial_shape)

    def conv_order(self) -> torch.Tensor:
        """Row order the convs use (tsc_map_conv_order), computed on first use and cached."""
        if self._conv_order is None:
            self._conv_order = map_conv_order(self.nbr, self.perm)
        return self._conv_order

    def gather_plan(self) -> torch.Tensor:
        """Gather plan of the narrow convs (tsc_map_gather_plan), computed on first use and cached."""
        if self._gather_plan is None:
            if self.coords is None:
                raise TscError(_lib.TSC_ERR_INVALID, "gather plan needs the map's coords")
            self._gather_plan = map_gather_plan(self.coords, self.nbr, self.batch_size,
                                                self.spatial_shape)
        return self._gather_plan


def map_conv_order(nbr: torch.Tensor, perm: torch.Tensor | None = None) -> torch.Tensor:
    """Rows grouped by their set of present neighbors inside windows of the sorted order."""
    if nbr.dtype != torch.int32 or nbr.dim() != 2 or nbr.shape[1] != 27:
        raise TscError(_lib.TSC_ERR_INVALID, "nbr must be int32 (N,27)")
    n = nbr.shape[0]
    if perm is not None and (perm.dtype != torch.int32 or perm.numel() != n):
        raise TscError(_lib.TSC_ERR_INVALID, "perm must be int32 (N,)")
    dev = _dev(nbr, perm)
    ctx = _lib.context(dev)
    order = torch.empty((n,), dtype=torch.int32, device=nbr.device)
    check(ctx.lib.tsc_map_conv_order(ctx.bind(), _p(nbr), _p(perm), n, _p(order)))
    return order


def map_gather_plan(coords: torch.Tensor, nbr: torch.Tensor, batch_size: int,
                    spatial_shape) -> torch.Tensor:
    """Gather plan (uint8 device buffer) of the narrow convs over this coordinate set and map."""
    if coords.dtype != torch.int32 or coords.dim() != 2 or coords.shape[1] != 4:
        raise TscError(_lib.TSC_ERR_INVALID, "coords must be int32 of shape (N,4)")
    n = coords.shape[0]
    if nbr.dtype != torch.int32 or tuple(nbr.shape) != (n, 27):
        raise TscError(_lib.TSC_ERR_INVALID, "nbr must be int32 (N,27)")
    dev = _dev(coords, nbr)
    ctx = _lib.context(dev)
    nbytes = ctx.lib.tsc_map_gather_plan_bytes(n)
    if nbytes < 0:
        raise TscError(_lib.TSC_ERR_INVALID, f"gather plan: N={n} out of range")
    plan = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=coords.device)
    X, Y, Z = (int(s) for s in spatial_shape)
    check(ctx.lib.tsc_map_gather_plan(ctx.bind(), _p(coords), _p(nbr), n, int(batch_size), X, Y, Z,
                                      _p(plan)))
    return plan


def _raise_status(st: int, batch_size, spatial_shape) -> None:
    if st:
        X, Y, Z = spatial_shape
        what = []
        if st & _lib.TSC_MAP_DUPLICATE:
            what.append("duplicate coordinates")
        if st & _lib.TSC_MAP_OUT_OF_RANGE:
            what.append(f"coordinates outside [0,{batch_size})x[0,{X})x[0,{Y})x[0,{Z})")
        raise TscError(_lib.TSC_ERR_INVALID, "map build: " + ", ".join(what))


def build_neighbor_map(coords: torch.Tensor, spatial_shape, batch_size: int,
                       dilation=(1, 1, 1), kernel_size=(3, 3, 3), method: str = "auto",
                       validate: bool = True) -> NeighborMap:
    """Neighbor map of int32 (N,4) [b,x,y,z] coords on the GPU.

    validate=True reads the device status word back (one 4-byte sync) and raises on duplicate or
    out-of-range coordinates, whose outputs are undefined.  validate=False only enqueues the
    build (the operator path: the reference never checks either); NeighborMap.check() reads the
    status later.
    """
    if coords.dtype != torch.int32 or coords.dim() != 2 or coords.shape[1] != 4:
        raise TscError(_lib.TSC_ERR_INVALID, "coords must be int32 of shape (N,4)")
    dev = _dev(coords)
    ctx = _lib.context(dev)
    n = coords.shape[0]
    X, Y, Z = (int(s) for s in spatial_shape)
    kb = ctx.lib.tsc_map_key_bytes(int(batch_size), X, Y, Z)
    if kb == 0:
        raise TscError(_lib.TSC_ERR_INVALID, f"bad grid B={batch_size} shape={spatial_shape}")
    kdt = torch.int32 if kb == 4 else torch.int64
    nbr = torch.empty((n, 27), dtype=torch.int32, device=coords.device)
    keys = torch.empty((n,), dtype=kdt, device=coords.device)
    perm = torch.empty((n,), dtype=torch.int32, device=coords.device)
    status = torch.empty((1,), dtype=torch.int32, device=coords.device)
    k = (ctypes.c_int32 * 3)(*kernel_size)
    d = (ctypes.c_int32 * 3)(*dilation)
    check(ctx.lib.tsc_map_build(ctx.bind(), _p(coords), n, int(batch_size), X, Y, Z, k, d,
                                _lib.MAP_METHODS[method], _p(keys), _p(perm), _p(nbr), _p(status)))
    nmap = NeighborMap(nbr, keys, perm, (X, Y, Z), int(batch_size), tuple(dilation), coords,
                       status)
    if validate:
        nmap.check()
    return nmap


def _nbr_and_order(nmap, order):
    if isinstance(nmap, NeighborMap):
        return nmap.nbr, (nmap.conv_order() if order is None else order)
    return nmap, order


def _uses_gather_plan(nmap, order, feats, weight) -> bool:
    """Narrow 16-bit convs (Ci = 32, Co = 32/64) on a NeighborMap without an explicit order."""
    if not isinstance(nmap, NeighborMap) or order is not None or nmap.coords is None:
        return False
    return (feats.dtype in (torch.float16, torch.bfloat16) and weight.dim() == 5
            and weight.shape[4] == 32 and weight.shape[0] in (32, 64))


def sparse_conv3d(feats: torch.Tensor, weight: torch.Tensor, bias, nmap, order=None,
                  epilogue: str = "bias", residual=None, ln_weight=None, ln_bias=None,
                  eps: float = 1e-6, out=None) -> torch.Tensor:
    """out = bias + sum_v feats[nbr[:,v]] @ W[:,v,:]^T  (+ residual | -> LN -> SiLU).

    weight is (Co,Kd,Kh,Kw,Ci) = (Co,3,3,3,Ci), same dtype as feats; accumulation is fp32.
    nmap is a NeighborMap (its cached row order, or for Ci = 32 in fp16/bf16 its cached gather
    plan, is used for locality) or an (N,27) int32 table.
    """
    plan = nmap.gather_plan() if _uses_gather_plan(nmap, order, feats, weight) else None
    nbr, order = (nmap.nbr, None) if plan is not None else _nbr_and_order(nmap, order)
    if weight.dim() != 5 or tuple(weight.shape[1:4]) != (3, 3, 3):
        raise TscError(_lib.TSC_ERR_UNSUPPORTED, f"weight must be (Co,3,3,3,Ci), got {tuple(weight.shape)}")
    co, ci = weight.shape[0], weight.shape[4]
    n = feats.shape[0]
    if feats.dim() != 2 or feats.shape[1] != ci:
        raise TscError(_lib.TSC_ERR_INVALID, f"feats {tuple(feats.shape)} do not match Ci={ci}")
    if nbr.dtype != torch.int32 or tuple(nbr.shape) != (n, 27):
        raise TscError(_lib.TSC_ERR_INVALID, "neighbor map must be int32 (N,27)")
    for t in (weight, bias, residual, ln_weight, ln_bias, out):
        if t is not None and t.dtype != feats.dtype:
            raise TscError(_lib.TSC_ERR_INVALID, "all float tensors must share feats' dtype")
    if bias is not None and bias.numel() != co:
        raise TscError(_lib.TSC_ERR_INVALID, "bias must have Co elements")
    if order is not None and (order.dtype != torch.int32 or order.numel() != n):
        raise TscError(_lib.TSC_ERR_INVALID, "order must be int32 (N,)")
    epi = {"bias": _lib.TSC_EPI_BIAS, "residual": _lib.TSC_EPI_BIAS_RESIDUAL,
           "ln_silu": _lib.TSC_EPI_BIAS_LN_SILU}[epilogue]
    if epi == _lib.TSC_EPI_BIAS_RESIDUAL and (residual is None or tuple(residual.shape) != (n, co)):
        raise TscError(_lib.TSC_ERR_INVALID, "residual epilogue needs an (N,Co) residual")
    dev = _dev(feats, weight, bias, nbr, order, residual, ln_weight, ln_bias, out)
    if out is None:
        out = torch.empty((n, co), dtype=feats.dtype, device=feats.device)
    ctx = _lib.context(dev)
    if plan is not None:
        check(ctx.lib.tsc_conv_planned(ctx.bind(), _code(feats), _p(feats), _p(weight), _p(bias),
                                       _p(nbr), _p(plan), n, ci, co, epi, _p(residual), _p(ln_weight),
                                       _p(ln_bias), float(eps), _p(out)))
        return out
    check(ctx.lib.tsc_conv_fused(ctx.bind(), _code(feats), _p(feats), _p(weight), _p(bias), _p(nbr),
                                 _p(order), n, ci, co, epi, _p(residual), _p(ln_weight), _p(ln_bias),
                                 float(eps), _p(out)))
    return out


def layer_norm(x: torch.Tensor, weight=None, bias=None, eps: float = 1e-6, silu: bool = False,
               out=None) -> torch.Tensor:
    """Row LayerNorm over the last dim (fp32 math), optionally fused with SiLU."""
    c = x.shape[-1]
    rows = x.numel() // c if c else 0
    dev = _dev(x, weight, bias, out)
    if out is None:
        out = torch.empty_like(x)
    ctx = _lib.context(dev)
    check(ctx.lib.tsc_layernorm(ctx.bind(), _code(x), _p(x), rows, c,
                                _p(weight), _p(bias), float(eps), int(silu), _p(out)))
    return out


def silu(x: torch.Tensor, out=None) -> torch.Tensor:
    dev = _dev(x, out)
    if out is None:
        out = torch.empty_like(x)
    ctx = _lib.context(dev)
    check(ctx.lib.tsc_silu(ctx.bind(), _code(x), _p(x), x.numel(), _p(out)))
    return out


def add(a: torch.Tensor, b: torch.Tensor, out=None) -> torch.Tensor:
    if a.shape != b.shape or a.dtype != b.dtype:
        raise TscError(_lib.TSC_ERR_INVALID, "add: shapes and dtypes must match")
    dev = _dev(a, b, out)
    if out is None:
        out = torch.empty_like(a)
    ctx = _lib.context(dev)
    check(ctx.lib.tsc_add(ctx.bind(), _code(a), _p(a), _p(b), a.numel(), _p(out)))
    return out


def sparse_resblock(x: torch.Tensor, nmap, w1, b1, w2, b2, ln_weight=None, ln_bias=None,
                    eps: float = 1e-6, order=None, out=None) -> torch.Tensor:
    """out = x + conv2(silu(LN(conv1(x) + b1))) + b2, C = Ci = Co."""
    nbr, order = _nbr_and_order(nmap, order)
    n, c = x.shape
    for w in (w1, w2):
        if tuple(w.shape) != (c, 3, 3, 3, c) or w.dtype != x.dtype:
            raise TscError(_lib.TSC_ERR_INVALID, "resblock weights must be (C,3,3,3,C) of x's dtype")
    dev = _dev(x, nbr, order, w1, b1, w2, b2, ln_weight, ln_bias, out)
    if out is None:
        out = torch.empty_like(x)
    ctx = _lib.context(dev)
    check(ctx.lib.tsc_resblock(ctx.bind(), _code(x), _p(x), _p(nbr), _p(order), n, c, _p(w1), _p(b1),
                               _p(ln_weight), _p(ln_bias), float(eps), _p(w2), _p(b2), _p(out)))
    return out


def subdivide_count(keep: torch.Tensor) -> int:
    """Number of children a keep mask selects (uint8 (N,), bit c = child c); one stream sync."""
    if keep.dtype != torch.uint8 or keep.dim() != 1:
        raise TscError(_lib.TSC_ERR_INVALID, "keep must be uint8 of shape (N,)")
    ctx = _lib.context(_dev(keep))
    out = ctypes.c_int64(0)
    check(ctx.lib.tsc_subdivide_count(ctx.bind(), _p(keep), keep.shape[0], ctypes.byref(out)))
    return int(out.value)


def sparse_subdivide(coords: torch.Tensor, feats: torch.Tensor | None = None,
                     keep: torch.Tensor | None = None):
    """Children at twice the resolution (tsc_subdivide): (coords_out (M,4), feats_out (M,C)).

    Parent [b,x,y,z] -> children [b, 2x+dx, 2y+dy, 2z+dz], c = dx*4 + dy*2 + dz, parent-major,
    each with a copy of the parent's feature row; keep (uint8 (N,), bit c = keep child c) selects
    children (M = its set bits; counting them costs one stream sync), else M = 8N.
    """
    if coords.dtype != torch.int32 or coords.dim() != 2 or coords.shape[1] != 4:
        raise TscError(_lib.TSC_ERR_INVALID, "coords must be int32 of shape (N,4)")
    if feats is not None and (feats.dim() != 2 or feats.shape[0] != coords.shape[0]):
        raise TscError(_lib.TSC_ERR_INVALID, "feats must be (N,C) with the coords' N")
    if keep is not None and (keep.dtype != torch.uint8 or keep.shape != (coords.shape[0],)):
        raise TscError(_lib.TSC_ERR_INVALID, "keep must be uint8 of shape (N,)")
    dev = _dev(coords, feats, keep)
    ctx = _lib.context(dev)
    n = coords.shape[0]
    m = 8 * n if keep is None else subdivide_count(keep)
    coords_out = torch.empty((m, 4), dtype=torch.int32, device=coords.device)
    feats_out = None
    dtype, c = 0, 0
    if feats is not None:
        dtype, c = _code(feats), feats.shape[1]
        feats_out = torch.empty((m, c), dtype=feats.dtype, device=feats.device)
    if m:
        check(ctx.lib.tsc_subdivide(ctx.bind(), _p(coords), n, dtype, _p(feats), c, _p(keep),
                                    _p(coords_out), _p(feats_out)))
    return coords_out, feats_out


def sparse_linear(x: torch.Tensor, weight: torch.Tensor, bias=None, residual=None,
                  out=None) -> torch.Tensor:
    """out (N,Cout) = x (N,Cin) @ weight.T + bias (+ residual) (tsc_linear, one hipBLASLt GEMM);
    weight (Cout,Cin) as nn.Linear.  out may alias residual."""
    if x.dim() != 2 or weight.dim() != 2 or weight.shape[1] != x.shape[1]:
        raise TscError(_lib.TSC_ERR_INVALID, f"linear: x {tuple(x.shape)} vs weight {tuple(weight.shape)}")
    n, cin = x.shape
    cout = weight.shape[0]
    if bias is not None and bias.shape != (cout,):
        raise TscError(_lib.TSC_ERR_INVALID, "linear: bias must be (Cout,)")
    if residual is not None and residual.shape != (n, cout):
        raise TscError(_lib.TSC_ERR_INVALID, "linear: residual must be (N,Cout)")
    for t in (weight, bias, residual):
        if t is not None and t.dtype != x.dtype:
            raise TscError(_lib.TSC_ERR_INVALID, "linear: dtype mismatch")
    if out is None:
        out = torch.empty((n, cout), dtype=x.dtype, device=x.device)
    ctx = _lib.context(_dev(x, weight, bias, residual, out))
    check(ctx.lib.tsc_linear(ctx.bind(), _code(x), _p(x), n, cin, _p(weight), _p(bias),
                             _p(residual), cout, _p(out)))
    return out


def _cu_seqlens(cu, total: int, dev: int, what: str):
    """cu_seqlens as (host int64 array or None, device int32 tensor).

    A host sequence is checked non-decreasing within [0, total] and copied to the device.  A
    device tensor is taken as given (host None): reading it would synchronize the stream, and the
    kernels clamp every offset into [0, total], so a malformed array cannot read out of bounds."""
    import numpy as np

    if isinstance(cu, torch.Tensor) and cu.is_cuda:
        if cu.dim() != 1 or cu.numel() < 1:
            raise TscError(_lib.TSC_ERR_INVALID, f"{what} must be a 1-D (B+1,) sequence")
        d = cu if cu.dtype == torch.int32 and cu.is_contiguous() else cu.to(torch.int32).contiguous()
        return None, d
    host = (cu.detach().to("cpu", torch.int64).numpy() if isinstance(cu, torch.Tensor)
            else np.asarray(cu, np.int64))
    if host.ndim != 1 or host.size < 1:
        raise TscError(_lib.TSC_ERR_INVALID, f"{what} must be a 1-D (B+1,) sequence")
    if (np.diff(host) < 0).any() or host[0] < 0 or host[-1] > total:
        raise TscError(_lib.TSC_ERR_INVALID, f"{what} must be non-decreasing within [0, {total}]")
    return host, torch.from_numpy(host.astype(np.int32)).to(f"cuda:{dev}")


def sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q,
                     cu_seqlens_kv=None, num_heads: int | None = None, head_dim: int | None = None,
                     scale: float | None = None, out=None,
                     max_seqlen_q: int | None = None) -> torch.Tensor:
    """sparseAttention (src/sparse/ops/attention.ts:24-79) on the GPU for any batch size.

    q (total_q, H, D) and k / v (total_kv, H, D), or (total, H*D) with num_heads; cu_seqlens_q /
    cu_seqlens_kv (B+1,) row offsets of each sequence (host sequence or tensor; cu_seqlens_kv
    defaults to cu_seqlens_q).  Returns (total_q, H, D) in q's dtype.  scale defaults to
    1/sqrt(D).  One tsc_attention call; no host round trip: device cu_seqlens are never read on
    the host (they are not validated there; the kernel clamps them), and then max_seqlen_q, which
    only sizes the grid, defaults to min(total_q, 2 * ceil(total_q / B)) — every query is covered
    whatever its sequence's length, longer ones at a lower parallelism.  Rows of a new `out`
    outside every query sequence are zero, as in the reference's zero-initialised output
    (attention.ts:49)."""
    dev = _dev(q, k, v, out)
    if q.dim() == 2:
        if not num_heads:
            raise TscError(_lib.TSC_ERR_INVALID, "num_heads is required for (total, H*D) inputs")
        h = num_heads
        d = q.shape[1] // h
    else:
        h, d = q.shape[1], q.shape[2]
    if num_heads is not None and num_heads != h or head_dim is not None and head_dim != d:
        raise TscError(_lib.TSC_ERR_INVALID, f"num_heads/head_dim {num_heads}/{head_dim} do not "
                                             f"match the query shape {tuple(q.shape)}")
    tq, tkv = q.shape[0], k.shape[0]
    for name, t, n in (("q", q, tq), ("k", k, tkv), ("v", v, tkv)):
        if t.numel() != n * h * d or t.dtype != q.dtype:
            raise TscError(_lib.TSC_ERR_INVALID, f"{name} must hold ({n}, {h}, {d}) {q.dtype} values")
    cq_host, cq = _cu_seqlens(cu_seqlens_q, tq, dev, "cu_seqlens_q")
    if cu_seqlens_kv is None:
        cu_seqlens_kv = cu_seqlens_q
    _, ck = _cu_seqlens(cu_seqlens_kv, tkv, dev, "cu_seqlens_kv")
    if ck.numel() != cq.numel():
        raise TscError(_lib.TSC_ERR_INVALID, "cu_seqlens_q and cu_seqlens_kv differ in length")
    b = cq.numel() - 1
    if out is None:
        # the kernel writes every row inside a query sequence; zero-fill unless they cover all
        covered = cq_host is not None and b > 0 and cq_host[0] == 0 and cq_host[-1] == tq
        out = (torch.empty if covered else torch.zeros)((tq, h, d), dtype=q.dtype, device=q.device)
    elif out.numel() != tq * h * d or out.dtype != q.dtype:
        raise TscError(_lib.TSC_ERR_INVALID, "out has the wrong size or dtype")
    if max_seqlen_q is None:
        if cq_host is not None:
            max_seqlen_q = int((cq_host[1:] - cq_host[:-1]).max()) if b > 0 else 0
        else:
            max_seqlen_q = min(tq, 2 * -(-tq // b)) if b > 0 else 0
    ctx = _lib.context(dev)
    check(ctx.lib.tsc_attention(ctx.bind(), _code(q), _p(q), _p(k), _p(v), _p(cq), _p(ck), b, tq,
                                tkv, h, d, float(scale) if scale else 0.0, int(max_seqlen_q),
                                _p(out)))
    return out.view(tq, h, d)


def scaled_dot_product_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                 num_heads: int, batch_size: int = 1, scale=None) -> torch.Tensor:
    """scaledDotProductAttention (src/dense/ops/attention.ts:36-110): q (B*S_q, H, D) or
    (B, S_q, H, D), k / v likewise with S_kv; batch_size equal-length sequences."""
    sq = q.numel() // (batch_size * q.shape[-1] * num_heads)
    skv = k.numel() // (batch_size * k.shape[-1] * num_heads)
    d = q.shape[-1]
    cq = [i * sq for i in range(batch_size + 1)]
    ck = [i * skv for i in range(batch_size + 1)]
    o = sparse_attention(q.reshape(-1, num_heads, d), k.reshape(-1, num_heads, d),
                         v.reshape(-1, num_heads, d), cq, ck, scale=scale)
    return o.view(q.shape)
