"""The ResBlock chain at its full stated size: 4 x (conv 1024->1024 -> LN(eps 1e-6) -> SiLU ->
conv 1024->1024 -> + x), bf16, batch 2 x ~32k voxels of 2-voxel shells in 64^3
(workloads.make_coords("resblock64_bf16")).

Checks, all on the full two-sample coordinate set unless stated:
  * one block against the fp64 oracle on 150 sampled rows per sample: conv1 is evaluated by the
    oracle only on the union of the sampled rows' neighbourhoods (the rows conv2 reads);
  * the 4-block chain against the fp32 restatement of conv_none (oracle/torch_path.py, run on the
    GPU with torch fp32 matmuls) plus fp32 LayerNorm / SiLU, every row;
  * exact properties of the chain: with W2 = 0 every block returns bf16(x + b2) bit for bit, and
    the rows of sample 0 in the batch-2 run equal a batch-1 run of sample 0 alone bit for bit;
  * the 4-block chain on a batch-2 subset (a compact 400-voxel patch per sample) against
    oracle.resblock applied 4 times in fp64.
Tolerance: norm-wise relative max|y - r| / max|r| <= 2e-2 (bf16 storage, fp32 accumulation),
reference computed from the same bf16-rounded inputs and weights.  Block semantics: the config's
chain as stated (conv -> LN -> SiLU -> conv -> +x); the reference's decoder blocks compose the
same ops (src/models/sparse_unet_vae_decoder.ts:48-78).
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import torch_path

pytestmark = pytest.mark.gpu

C = 1024
BLOCKS = 4
TOL = 2e-2


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


@pytest.fixture(scope="module")
def res64(pkg, dev):
    coords = pkg.workloads.make_coords("resblock64_bf16")
    n = len(coords)
    print(f"  resblock64 full: N={n} B=2 C={C}", flush=True)
    cd = torch.from_numpy(coords).to(dev)
    nmap = pkg.build_neighbor_map(cd, (64, 64, 64), 2)
    dt = torch.bfloat16
    x = torch.from_numpy(pkg.workloads.features(n, C, 1)).to(dev).to(dt)
    ws = []
    for i in range(BLOCKS):
        w1 = torch.from_numpy(pkg.workloads.conv_weight(C, C, 10 + i)).to(dev).to(dt)
        w2 = torch.from_numpy(pkg.workloads.conv_weight(C, C, 20 + i)).to(dev).to(dt)
        b1 = torch.linspace(-0.05, 0.05, C, device=dev).to(dt)
        b2 = torch.linspace(0.05, -0.05, C, device=dev).to(dt)
        ws.append((w1, b1, w2, b2))
    return {"coords": coords, "nmap": nmap, "x": x, "ws": ws, "n": n}


def _chain(pkg, x, nmap, ws):
    h = x
    for w1, b1, w2, b2 in ws:
        h = pkg.sparse_resblock(h, nmap, w1, b1, w2, b2, eps=1e-6)
    return h


def test_block_full_size_sampled_rows_vs_oracle(pkg, dev, res64):
    nmap, x, n = res64["nmap"], res64["x"], res64["n"]
    w1, b1, w2, b2 = res64["ws"][0]
    out = pkg.sparse_resblock(x, nmap, w1, b1, w2, b2, eps=1e-6).float().cpu().numpy()
    nbr = nmap.nbr.cpu().numpy()
    batch = res64["coords"][:, 0]
    rng = np.random.default_rng(31)
    rows = np.sort(np.concatenate([rng.choice(np.nonzero(batch == b)[0], 150, replace=False)
                                   for b in (0, 1)]))
    sub = nbr[rows]
    need = np.unique(sub[sub >= 0])  # rows of h that conv2 reads for the sampled outputs
    print(f"  oracle conv1 on {len(need)} rows", flush=True)
    x64 = torch.from_numpy(x.float().cpu().numpy().astype(np.float64))
    h = torch_path.conv_none(x64, w1.float().cpu().double(), b1.float().cpu().double(),
                             torch.from_numpy(nbr[need]), acc_dtype=torch.float64).numpy()
    h = oracle.layernorm(h, None, None, 1e-6, silu=True)
    local = np.full(n, -1, np.int32)
    local[need] = np.arange(len(need), dtype=np.int32)
    sub_local = np.where(sub >= 0, local[np.maximum(sub, 0)], -1).astype(np.int32)
    ref = x64.numpy()[rows] + oracle.conv(h, w2.float().cpu().numpy(),
                                          b2.float().cpu().numpy(), sub_local)
    err = rel_err(out[rows], ref)
    print(f"  block rel err {err:.3e}", flush=True)
    assert err <= TOL, err


def test_chain_full_size_vs_fp32_restatement(pkg, dev, res64):
    """All rows of the 4-block chain against conv_none in fp32 on the GPU (intermediates fp32)."""
    nmap, x = res64["nmap"], res64["x"]
    got = _chain(pkg, x, nmap, res64["ws"]).float()
    nbr = nmap.nbr
    ref = x.float()
    for w1, b1, w2, b2 in res64["ws"]:
        h = torch_path.conv_none(ref, w1.float(), b1.float(), nbr, acc_dtype=torch.float32)
        h = torch.nn.functional.silu(torch.nn.functional.layer_norm(h, (C,), eps=1e-6))
        ref = ref + torch_path.conv_none(h, w2.float(), b2.float(), nbr, acc_dtype=torch.float32)
    err = float((got - ref).abs().max() / ref.abs().max())
    print(f"  chain rel err {err:.3e}", flush=True)
    assert err <= TOL, err


def test_chain_full_size_zero_w2_is_residual_plus_bias(pkg, dev, res64):
    """W2 = 0: conv2 contributes exact zeros, so each block returns bf16(x + b2) bit for bit."""
    nmap, x = res64["nmap"], res64["x"]
    h = x
    for w1, b1, w2, b2 in res64["ws"]:
        out = pkg.sparse_resblock(h, nmap, w1, b1, torch.zeros_like(w2), b2, eps=1e-6)
        want = (h.float() + b2.float()).to(torch.bfloat16)
        assert torch.equal(out, want)
        h = out


def test_chain_batch_independence_bit_exact(pkg, dev, res64):
    """Sample 0's rows of the batch-2 chain equal a batch-1 chain of sample 0 alone, bit for bit
    (rows are grouped by batch, sample 0 first, so its neighbor indices are the same)."""
    coords, x = res64["coords"], res64["x"]
    n0 = int((coords[:, 0] == 0).sum())
    assert (coords[:n0, 0] == 0).all()
    both = _chain(pkg, x, res64["nmap"], res64["ws"])
    m0 = pkg.build_neighbor_map(torch.from_numpy(coords[:n0].copy()).to(dev), (64, 64, 64), 1)
    assert torch.equal(m0.nbr, res64["nmap"].nbr[:n0])
    alone = _chain(pkg, x[:n0].contiguous(), m0, res64["ws"])
    assert torch.equal(both[:n0], alone)


def _patch(coords, b, k):
    """A compact patch of sample b: its k voxels with the smallest x + y + z."""
    idx = np.nonzero(coords[:, 0] == b)[0]
    s = coords[idx, 1:].sum(1)
    return idx[np.argsort(s, kind="stable")[:k]]


def test_chain_batch2_subset_vs_oracle(pkg, dev, res64):
    coords = res64["coords"]
    sel = np.concatenate([_patch(coords, 0, 400), _patch(coords, 1, 400)])
    sub = coords[sel].copy()
    n = len(sub)
    m = pkg.build_neighbor_map(torch.from_numpy(sub).to(dev), (64, 64, 64), 2)
    nbr = m.nbr.cpu().numpy()
    print(f"  subset N={n}, valid taps per row {np.mean((nbr >= 0).sum(1)):.1f}", flush=True)
    x = res64["x"][torch.from_numpy(sel).to(dev)].contiguous()
    got = _chain(pkg, x, m, res64["ws"]).float().cpu().numpy()
    ref = x.float().cpu().numpy().astype(np.float64)
    for w1, b1, w2, b2 in res64["ws"]:
        ref = oracle.resblock(ref, nbr, w1.float().cpu().numpy(), b1.float().cpu().numpy(),
                              w2.float().cpu().numpy(), b2.float().cpu().numpy(), eps=1e-6)
    err = rel_err(got, ref)
    print(f"  subset chain rel err {err:.3e}", flush=True)
    assert err <= TOL, err
