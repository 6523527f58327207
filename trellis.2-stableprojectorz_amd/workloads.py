"""Seeded synthetic workloads: voxel shells of randomly perturbed ellipsoids.

A solid is the set of voxels whose centre p+0.5 satisfies
    |q| < 1 + amp * sin(f1*theta + phi0) * cos(f2*phi + phi1),   q = (p+0.5 - c) / axes,
with theta/phi the polar/azimuthal angles of q, centre c = grid/2 + U[-1,1]^3, semi-axes
U[lo,hi]^3 and phases U[0,2pi).  A k-voxel shell is the solid minus its k-fold 6-connected
erosion.  Rows are shuffled with the same seed.  Everything is numpy with a seeded PCG64
generator, so the same seed gives the same voxels on any machine.

The five workloads of the sparse conv3d path (sizes as used by tests and bench.py):
  conv64_f32      64^3, 2-voxel shell, ~20k voxels, conv 64->64 fp32
  map512          512^3, 1-voxel shell, ~1.5M voxels, shuffled: neighbor-map build
  narrow512_f16   the map512 voxels, conv 32->32 and 32->64 fp16
  wide128_bf16    4 samples x ~60k voxels, 128^3, 2-voxel shells, conv 512->512 bf16
  resblock64_bf16 2 samples x ~30k voxels, 64^3, 2-voxel shells, 4 ResBlocks at C=1024 bf16
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class ShellSpec:
    grid: int
    axes_lo: float
    axes_hi: float
    thickness: int
    amp: float
    freqs: tuple


SHELLS = {
    "conv64": ShellSpec(64, 20.0, 30.0, 2, 0.30, (6, 5)),
    "map512": ShellSpec(512, 200.0, 250.0, 1, 0.35, (10, 8)),
    "map512s2": ShellSpec(512, 200.0, 250.0, 2, 0.35, (10, 8)),
    "wide128": ShellSpec(128, 34.0, 45.0, 2, 0.30, (7, 6)),
    "res64": ShellSpec(64, 22.0, 27.0, 2, 0.40, (8, 7)),
}


def _solid(spec: ShellSpec, rng: np.random.Generator) -> np.ndarray:
    g = spec.grid
    axes = rng.uniform(spec.axes_lo, spec.axes_hi, 3).astype(np.float32)
    centre = (g / 2 + rng.uniform(-1.0, 1.0, 3)).astype(np.float32)
    phases = rng.uniform(0.0, 2 * np.pi, 2).astype(np.float32)
    idx = np.arange(g, dtype=np.float32) + np.float32(0.5)
    out = np.zeros((g, g, g), dtype=bool)
    f1, f2 = np.float32(spec.freqs[0]), np.float32(spec.freqs[1])
    amp = np.float32(spec.amp)
    qy = ((idx - centre[1]) / axes[1])[None, :, None]
    qz = ((idx - centre[2]) / axes[2])[None, None, :]
    for x0 in range(0, g, 32):
        qx = ((idx[x0:x0 + 32] - centre[0]) / axes[0])[:, None, None]
        r = np.sqrt(qx * qx + qy * qy + qz * qz)
        theta = np.arccos(np.clip(qz / np.maximum(r, np.float32(1e-12)), -1.0, 1.0))
        phi = np.arctan2(qy, qx)
        lim = 1.0 + amp * np.sin(f1 * theta + phases[0]) * np.cos(f2 * phi + phases[1])
        out[x0:x0 + 32] = r < lim
    return out


def _erode6(m: np.ndarray) -> np.ndarray:
    e = m.copy()
    e[1:] &= m[:-1]
    e[:-1] &= m[1:]
    e[:, 1:] &= m[:, :-1]
    e[:, :-1] &= m[:, 1:]
    e[:, :, 1:] &= m[:, :, :-1]
    e[:, :, :-1] &= m[:, :, 1:]
    e[0] = e[-1] = False
    e[:, 0] = e[:, -1] = False
    e[:, :, 0] = e[:, :, -1] = False
    return e


def shell_coords(spec: ShellSpec, seed: int, batch: int = 1, shuffle: bool = True) -> np.ndarray:
    """(N,4) int32 rows [b,x,y,z]: `batch` independent shells, concatenated by batch."""
    rng = np.random.default_rng(seed)
    parts = []
    for b in range(batch):
        solid = _solid(spec, rng)
        core = solid
        for _ in range(spec.thickness):
            core = _erode6(core)
        xyz = np.argwhere(solid & ~core).astype(np.int32)
        if shuffle:
            xyz = xyz[rng.permutation(len(xyz))]
        parts.append(np.concatenate([np.full((len(xyz), 1), b, np.int32), xyz], axis=1))
    return np.ascontiguousarray(np.concatenate(parts, axis=0))


def features(n: int, c: int, seed: int) -> np.ndarray:
    """N(0,1) features, float32."""
    return np.random.default_rng(seed).standard_normal((n, c), dtype=np.float32)


def conv_weight(co: int, ci: int, seed: int) -> np.ndarray:
    """(Co,3,3,3,Ci) float32 weights ~ N(0, 1/sqrt(27*Ci))."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((co, 3, 3, 3, ci), dtype=np.float32)
    return w * np.float32(1.0 / np.sqrt(27.0 * ci))


@dataclass(frozen=True)
class Workload:
    name: str
    shell: str
    batch: int
    seed: int
    channels: tuple  # (Ci, Co) pairs of the convs measured on this voxel set
    dtype: str       # "float32" | "float16" | "bfloat16" | "int32" (map build only)
    description: str


WORKLOADS = {
    "conv64_f32": Workload("conv64_f32", "conv64", 1, 101, ((64, 64),), "float32",
                           "conv3x3x3 64->64 fp32, ~20k voxels, 2-voxel shell in 64^3"),
    "map512": Workload("map512", "map512", 1, 202, (), "int32",
                       "neighbor-map build, ~1.5M voxels, 1-voxel shell in 512^3, shuffled"),
    "narrow512_f16": Workload("narrow512_f16", "map512", 1, 202, ((32, 32), (32, 64)), "float16",
                              "conv3x3x3 32->32 and 32->64 fp16, ~1.5M voxels in 512^3"),
    "narrow512s2_f16": Workload("narrow512s2_f16", "map512s2", 1, 202, ((32, 32), (32, 64)),
                                "float16", "conv3x3x3 32->32 and 32->64 fp16, ~3.0M voxels of a "
                                "2-voxel shell in 512^3 (the thickness subdivision gives)"),
    "wide128_bf16": Workload("wide128_bf16", "wide128", 4, 404, ((512, 512),), "bfloat16",
                             "conv3x3x3 512->512 bf16, 4 x ~60k voxels, 2-voxel shells in 128^3"),
    "resblock64_bf16": Workload("resblock64_bf16", "res64", 2, 505, ((1024, 1024),), "bfloat16",
                                "4 x ResBlock(conv-LN-SiLU-conv-+x) C=1024 bf16, 2 x ~30k voxels"),
}


def make_coords(workload: str) -> np.ndarray:
    w = WORKLOADS[workload]
    return shell_coords(SHELLS[w.shell], w.seed, w.batch)


def grid_shape(workload: str) -> tuple:
    g = SHELLS[WORKLOADS[workload].shell].grid
    return (g, g, g)
