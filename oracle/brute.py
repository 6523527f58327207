"""Pure-Python brute-force neighbor map for tiny inputs — TEST INFRASTRUCTURE ONLY.

Straight from the definition in src/sparse/ops/conv3d_wgsl.ts:91-124: for each voxel and each of
the 27 offsets, scan a Python dict of (b,x,y,z) -> row.  No sorting, no packing, no bitmaps.
"""
from __future__ import annotations


def neighbor_map(coords, shape, dilation=(1, 1, 1)):
    X, Y, Z = shape
    table = {}
    for i, (b, x, y, z) in enumerate(coords):
        table[(int(b), int(x), int(y), int(z))] = i
    out = []
    for b, x, y, z in coords:
        row = []
        for kd in range(3):
            for kh in range(3):
                for kw in range(3):
                    nx = int(x) + (kd - 1) * dilation[0]
                    ny = int(y) + (kh - 1) * dilation[1]
                    nz = int(z) + (kw - 1) * dilation[2]
                    if 0 <= nx < X and 0 <= ny < Y and 0 <= nz < Z:
                        row.append(table.get((int(b), nx, ny, nz), -1))
                    else:
                        row.append(-1)
        out.append(row)
    return out
