"""Reader of the golden fixtures in tests/golden (format of src/validation/loader.ts:1-68)."""
import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def cases():
    return sorted(p.name for p in GOLDEN.iterdir() if (p / "metadata.json").exists())


def load(case: str):
    d = GOLDEN / case
    md = json.loads((d / "metadata.json").read_text())
    arrays = {}
    for kind in ("inputs", "expected"):
        for e in md[kind]:
            key = e["file"].split("_", 1)[1].rsplit(".", 1)[0]
            arr = np.fromfile(d / e["file"], dtype=np.dtype(e["dtype"])).reshape(e["shape"])
            arrays[("in" if kind == "inputs" else "exp", key)] = arr
    return md, arrays


def meta_tuple(md, key):
    return tuple(int(v) for v in md["metadata"][key].split(","))
