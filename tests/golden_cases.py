"""Loading of the golden fixtures in tests/golden/ (see make_golden.py there)."""

from __future__ import annotations

import functools
import json
from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"


def _tensor(a: np.ndarray, bf16: bool) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.view(torch.int16).view(torch.bfloat16) if bf16 else t


def load(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        meta = json.loads(str(z["meta"]))
        return {
            "meta": meta,
            "x": _tensor(z["x"].astype(np.uint16).view(np.int16), True),
            "logits": _tensor(z["logits"].astype(np.uint16).view(np.int16), True),
            "weights": _tensor(z["weights"].astype(np.uint16).view(np.int16), True),
            "indices": _tensor(z["indices"], False),
            "out": _tensor(z["out"].astype(np.uint16).view(np.int16), True),
        }


def names() -> list[str]:
    return sorted(p.stem for p in GOLDEN.glob("*.npz"))


@functools.lru_cache(maxsize=2)
def regenerate(name: str):
    """(shape, layer, dense, x, layer_index, bias) rebuilt on the CPU from the seeds."""
    from golden.make_golden import case_inputs

    return case_inputs(name)
