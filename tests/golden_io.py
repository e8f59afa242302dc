"""Reading the golden fixtures of tests/golden into torch tensors."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"


def names(prefix: str) -> list[str]:
    return sorted(p.stem for p in GOLDEN.glob(f"{prefix}_*.npz"))


def load(name: str) -> dict:
    """Inputs as float32 tensors (bf16 bits widened exactly), bounds as lists, spans as (s, e) tuples."""
    z = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    case = {}
    for t in ("q", "k", "v"):
        if f"{t}_bf16" in z:
            bits = z[f"{t}_bf16"].astype(np.uint32) << 16
            case[t] = torch.from_numpy(bits.view(np.float32).copy())
        else:
            case[t] = torch.from_numpy(z[t].astype(np.float32))
    case["q_cu"] = [int(x) for x in z["q_cu"]]
    case["k_cu"] = [int(x) for x in z["k_cu"]]
    case["left"], case["right"] = int(z["left"]), int(z["right"])
    case["spans"] = [(int(s), int(e)) for s, e in z["spans"]]
    case["scale"] = float(z["scale"])
    case["want"] = torch.from_numpy(z["want"].astype(np.float64))
    return case
