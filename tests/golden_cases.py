"""Loader for tests/golden/reference_cases.npz (made by tests/golden/make_golden.py)."""
from pathlib import Path

import numpy as np

PATH = Path(__file__).resolve().parent / "golden" / "reference_cases.npz"


def load():
    z = np.load(PATH, allow_pickle=False)
    gemv, deq = {}, {}
    for key in z.files:
        name, field = key.split("__")
        (deq if name.startswith("dq_") else gemv).setdefault(name, {})[field] = z[key]
    for d in (gemv, deq):
        for v in d.values():
            v["fmt"] = str(v["fmt"])
    return gemv, deq
