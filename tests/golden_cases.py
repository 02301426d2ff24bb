"""Loader for the committed golden fixtures (tests/golden/*.npz)."""
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def names():
    with open(os.path.join(GOLDEN, "cases.json")) as f:
        return [c["name"] for c in json.load(f)]


def load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    d["alpha"] = float(d["alpha"])
    d["beta"] = float(d["beta"])
    d["K"] = int(d["K"])
    return d
