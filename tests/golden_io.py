"""Loads the golden fixtures of tests/golden/ (written by tests/golden/make_golden.py)."""
import glob
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def names(kind):
    return sorted(os.path.basename(p)[len(kind) + 1:-4] for p in glob.glob(os.path.join(GOLDEN, f"{kind}_*.npz")))


def load(kind, name):
    with np.load(os.path.join(GOLDEN, f"{kind}_{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}
