"""Loader of the committed config1 fixture (tests/golden/config1.npz)."""

from __future__ import annotations

import os

import numpy as np

from oracle.projection import Canonical

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config1.npz")


def load():
    with np.load(PATH, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def canonical(g):
    ptr, idx, val = g["indptr"], g["indices"], g["data"]
    rows = [list(map(int, idx[ptr[i]:ptr[i + 1]])) for i in range(len(ptr) - 1)]
    coef = [list(map(float, val[ptr[i]:ptr[i + 1]])) for i in range(len(ptr) - 1)]
    return Canonical(n=g["target"].shape[1], me=int(g["me"]), rows=rows, coef=coef)


def masks(y, multipliers, me, mi_general, lower=-1.0, upper=1.0):
    """Active sets: y == lower, y == upper, d_I > 0 on the general inequality rows,
    recovered bound multipliers > 0."""
    ineq = multipliers[:, me:]
    return (y == lower, y == upper, ineq[:, :mi_general] > 0, ineq[:, mi_general:] > 0)
