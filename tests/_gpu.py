"""Helpers shared by the GPU parity tests (they compare the HIP path with the oracle)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle.projection import Canonical


def require_gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from purin_amd import _lib

    _lib.load()  # raises if the HIP library is missing: never a silent fallback
    return torch


def csr_from_canonical(canon: Canonical):
    indptr = np.zeros(len(canon.rows) + 1, np.int64)
    indptr[1:] = np.cumsum([len(r) for r in canon.rows])
    indices = np.asarray([c for r in canon.rows for c in r], np.int32)
    data = np.asarray([v for c in canon.coef for v in c], np.float64)
    return indptr, indices, data


def canonical_from_workload(w):
    return Canonical(n=w.n, me=w.me, rows=w.rows(), coef=w.coefs())


def plan_for(canon: Canonical, *, dtype, accelerated=False, **kw):
    from purin_amd.plan import Plan

    indptr, indices, data = csr_from_canonical(canon)
    return Plan(canon.n, canon.me, canon.mi, indptr, indices, data, dtype=dtype,
                accelerated=accelerated, **kw)


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = max(np.max(np.abs(b)), 1e-300) if b.size else 1.0
    return float(np.max(np.abs(a - b)) / scale) if b.size else 0.0


def to_np(t):
    return t.detach().cpu().numpy()
