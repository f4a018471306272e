"""Shared helpers of the GPU parity tests (the oracle is the checker)."""
import numpy as np

from oracle import core, kvpool as kp


def rel_err(got, want):
    """max |got - want| / max |want| per row, then the max over rows."""
    got = np.asarray(got, np.float64).reshape(len(want), -1)
    want = np.asarray(want, np.float64).reshape(len(want), -1)
    den = np.maximum(np.abs(want).max(axis=1), 1e-30)
    return float((np.abs(got - want).max(axis=1) / den).max())


def lcg_ints(seed, n, lo, hi):
    """Integers U[lo, hi) from the reference LCG (test/tiny.lua:16-22)."""
    r = core.Lcg(seed)
    return [lo + int(r.next() * (hi - lo)) for _ in range(n)]


class Schedule:
    """Pool sequences over one oracle pool bookkeeping (block tables)."""

    def __init__(self, n_blocks, n_seqs):
        self.pool = kp.Pool(n_blocks, 64)
        self.seqs = [kp.Seq(self.pool) for _ in range(n_seqs)]

    def grow(self, s, n):
        kp.reserve(self.seqs[s], n)

    def table(self, which):
        nb = max(1, max(len(self.seqs[s].blocks) for s in which))
        bt = np.full((len(which), nb), -1, np.int32)
        for i, s in enumerate(which):
            b = self.seqs[s].blocks
            bt[i, :len(b)] = b
        return bt


def oracle_pools(hp, n_cells):
    row = hp["n_head_kv"] * hp["head_dim"]
    return ([np.zeros((n_cells, row), np.uint16) for _ in range(hp["n_layer"])],
            [np.zeros((n_cells, row), np.uint16) for _ in range(hp["n_layer"])])
