"""ORACLE — TEST INFRASTRUCTURE ONLY.  Verify-step mask producers with loops.

* ``mtp_mask`` — batchspec/backends/mtp_engine.py:172-208 (rule in its docstring:
  a regular row sees earlier-or-equal regular columns; a mask row additionally sees
  the same group's mask columns up to itself; position = group + slot).
* ``tree_ancestor_mask`` — draft tree from a parent array: node i sees node j iff j
  is i or an ancestor of i (EAGLE tree verification).
"""
from __future__ import annotations

import numpy as np


def mtp_mask(k: int):
    S = (k + 1) ** 2
    m = np.zeros((S, S), dtype=bool)
    pos = np.zeros(S, dtype=np.int64)
    for i in range(S):
        gi, ri = divmod(i, k + 1)
        pos[i] = gi + ri
        for j in range(S):
            gj, rj = divmod(j, k + 1)
            if rj == 0 and j <= i:
                m[i, j] = True
            elif gi == gj and 1 <= rj <= ri:
                m[i, j] = True
    return m, pos


def tree_ancestor_mask(parents):
    n = len(parents)
    m = np.zeros((n, n), dtype=bool)
    depth = np.zeros(n, dtype=np.int64)
    for i in range(n):
        j = i
        d = 0
        while j >= 0:
            m[i, j] = True
            j = parents[j]
            d += 1
        depth[i] = d - 1
    return m, depth
