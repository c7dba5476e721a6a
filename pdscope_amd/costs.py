"""Per-expert cost tables for the placement planner.

A table file is JSON with ``"kind": "pdscope_cost_table"`` and ``points``: for
each measured routed-token count of one expert (the domain runs from 1 to
4096) the milliseconds that expert costs on the CPU backend (``cpu_ms``), as
resident GPU work (``gpu_ms``) and staged from host memory then computed
(``h2d_ms``).  This is the format the reference planner reads through its
FileCosts (benchmarks/pdscope_compare.py:55-85); ``for_load(n)`` answers with
``{"tokens": n, <field>: ms, ...}``.

Between measured counts every field is interpolated linearly (each segment
on its own, so a table may bend); outside the measured domain the table
refuses to extrapolate.  ``costs/mi355x_cost_table.json`` is the table
measured on MI355X by ``bench.py --calibrate-costs``.

``ResidentGraphCosts`` wraps a table for a runtime that serves resident
decode layers through a cheaper resident launch (the reference's captured
graphs; the cost modes of expertbench/pdscope_runtime.py:40-59).
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

COSTS_DIR = Path(__file__).resolve().parent.parent / "costs"
TABLE_KIND = "pdscope_cost_table"
DOMAIN = (1, 4096)


class FileCosts:
    """A measured cost table loaded from JSON (see the module docstring)."""

    def __init__(self, path):
        path = Path(path)
        blob = path.read_bytes()
        doc = json.loads(blob)
        if doc.get("kind") != TABLE_KIND:
            raise ValueError(f"not a cost table: kind is {doc.get('kind')!r}, expected {TABLE_KIND!r}")
        measured = sorted((int(n), {field: float(ms) for field, ms in row.items()})
                          for n, row in doc.get("points", {}).items())
        if not measured or (measured[0][0], measured[-1][0]) != DOMAIN:
            raise ValueError(f"cost table must be measured at both ends of its domain {DOMAIN[0]}..{DOMAIN[1]}")
        fields = set(measured[0][1])
        if any(set(row) != fields for _, row in measured):
            raise ValueError("every point of a cost table must carry the same fields")
        self.loads = [n for n, _ in measured]
        self.points = dict(measured)
        self._fields = sorted(fields)
        self._grid = np.array(self.loads, dtype=np.float64)
        self._curves = {f: np.array([row[f] for _, row in measured], dtype=np.float64) for f in self._fields}
        # provenance of the numbers a plan rests on (recorded next to results)
        self.sources = [dict(path=str(path.resolve()), sha256=hashlib.sha256(blob).hexdigest(),
                             kind="shipped_cost_table", platform=doc.get("platform"), model=doc.get("model"),
                             scope=doc.get("scope"))]

    def for_load(self, n):
        """Costs of one expert serving n routed tokens."""
        if not DOMAIN[0] <= n <= DOMAIN[1]:
            raise ValueError(f"expert load {n} lies outside the measured domain {DOMAIN[0]}..{DOMAIN[1]}")
        exact = self.points.get(n)
        if exact is not None:
            return {"tokens": n, **exact}
        return {"tokens": n, **{f: float(np.interp(n, self._grid, self._curves[f])) for f in self._fields}}


class ResidentGraphCosts:
    """A cost table seen by a runtime whose resident decode experts run a
    cheaper resident launch (the reference's captured graphs; here the bound
    single-launch layer).  mode 'eager_bound' leaves every cost as measured
    eagerly (the default: misses and speculative copies still run eagerly);
    'measured' charges one-token GPU work at the calibrated resident-launch
    cost and keeps the staged path's total (copy + compute) unchanged."""

    MODES = ("eager_bound", "measured")

    def __init__(self, base, graph_gpu_ms, mode):
        if mode not in self.MODES:
            raise ValueError(f"resident graph cost mode must be one of {self.MODES}")
        if not graph_gpu_ms > 0:
            raise ValueError("a calibrated resident launch must take positive time")
        self.base, self.graph_gpu_ms, self.mode = base, float(graph_gpu_ms), mode
        self.sources = list(getattr(base, "sources", []))

    def for_load(self, n):
        row = self.base.for_load(n)
        if n != 1 or self.mode == "eager_bound":
            return row
        staged_total = row["h2d_ms"] + row["gpu_ms"]
        return dict(row, gpu_ms=self.graph_gpu_ms, h2d_ms=max(1e-6, staged_total - self.graph_gpu_ms))


def mi355x_costs():
    """The cost table measured on MI355X (costs/mi355x_cost_table.json)."""
    return FileCosts(COSTS_DIR / "mi355x_cost_table.json")
