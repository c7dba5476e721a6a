"""Measured per-expert cost tables for the placement planner (the FileCosts
format of benchmarks/pdscope_compare.py:55-85).

A table is JSON with kind "pdscope_cost_table" and ``points`` keyed by the
routed token count of one expert (1 .. 4096), each giving ``cpu_ms`` (the CPU
backend's time for that expert), ``gpu_ms`` (resident GPU compute) and
``h2d_ms`` (staging copy plus GPU compute).  ``for_load(n)`` returns the
point itself or a linear interpolation between the neighbouring points;
loads outside the measured domain are refused.  ``costs/mi355x_cost_table.json``
is the table measured on MI355X by ``bench.py --calibrate-costs``.
"""
from __future__ import annotations

import bisect
import hashlib
import json
from pathlib import Path

COSTS_DIR = Path(__file__).resolve().parent.parent / "costs"


class FileCosts:
    def __init__(self, path):
        path = Path(path)
        raw = path.read_bytes()
        payload = json.loads(raw)
        if payload.get("kind") != "pdscope_cost_table":
            raise ValueError("cost table file has an unexpected kind")
        self.points = {int(n): {k: float(v) for k, v in row.items()} for n, row in payload["points"].items()}
        self.loads = sorted(self.points)
        if not self.loads or self.loads[0] != 1 or self.loads[-1] != 4096:
            raise ValueError("cost table must cover the measured 1..4096 domain")
        self.sources = [dict(path=str(path.resolve()), sha256=hashlib.sha256(raw).hexdigest(),
                             kind="shipped_cost_table", platform=payload.get("platform"),
                             model=payload.get("model"), scope=payload.get("scope"))]

    def for_load(self, n):
        if not self.loads[0] <= n <= self.loads[-1]:
            raise ValueError("expert load outside the measured domain")
        if n in self.points:
            return dict(tokens=n, **self.points[n])
        hi = bisect.bisect_left(self.loads, n)
        a, b = self.loads[hi - 1], self.loads[hi]
        t = (n - a) / (b - a)
        return dict(tokens=n, **{k: self.points[a][k] + t * (self.points[b][k] - self.points[a][k])
                                 for k in self.points[a]})


def mi355x_costs():
    """The cost table measured on MI355X (costs/mi355x_cost_table.json)."""
    return FileCosts(COSTS_DIR / "mi355x_cost_table.json")
