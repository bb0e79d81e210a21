"""Helpers shared by the layers: scaling-factor validation and the section
profiler hook used around every sub-op (same contract as neuralop/utils.py
:154-200 and :232-366)."""
from __future__ import annotations

import contextvars
import time
from contextlib import contextmanager, nullcontext
from typing import List, Optional, Union

import torch

Number = Union[float, int]


def validate_scaling_factor(scaling_factor, n_dim: int, n_layers: Optional[int] = None):
    """None / number / list / list-of-lists -> per-dim (and per-layer) factors
    (neuralop/utils.py:154-200)."""
    if scaling_factor is None:
        return None
    if isinstance(scaling_factor, (float, int)):
        if n_layers is None:
            return [float(scaling_factor)] * n_dim
        return [[float(scaling_factor)] * n_dim] * n_layers
    if (isinstance(scaling_factor, list) and len(scaling_factor) > 0
            and all(isinstance(s, (float, int)) for s in scaling_factor)):
        if n_layers is None and len(scaling_factor) == n_dim:
            return [float(s) for s in scaling_factor]
        return [[float(s)] * n_dim for s in scaling_factor]
    if (isinstance(scaling_factor, list) and len(scaling_factor) > 0
            and all(isinstance(s, list) for s in scaling_factor)):
        s_sub_pass = True
        for s in scaling_factor:
            if not all(isinstance(s_sub, (int, float)) for s_sub in s):
                s_sub_pass = False
            if s_sub_pass:
                return scaling_factor
    return None


def count_model_params(model) -> int:
    """Parameter count with complex parameters counted twice (neuralop/utils.py:19-28)."""
    return sum(p.numel() * (2 if p.is_complex() else 1) for p in model.parameters())


_ACTIVE_PROFILER = contextvars.ContextVar("neuraloperator_amd_active_profiler", default=None)


class TimingProfiler:
    """Accumulates wall time per named section (GPU sections use events)."""

    def __init__(self):
        self._stats = {}

    def reset(self):
        self._stats = {}

    def record(self, name: str, duration_s: float):
        tot, cnt = self._stats.get(name, (0.0, 0))
        self._stats[name] = (tot + duration_s, cnt + 1)

    def section(self, name: str, device=None):
        return _TimingSection(self, name, device)

    def stats(self):
        return dict(self._stats)

    def summary(self, title: Optional[str] = None) -> str:
        total = sum(t for t, _ in self._stats.values()) or 1.0
        lines = [title] if title else []
        lines.append("section | total(s) | avg(ms) | pct | count")
        for name, (t, c) in sorted(self._stats.items(), key=lambda kv: -kv[1][0]):
            lines.append(f"{name} | {t:.4f} | {t / max(c, 1) * 1e3:.3f} | {100 * t / total:5.1f}% | {c}")
        return "\n".join(lines)


class _TimingSection:
    def __init__(self, prof, name, device):
        self.prof, self.name, self.device = prof, name, device

    def __enter__(self):
        if self.device is not None and getattr(self.device, "type", None) == "cuda":
            self.e0 = torch.cuda.Event(enable_timing=True)
            self.e1 = torch.cuda.Event(enable_timing=True)
            self.e0.record()
        else:
            self.e0 = None
            self.t0 = time.perf_counter()
        return self

    def __exit__(self, *exc):
        if self.e0 is not None:
            self.e1.record()
            self.e1.synchronize()
            self.prof.record(self.name, self.e0.elapsed_time(self.e1) / 1e3)
        else:
            self.prof.record(self.name, time.perf_counter() - self.t0)
        return False


@contextmanager
def profiling(profiler: TimingProfiler):
    token = _ACTIVE_PROFILER.set(profiler)
    try:
        yield profiler
    finally:
        _ACTIVE_PROFILER.reset(token)


def get_active_profiler() -> Optional[TimingProfiler]:
    return _ACTIVE_PROFILER.get()


def maybe_profile(profiler, name: str, device=None):
    return nullcontext() if profiler is None else profiler.section(name, device)
