"""Per-token wall time of a ``generate`` call, measured on the device.

Same interface and output as the reference's ``StepTimer``
(src/benchmarks/scripts/_timing.py:8-29), the ``timing`` record of its
result files (src/benchmarks/scripts/eval_wnw.py:110-117, 136): an HF
stopping criterion that never stops generation and records a device event
each time it is consulted (once per generated token).  ``result()``
synchronises once and returns the prefill time (construction to the first
token) and the time of every later decode step, in seconds, rounded to
0.1 ms.  Events go to the current stream, so the figures include every
kernel launched between two tokens, not the host's launch latency.
"""
from __future__ import annotations

import torch

try:  # transformers is the caller's dependency, as in the reference
    from transformers import StoppingCriteria as _Criterion
except ImportError:  # pragma: no cover - the class also works standalone
    _Criterion = object


class StepTimer(_Criterion):
    def __init__(self, device: torch.device | str | None = None):
        self.device = device
        self._marks: list[torch.cuda.Event] = [self._mark()]

    @staticmethod
    def _mark() -> torch.cuda.Event:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        return ev

    def __call__(self, input_ids, scores, **kwargs) -> bool:
        self._marks.append(self._mark())
        return False

    def result(self) -> dict:
        """{"prefill": seconds or None, "decode": [seconds per later token]}."""
        if len(self._marks) < 2:
            return {"prefill": None, "decode": []}
        torch.cuda.synchronize(self.device)
        secs = [a.elapsed_time(b) / 1000.0 for a, b in zip(self._marks, self._marks[1:])]
        return {"prefill": round(secs[0], 4), "decode": [round(x, 4) for x in secs[1:]]}
