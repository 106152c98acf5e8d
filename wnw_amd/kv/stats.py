"""Per-sample runtime statistics of the cache (the ``stats`` record).

Same interface and output as the reference's ``InferenceStats``
(src/common/monitoring/inference_stats.py:11-137) and ``GPUMonitor``
(src/common/monitoring/gpu_monitor.py), whose schema is documented in the
reference's docs/data_format.md ("Runtime stats Schema"):

* ``get_all_stats()`` returns, per sample, ``prefill_before``, ``prefill``
  (cache snapshot merged with a device-memory snapshot), ``decode_snapshots``
  (every ``interval`` decode steps), ``decode_final`` (last snapshot, else
  the prefill one) and ``cpu_gpu_events``: per-step tuples ``(step,
  c2g_tokens, g2c_tokens, c2g_bytes, g2c_bytes)`` of steps with traffic.
* ``interval`` 0 disables collection; the default is every 5 steps.
* Transfers recorded during prefill are flushed as step -1.
"""
from __future__ import annotations

from collections import defaultdict
from collections.abc import Callable

import torch


class GPUMonitor:
    """Device-memory snapshot of one GPU (None values when unavailable)."""

    def __init__(self, gpu_index: int):
        self.gpu_index = gpu_index

    def snapshot(self) -> dict:
        try:
            free, total = torch.cuda.mem_get_info(self.gpu_index)
        except Exception:  # no device, wrong index: the reference reports None
            return {"gpu_index": self.gpu_index, "memory_total_bytes": None, "memory_free_bytes": None,
                    "memory_used_bytes": None}
        return {"gpu_index": self.gpu_index, "memory_total_bytes": int(total), "memory_free_bytes": int(free),
                "memory_used_bytes": int(total - free)}


class InferenceStats:
    def __init__(self, device: torch.device | None = None, interval: int = 5):
        self.device = device
        index = device.index if device is not None and device.index is not None else 0
        self._gpu_monitor = GPUMonitor(index)
        self.set_interval(interval)
        self.reset(0)

    def set_interval(self, interval: int) -> None:
        """0 disables collection."""
        self.interval = interval
        self.enabled = interval > 0

    def reset(self, batch_size: int) -> None:
        self._batch_size = batch_size
        self._prefill_before: list[dict] = []
        self._prefill: list[dict] = []
        self._decode: list[list[dict]] = []
        self._events: dict[int, list[tuple]] = defaultdict(list)
        self._pending = defaultdict(lambda: [0, 0, 0, 0])  # b -> c2g_tokens, g2c_tokens, c2g_bytes, g2c_bytes
        self._prefill_before_done = False

    def _snapshot(self, cache_stats_fn: Callable[..., list[dict]], step: int) -> list[dict]:
        mem = self._gpu_monitor.snapshot()
        return [{**s, **mem} for s in cache_stats_fn(step=step)]

    def record_prefill_before(self, cache_stats_fn: Callable[..., list[dict]]) -> None:
        """Once per sample, before the first prefill layer."""
        if self.enabled and not self._prefill_before_done:
            self._prefill_before = self._snapshot(cache_stats_fn, -1)
            self._prefill_before_done = True

    def record_prefill(self, cache_stats_fn: Callable[..., list[dict]]) -> None:
        if self.enabled:
            self._prefill = self._snapshot(cache_stats_fn, -1)
            self.flush_decode_step(-1)

    def record_decode(self, step: int, cache_stats_fn: Callable[..., list[dict]]) -> None:
        if self.enabled:
            self._decode.append(self._snapshot(cache_stats_fn, step))

    def record_cpu_gpu_transfer(self, b: int, c2g_tokens: int = 0, g2c_tokens: int = 0, c2g_bytes: int = 0,
                                g2c_bytes: int = 0) -> None:
        if self.enabled:
            acc = self._pending[b]
            acc[0] += int(c2g_tokens)
            acc[1] += int(g2c_tokens)
            acc[2] += int(c2g_bytes)
            acc[3] += int(g2c_bytes)

    def flush_decode_step(self, step: int) -> None:
        """Turn this step's transfers into events (samples without traffic add none)."""
        if not self.enabled:
            return
        for b in sorted(self._pending):
            c2g_t, g2c_t, c2g_b, g2c_b = self._pending[b]
            if c2g_t or g2c_t or c2g_b or g2c_b:
                self._events[b].append((int(step), c2g_t, g2c_t, c2g_b, g2c_b))
        self._pending.clear()

    def get_all_stats(self) -> list[dict]:
        out = []
        for b in range(self._batch_size):
            before = self._prefill_before[b] if b < len(self._prefill_before) else {}
            prefill = self._prefill[b] if b < len(self._prefill) else {}
            snaps = [s[b] for s in self._decode if b < len(s)]
            out.append({"prefill_before": before, "prefill": prefill, "decode_snapshots": snaps,
                        "decode_final": snaps[-1] if snaps else prefill,
                        "cpu_gpu_events": list(self._events.get(b, []))})
        return out
