"""Per-sample runtime counters of the cache.

Keeps the method names the reference's cache calls on its
``InferenceStats`` (src/common/monitoring/inference_stats.py, used from
src/algorithms/wnw/code/cache.py) so a cache written against it runs
unchanged; it records host<->device transfer volumes and the cache
snapshots the cache hands in.
"""
from __future__ import annotations


class InferenceStats:
    def __init__(self, device=None, interval: int = 5):
        self.device = device
        self.interval = interval
        self.enabled = False
        self.reset(0)

    def set_interval(self, interval: int) -> None:
        self.interval = interval
        self.enabled = True

    def reset(self, batch_size: int) -> None:
        self.batch_size = batch_size
        self.transfers = [dict(c2g_tokens=0, c2g_bytes=0, g2c_tokens=0, g2c_bytes=0) for _ in range(batch_size)]
        self.snapshots: list[tuple[str, int, list[dict]]] = []
        self.decode_steps = 0

    def record_cpu_gpu_transfer(self, b: int, c2g_tokens: int = 0, c2g_bytes: int = 0, g2c_tokens: int = 0,
                                g2c_bytes: int = 0) -> None:
        if 0 <= b < len(self.transfers):
            t = self.transfers[b]
            t["c2g_tokens"] += c2g_tokens
            t["c2g_bytes"] += c2g_bytes
            t["g2c_tokens"] += g2c_tokens
            t["g2c_bytes"] += g2c_bytes

    def record_prefill_before(self, snapshot_fn) -> None:
        pass  # the snapshot before prefill holds nothing yet

    def record_prefill(self, snapshot_fn) -> None:
        if self.enabled:
            self.snapshots.append(("prefill", 0, snapshot_fn()))

    def flush_decode_step(self, step: int) -> None:
        self.decode_steps = step

    def record_decode(self, step: int, snapshot_fn) -> None:
        self.snapshots.append(("decode", step, snapshot_fn(step)))

    def get_all_stats(self) -> list[dict]:
        out = []
        for b in range(self.batch_size):
            snaps = [(kind, step, s[b]) for kind, step, s in self.snapshots if b < len(s)]
            out.append({"transfers": dict(self.transfers[b]), "decode_steps": self.decode_steps,
                        "snapshots": snaps})
        return out
