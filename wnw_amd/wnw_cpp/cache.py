"""WnW cache variant with a deferred plan (the reference's ``wnw_cpp``).

Mirrors ``WnWCppCache`` (src/algorithms/wnw_cpp/code/cache.py:11-304):
``decode_all_layers_done`` only launches the chunk top-k on the device
(no host synchronisation at the end of the step); the next step's layer 0
reads it back, runs the native planner and starts the host->device copy of
the rows to load (``_finalize_pending_plan``).  The plans, and so the
layouts, are the ones ``WnWCache`` produces.  ``WNW_CPP_FALLBACK=1`` runs
the ``WnWCache`` flow instead (cache.py:14, :193-195).

Difference: with the out-of-place compaction fallback selected
(``WNW_DISABLE_TRITON_REBUILD=1``) a plan is still applied (through that
fallback); the reference computes the plan and then drops it
(wnw_cpp/code/cache.py:230-234), leaving its planner ahead of its layout.
"""
from __future__ import annotations

import os

from ..wnw.cache import WnWCache


class WnWCppCache(WnWCache):
    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        self._fallback = os.environ.get("WNW_CPP_FALLBACK", "0") == "1"
        self._record_plan_transfers = self._fallback  # the C++-planner flow counts no decode loads
        self._topk_pending = False
        self._topk_idx_masked = None

    def setup_audio(self, audio_starts, audio_ends, attention_mask=None):
        self._topk_pending = False
        self._topk_idx_masked = None
        super().setup_audio(audio_starts, audio_ends, attention_mask)

    def _before_decode_layer(self, layer_idx):
        """wnw_cpp/code/cache.py:197-224: the plan of the previous step's
        scores is finalised at layer 0, before its first rebuild."""
        if not self._fallback and layer_idx == 0 and self._topk_pending:
            self._finalize_pending_plan()

    def _finalize_pending_plan(self) -> None:
        """wnw_cpp/code/cache.py:226-241."""
        self._topk_pending = False
        topk, off = self._topk_finalize(self._topk_idx_masked)
        self._topk_idx_masked = None
        if self._plan(topk, off):
            self._pending_chunk_update = True
            self._prepare_pending_rebuild()
        else:
            self._pending_chunk_update = False

    def decode_all_layers_done(self):
        """wnw_cpp/code/cache.py:243-254."""
        if self._fallback:
            return super().decode_all_layers_done()
        self._flush_pending_scores()  # the step's last deferred class-A scores
        self._decode_step += 1
        self.stats.flush_decode_step(self._decode_step)
        if self.stats.enabled and self._decode_step % self.stats.interval == 0:
            self.stats.record_decode(self._decode_step, self._snapshot_cache_stats)
        self._topk_idx_masked = self._topk_scores_async()
        self._topk_pending = True
        self.score_accumulator.zero_()
