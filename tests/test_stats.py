"""InferenceStats: the per-sample ``stats`` record (CPU only)."""
import torch

from wnw_amd.kv.stats import GPUMonitor, InferenceStats


def _snap(step=-1):
    return [{"step": step, "gpu_total_tokens": 10 + step}, {"step": step, "gpu_total_tokens": 20 + step}]


def test_record_flow_and_events():
    st = InferenceStats(torch.device("cpu"), interval=2)
    st.reset(2)
    st.record_prefill_before(_snap)
    st.record_prefill_before(lambda step=-1: [{"late": True}] * 2)  # only the first counts
    st.record_cpu_gpu_transfer(0, g2c_tokens=5, g2c_bytes=50)
    st.record_prefill(_snap)  # flushes the prefill transfers as step -1
    for step in range(1, 5):
        if step == 3:
            st.record_cpu_gpu_transfer(1, c2g_tokens=2, c2g_bytes=8)
            st.record_cpu_gpu_transfer(1, c2g_tokens=1, c2g_bytes=4)
        st.flush_decode_step(step)
        if step % st.interval == 0:
            st.record_decode(step, _snap)
    out = st.get_all_stats()
    assert len(out) == 2
    assert out[0]["prefill_before"]["gpu_total_tokens"] == 9 and "late" not in out[0]["prefill_before"]
    assert out[0]["cpu_gpu_events"] == [(-1, 0, 5, 0, 50)]
    assert out[1]["cpu_gpu_events"] == [(3, 3, 0, 12, 0)]  # (step, c2g_t, g2c_t, c2g_b, g2c_b)
    assert [s["step"] for s in out[1]["decode_snapshots"]] == [2, 4]
    assert out[1]["decode_final"]["gpu_total_tokens"] == 24
    # snapshots carry the device-memory fields
    assert {"gpu_index", "memory_total_bytes", "memory_free_bytes", "memory_used_bytes"} <= set(out[0]["prefill"])


def test_disabled_records_nothing():
    st = InferenceStats(torch.device("cpu"), interval=0)
    st.reset(1)
    st.record_prefill(_snap)
    st.record_cpu_gpu_transfer(0, c2g_tokens=3)
    st.flush_decode_step(1)
    st.record_decode(1, _snap)
    assert st.get_all_stats() == [{"prefill_before": {}, "prefill": {}, "decode_snapshots": [], "decode_final": {},
                                   "cpu_gpu_events": []}]


def test_final_falls_back_to_prefill():
    st = InferenceStats(None, interval=5)
    st.reset(1)
    st.record_prefill(_snap)
    assert st.get_all_stats()[0]["decode_final"]["gpu_total_tokens"] == 9


def test_gpu_monitor_without_device_reports_none():
    if torch.cuda.is_available():
        snap = GPUMonitor(0).snapshot()
        assert snap["memory_used_bytes"] == snap["memory_total_bytes"] - snap["memory_free_bytes"]
    else:
        assert GPUMonitor(0).snapshot() == {"gpu_index": 0, "memory_total_bytes": None, "memory_free_bytes": None,
                                            "memory_used_bytes": None}
