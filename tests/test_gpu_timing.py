"""StepTimer: the per-token timing record of the reference's result files."""
import pytest
import torch

from wnw_amd.kv.timing import StepTimer

pytestmark = pytest.mark.gpu


def test_step_timer_records_prefill_and_decode_steps():
    dev = torch.device("cuda", 0)
    x = torch.randn(1 << 20, device=dev)
    timer = StepTimer(dev)
    assert timer.result() == {"prefill": None, "decode": []}
    waits = [0.02, 0.005, 0.01]  # "prefill", then two decode steps
    for w in waits:
        torch.cuda._sleep(int(w * 2e9))  # ~w seconds of device time at ~2 GHz (spin kernel)
        x.mul_(1.0)
        assert timer(None, None) is False  # never stops generation
    r = timer.result()
    assert set(r) == {"prefill", "decode"} and len(r["decode"]) == 2
    assert all(isinstance(v, float) and v > 0 for v in [r["prefill"], *r["decode"]])
    assert r["prefill"] > r["decode"][0]  # 20 ms of spin vs 5 ms


def test_step_timer_is_a_stopping_criterion():
    transformers = pytest.importorskip("transformers")
    assert isinstance(StepTimer(torch.device("cuda", 0)), transformers.StoppingCriteria)
