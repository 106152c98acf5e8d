"""Host-side parts of the session (CPU): the prompt attention's float32
fallback, used when SDPA's fused backends do not take the inputs, against
SDPA itself (causal, additive float mask, boolean mask, query chunks that
do not divide the prompt)."""
import pytest
import torch
import torch.nn.functional as F

from wnw_amd.wnw import session


@pytest.mark.parametrize("mask", ["causal", "float", "bool"])
def test_prefill_attention_fallback_matches_sdpa(mask, monkeypatch):
    torch.manual_seed(0)
    q, k, v = (torch.randn(2, 4, 37, 16) for _ in range(3))
    m = None
    if mask == "float":
        m = torch.randn(2, 1, 37, 37)
    elif mask == "bool":
        m = torch.rand(2, 1, 37, 37) > 0.3
        m[..., 0] = True  # every row attends somewhere
    want = F.scaled_dot_product_attention(q, k, v, attn_mask=m, scale=0.3, is_causal=m is None)

    def no_fused_backend(*args, **kwargs):
        raise RuntimeError("no available kernel")

    monkeypatch.setattr(session.F, "scaled_dot_product_attention", no_fused_backend)
    got = session.prefill_attention(q, k, v, m, 0.3, q_chunk=10)
    torch.testing.assert_close(got, want, atol=2e-6, rtol=1e-5)
