"""The PyTorch CPU restatement timed as bench.py's CPU baseline
(``oracle/torch_cpu.py``) against the float64 C oracle: the append is
byte-exact, the attention within the bf16 tolerance of the decode path.
Config-1 shape (B = 2, 8 KV heads, G = 4, D = 128; class A 1024 rows, class
B 128), plus empty and one-row segments."""
import numpy as np
import torch

import oracle
from oracle import torch_cpu
from tests.helpers import allclose_report, cu_from_lens, rand_rows


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_append_and_attention_match_oracle():
    rng = np.random.default_rng(3)
    lens = [1024 if h < 2 else 128 for _ in range(2) for h in range(8)]
    lens[5], lens[9] = 0, 1
    n, G, D = len(lens), 4, 128
    cu = cu_from_lens(lens)
    k, v = rand_rows(rng, int(cu[-1]), D, "bfloat16"), rand_rows(rng, int(cu[-1]), D, "bfloat16")
    nk, nv = rand_rows(rng, n, D, "bfloat16"), rand_rows(rng, n, D, "bfloat16")
    q = rand_rows(rng, n * G, D, "bfloat16").reshape(n, G, D)
    cu_new = cu + np.arange(n + 1, dtype=np.int32)
    k2 = torch_cpu.append_by_cat(_bf16(k), _bf16(nk), cu.tolist())
    v2 = torch_cpu.append_by_cat(_bf16(v), _bf16(nv), cu.tolist())
    np.testing.assert_array_equal(_bits(k2), oracle.interleave_append(k, nk, cu, cu_new, dtype=oracle.DT_BF16))
    np.testing.assert_array_equal(_bits(v2), oracle.interleave_append(v, nv, cu, cu_new, dtype=oracle.DT_BF16))
    scale = D ** -0.5
    out = torch_cpu.decode_attn(_bf16(q), k2, v2, cu_new.tolist(), scale)
    ref = oracle.decode_attn(q, _bits(k2), _bits(v2), cu_new, scale, dtype=oracle.DT_BF16)
    ok, msg = allclose_report(oracle.to_f64(_bits(out), oracle.DT_BF16), ref, 2e-3, 1e-2)
    assert ok, msg
    # the one-row segment (after the append: two rows) and an appended-to-empty one
    # (one row: the new row itself, so the output is that V row exactly)
    np.testing.assert_array_equal(_bits(out[5]), np.tile(nv[5], (G, 1)))
