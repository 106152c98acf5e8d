"""The offload channel's groups of layers (WnWCache._group_layers): every
layer in exactly one group, groups in layer order, at most the configured
number of groups, and the first and last groups (the rows needed first, the
layers run after the last copy) no larger than any group between them."""
import pytest

from wnw_amd.wnw.cache import WnWCache


class _Cache:
    def __init__(self, layers, groups):
        self.num_layers = layers
        self._load_groups = groups


@pytest.mark.parametrize("layers", [1, 2, 3, 4, 5, 7, 8, 12, 28, 30, 32, 61, 64, 80])
@pytest.mark.parametrize("groups", [1, 2, 3, 6, 8])
def test_groups_partition_the_layers(layers, groups):
    g = WnWCache._group_layers(_Cache(layers, groups))
    assert g[0][0] == 0 and g[-1][1] == layers
    assert all(a < b for a, b in g)
    assert all(g[i][1] == g[i + 1][0] for i in range(len(g) - 1))
    assert len(g) <= max(1, min(groups, layers))
    if len(g) > 2:
        inner = min(b - a for a, b in g[1:-1])
        assert g[0][1] - g[0][0] <= inner and g[-1][1] - g[-1][0] <= inner
