"""The oracle reproduces every committed golden fixture (CPU). The GPU side of the same fixtures
is in test_gpu_scan.py."""
import pytest
import torch

from oracle.ssm_ref import selective_scan_ref
from tests import fixtures


@pytest.mark.parametrize("name", fixtures.names())
def test_oracle_reproduces_fixture(name):
    inputs, exp = fixtures.load(name)
    out, last = selective_scan_ref(**inputs, return_last_state=True)
    assert out.dtype == exp["out"].dtype
    torch.testing.assert_close(out.float(), exp["out"].float(), rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(last, exp["last_state"], rtol=1e-6, atol=1e-6)


def test_fixture_set_covers_edge_cases():
    n = set(fixtures.names())
    assert "cfg0" in n
    for needle in ("L1", "ragged", "chunk", "G2", "constBC", "noD", "N64"):
        assert any(needle in x for x in n), needle
