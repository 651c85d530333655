"""The bench's achievable-HBM probe (qxh_encode_hbm_read_probe): it reads the
buffer without writing the sink for real data, and rejects sizes that are not
whole 16-byte words."""
import pytest
import torch

from qx_amd import abi
from qx_amd import runtime as rt

pytestmark = pytest.mark.gpu


def test_probe_reads_without_writing_and_validates():
    ctx = rt.Context(0)
    x = torch.ones(1 << 20, dtype=torch.float32, device="cuda:0")  # xor of equal words folds to 0
    sink = torch.full((64,), 7, dtype=torch.int32, device="cuda:0")
    with rt.Graph(ctx) as g:
        rt.hbm_read_probe(g, x, sink, 64)
    assert torch.all(sink == 7)
    with rt.Graph(ctx) as g:
        with pytest.raises(abi.QxhError, match="multiple of 16"):
            rt.hbm_read_probe(g, x[:3], sink, 64)
