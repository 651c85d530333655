"""The bench's achievable-HBM probes: the read probe
(qxh_encode_hbm_read_probe) reads the buffer without writing the sink for
real data and rejects sizes that are not whole 16-byte words; the copy probe
(qxh_encode_hbm_copy_probe) copies every byte, both store kinds, and rejects
sizes that are not whole 4 KB rows and overlapping buffers."""
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


@pytest.mark.parametrize("nontemporal", [True, False])
def test_copy_probe_copies_every_byte_and_validates(nontemporal):
    ctx = rt.Context(0)
    n = 4096 * 37  # rows not a multiple of the four rows of a workgroup
    src = torch.randint(-2**31, 2**31 - 1, (n // 4,), dtype=torch.int32, device="cuda:0")
    dst = torch.zeros(n // 4 + 1024, dtype=torch.int32, device="cuda:0")
    with rt.Graph(ctx) as g:
        rt.hbm_copy_probe(g, src, dst, nontemporal)
    assert torch.equal(dst[:n // 4], src)
    assert torch.all(dst[n // 4:] == 0)  # nothing past the copied bytes
    with rt.Graph(ctx) as g:
        with pytest.raises(abi.QxhError, match="multiple of 4096"):
            rt.hbm_copy_probe(g, src[:100], dst, nontemporal)
        with pytest.raises(abi.QxhError, match="overlap"):
            rt.hbm_copy_probe(g, dst[:1024], dst[512:], nontemporal)
