"""The measurement probes behind the bench's floors (fracture_amd/csrc/probes.hip) move the bytes
they stand for: every output byte is the XOR of the inputs' bytes at the same offset, over
sizes and grids that exercise the grid-stride loop, its 4-way unroll and a partial last step,
and bytes past the stated size are left alone. A read-only probe leaves its sink untouched
(the XOR of random inputs never equals the sentinel pattern)."""
import numpy as np
import pytest
import torch

from fracture_amd import kernels as K

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nin,nout", [(1, 1), (2, 1), (3, 2), (0, 1), (2, 2)])
@pytest.mark.parametrize("nbytes,grid", [(16, 1), (4096 * 16 + 48, 3), (1 << 20, 64),
                                         (3 * (1 << 20) + 16 * 777, 1024)])
def test_probe_stream_moves_its_bytes(dev, nin, nout, nbytes, grid):
    g = torch.Generator(device=dev)
    g.manual_seed(nbytes + grid)
    pad = 256
    ins = [torch.randint(0, 256, (nbytes + pad,), generator=g, device=dev, dtype=torch.uint8)
           for _ in range(nin)]
    outs = [torch.full((nbytes + pad,), 0x5A, dtype=torch.uint8, device=dev) for _ in range(nout)]
    K.probe_stream(ins, outs, nbytes, grid)
    torch.cuda.synchronize()
    want = np.zeros(nbytes, np.uint8)
    for t in ins:
        want ^= t.cpu().numpy()[:nbytes]
    for o in outs:
        got = o.cpu().numpy()
        assert np.array_equal(got[:nbytes], want)
        assert (got[nbytes:] == 0x5A).all()


def test_probe_stream_read_only_keeps_sink(dev):
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    nbytes = 1 << 20
    ins = [torch.randint(0, 256, (nbytes,), generator=g, device=dev, dtype=torch.uint8)
           for _ in range(2)]
    sink = torch.full((256,), 7, dtype=torch.int32, device=dev)
    K.probe_stream(ins, [], nbytes, 128, sink=sink)
    torch.cuda.synchronize()
    assert (sink.cpu().numpy() == 7).all()


def test_probe_empty_runs(dev):
    for grid in (1, 256, 65536):
        K.probe_empty(grid)
    torch.cuda.synchronize()
