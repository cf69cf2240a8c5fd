"""The measurement probes (sltx_probe_*, q4_probe.hip) on the GPU: each
grid hand-off mode completes its rounds with no wait running out, the MFMA
loop's sums are what its register operands give, and a grid larger than the
device holds at once is refused before launch."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("fence", [0, 1])
def test_probe_sync_completes(pkg, dev, mode, fence):
    import torch
    for blocks in (1, 7, 64, 256):
        sync = torch.zeros(pkg.probe_sync_words(blocks), dtype=torch.int32, device=dev)
        faults = torch.zeros(1, dtype=torch.int32, device=dev)
        pkg.probe_sync(mode, fence, blocks, 25, sync, faults)
        torch.cuda.synchronize()
        assert int(faults.item()) == 0, (mode, fence, blocks)
        s = sync.cpu().numpy().view(np.uint32)
        if mode == 0:
            assert s[0] == 25 * blocks
        elif mode in (1, 3):
            assert s[0] == 25 * min(blocks, 8)
            if mode == 3:
                assert np.all(s[16 * 9:16 * 9 + 16 * blocks] == 25)
        else:
            assert np.all(s[16 * 9:16 * 9 + blocks] == 25)


def test_probe_sync_refuses_more_blocks_than_resident(pkg, dev):
    import torch
    blocks = 1 << 20
    sync = torch.zeros(pkg.probe_sync_words(blocks), dtype=torch.int32, device=dev)
    faults = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(pkg.SltxError, match="hold"):
        pkg.probe_sync(0, 0, blocks, 1, sync, faults)


def test_probe_mfma_sums(pkg, dev):
    """With ab = 1/16 everywhere each 32x32x16 product adds 16 / 256 to every
    accumulator element: after `iters` rounds each lane's 64 elements sum to
    64 * iters / 16."""
    import torch
    ab = torch.full((256, 8), 1.0 / 16, dtype=torch.float16, device=dev)
    blocks, iters = 4, 32
    sink = torch.empty(blocks * 256, device=dev)
    clocks = torch.zeros(blocks, 2, dtype=torch.int64, device=dev)
    pkg.probe_mfma(ab, blocks, iters, sink, clocks)
    pkg.probe_empty()
    torch.cuda.synchronize()
    assert torch.allclose(sink, torch.full_like(sink, 64 * iters / 16))
    c = clocks.cpu().numpy()
    assert np.all(c[:, 0] > 0) and np.all(c[:, 1] > 0)
