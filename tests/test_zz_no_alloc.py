"""mm_nl_scan_noalloc (the allocation-free receiver-CSR scan) against mm_nl_scan through the C ABI (marked gpu).

Integer output: bit-exact.  Two calls in a row on the shared static scratch, the second with a smaller input, and
the tile boundaries (4096 counts per tile) and the limits (N = 0, the largest accepted N is not allocated here; one
past the limit is rejected on the host before any launch)."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

TILE = 4096
MAX_ITEMS = 32768 * TILE


def _scan_with_workspace(NN):
    from mace_onegpu._lib import K, stream
    N = NN.numel()
    nbytes = ctypes.c_size_t(0)
    K.mm_nl_workspace_bytes(N + 1, ctypes.byref(nbytes))
    ws = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device="cuda")
    out = torch.full((N + 1,), -7, dtype=torch.int64, device="cuda")
    K.mm_nl_scan(NN, out, N, ws, ws.numel(), stream())
    return out


def _scan_noalloc(NN):
    from mace_onegpu._lib import K, stream
    N = NN.numel()
    out = torch.full((N + 1,), -7, dtype=torch.int64, device="cuda")
    K.mm_nl_scan_noalloc(NN, out, N, stream())
    return out


@pytest.mark.parametrize("sizes", [(3_000_001, 70_000), (TILE * 40, TILE - 1), (TILE, TILE + 1, 1, 0)])
def test_noalloc_scan_matches_workspace_scan(sizes):
    assert torch.cuda.is_available(), "GPU test without a GPU"
    g = torch.Generator().manual_seed(sum(sizes))
    for call, N in enumerate(sizes):
        print(f"case noalloc scan call {call}: N={N}", flush=True)
        NN = torch.randint(0, 250, (N,), generator=g, dtype=torch.int32).cuda()
        a = _scan_noalloc(NN)
        b = _scan_with_workspace(NN)
        torch.cuda.synchronize()
        assert torch.equal(a, b)
        assert int(a[0]) == 0 and int(a[-1]) == int(NN.long().sum())


def test_noalloc_scan_rejects_sizes_beyond_its_scratch():
    from mace_onegpu._lib import K, stream
    assert torch.cuda.is_available(), "GPU test without a GPU"
    dummy_in = torch.zeros(1, dtype=torch.int32, device="cuda")
    dummy_out = torch.full((1,), -7, dtype=torch.int64, device="cuda")
    print(f"case noalloc scan limit: N={MAX_ITEMS}", flush=True)
    with pytest.raises(RuntimeError, match="exceeds the scratch limit"):
        K.mm_nl_scan_noalloc(dummy_in, dummy_out, MAX_ITEMS, stream())     # N + 1 > limit: refused on the host
    torch.cuda.synchronize()
    assert int(dummy_out[0]) == -7
