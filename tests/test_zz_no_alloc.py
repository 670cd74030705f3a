"""The no-allocation sort entry point (zmoe_flatten_sort_count_noalloc) against the
workspace entry point (zmoe_flatten_sort_count), through the C ABI: bit-identical
sorted ids, slot ids, offsets, inverse permutation and out-of-range flag, on two calls
in a row (the second smaller, so it runs over the first call's leftover scratch). The
rejection of sizes above the scratch maximum is a host-only check in tests/test_capi.py."""

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu


def _sort_both(idx: torch.Tensor, E: int):
    from zmoe import _lib as L

    dev = idx.device
    flat = idx.reshape(-1).to(torch.int64).contiguous()
    R = flat.numel()
    stream = torch.cuda.current_stream(dev).cuda_stream

    def outs():
        return (torch.full((R,), -7, dtype=torch.int64, device=dev), torch.full((R,), -7, dtype=torch.int64, device=dev),
                torch.full((E,), -7, dtype=torch.int64, device=dev), torch.full((R,), -7, dtype=torch.int32, device=dev),
                torch.full((1,), -7, dtype=torch.int32, device=dev))

    a = outs()
    nbytes = L.load().zmoe_sort_workspace_bytes(R, E)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    L.call("zmoe_flatten_sort_count", flat.data_ptr(), R, E, a[0].data_ptr(), a[1].data_ptr(), a[2].data_ptr(),
           a[3].data_ptr(), ws.data_ptr(), nbytes, stream)
    a[4].copy_(ws[:4].view(torch.int32))
    b = outs()
    L.call("zmoe_flatten_sort_count_noalloc", flat.data_ptr(), R, E, b[0].data_ptr(), b[1].data_ptr(),
           b[2].data_ptr(), b[3].data_ptr(), b[4].data_ptr(), stream)
    torch.cuda.synchronize()
    return a, b


def _check(idx, E, expect_flag):
    a, b = _sort_both(idx, E)
    for name, x, y in zip(("sorted_expert_idxs", "sorted_scattered_idxs", "expert_offsets", "inverse", "flag"), a, b):
        assert torch.equal(x, y), name
    assert int(b[4]) == expect_flag
    if not expect_flag:  # and both equal the oracle's stable sort
        rse, rss, roff = O.flatten_sort_count(idx.cpu().numpy(), E)
        np.testing.assert_array_equal(b[0].cpu().numpy(), rse)
        np.testing.assert_array_equal(b[1].cpu().numpy(), rss)
        np.testing.assert_array_equal(b[2].cpu().numpy(), roff)


def test_noalloc_sort_matches_workspace_entry_point(hip_device):
    g = torch.Generator()
    g.manual_seed(3)
    # C3's routing size first, then a smaller one with more experts over the same scratch
    big = torch.argsort(torch.rand(32768, 128, generator=g), dim=1)[:, :8].contiguous().to(hip_device)
    _check(big, 128, 0)
    small = torch.argsort(torch.rand(1000, 300, generator=g), dim=1)[:, :6].contiguous().to(hip_device)
    _check(small, 300, 0)
    # an out-of-range id raises the flag in both (valid slots still sorted first)
    bad = small.clone()
    bad[17, 2] = 300
    _check(bad, 300, 1)
    # and an empty input
    _check(torch.empty(0, 4, dtype=torch.int64, device=hip_device), 16, 0)
