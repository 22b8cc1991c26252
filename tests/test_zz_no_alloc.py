"""r9k_moe_align_noalloc, the entry point that allocates nothing (its scratch is the library's fixed device array),
against r9k_moe_align with caller scratch, through the C-ABI: two calls in a row, the second smaller, tables bit for
bit; plus the refusal of a step larger than the array."""
import numpy as np
import pytest
import torch

from helpers import check_tables
from r9700_vllm.kernels import moe as K

pytestmark = pytest.mark.gpu


def _ids(T, E, topk, seed, dev):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16).to(dev)
    return K.moe_topk(logits, topk, True)[1]


def _tables(fn, ids, blk, E):
    sid, eid, ntpp = fn(ids, blk, E)
    torch.cuda.synchronize()
    n = int(ntpp.item())
    return sid[:n].cpu().numpy(), eid[: n // blk].cpu().numpy(), n


@pytest.mark.parametrize("E,topk,blk,Ts", [(288, 8, 256, (8192, 1024)), (384, 8, 16, (4096, 700)),
                                           (1024, 16, 64, (3000, 300)), (128, 8, 16, (600, 3))])
def test_align_noalloc_equals_align(dev, E, topk, blk, Ts):
    L = K.lib()
    assert L.r9k_moe_align_noalloc_max_ints() == 1 << 18
    for i, T in enumerate(Ts):                      # second call smaller: the shared array keeps the first's data
        ids = _ids(T, E, topk, 20261201 + 11000 + E + T, dev)
        numel = T * topk
        print(f"noalloc align E={E} k={topk} blk={blk} T={T} numel={numel} call {i + 1}", flush=True)
        a = _tables(K.moe_align, ids, blk, E)
        b = _tables(K.moe_align_noalloc, ids, blk, E)
        assert a[2] == b[2] and np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
        check_tables(b[0], b[1], np.array([b[2]]), ids.cpu().numpy(), blk, numel, E)


def test_align_noalloc_refuses_oversize(dev):
    """The array holds 16 + 255 chunk histograms of E = 1024: 255 * 2048 routed rows are served (tables as
    r9k_moe_align's), one more row needs a 256th chunk and is refused before any launch."""
    L = K.lib()
    E, numel = 1024, 255 * 2048
    assert L.r9k_moe_align_scratch_ints(numel, E) == 16 + 255 * 1024 <= L.r9k_moe_align_noalloc_max_ints()
    assert L.r9k_moe_align_scratch_ints(numel + 1, E) == 16 + 256 * 1024 > L.r9k_moe_align_noalloc_max_ints()
    ids = torch.randint(0, E, (numel + 1,), generator=torch.Generator().manual_seed(7), dtype=torch.int32).to(dev)
    a = _tables(K.moe_align, ids[:numel], 256, E)
    b = _tables(K.moe_align_noalloc, ids[:numel], 256, E)
    assert a[2] == b[2] and np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    with pytest.raises(RuntimeError, match="scratch ints"):
        K.moe_align_noalloc(ids, 256, E)
    assert L.r9k_moe_align_noalloc(ids.data_ptr(), numel + 1, E, 256, 0, 0, 0, 0) == -9   # refused before any launch
