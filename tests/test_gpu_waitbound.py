"""The bounded waits of the two cooperative single-pass kernels, forced to give up from
the host (zx_set_wait_bound_us(0)): every wave still exits, the call returns, the error
word carries ZX_KERR_SPIN and the drop-in classes raise (PagedFP8KVCache also undoes a
checked append).  After the default bound is restored, the same calls are bit-exact
against the oracle again, so an aborted launch leaves nothing behind in the workspace.
No kernel is made to fault or hang: a zero bound only makes the first wait without
progress take the release path."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from zenyx_amd import _native as N
from zenyx_amd import kv
from zenyx_amd.train.fp8_kv_quantization import FP8KVQuantizer, PagedFP8KVCache

pytestmark = pytest.mark.gpu


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.fixture
def zero_wait_bound(dev):
    kv.set_wait_bound_us(0)
    try:
        yield
    finally:
        kv.set_wait_bound_us(None)


def _append_case(dev, seed=3):
    L, H, D, P = 2, 8, 128, 16
    lens = [700, 333, 1201]  # ~2.2k tokens: the single-pass kernel's range
    nb = [(n + P - 1) // P for n in lens]
    g = torch.Generator().manual_seed(seed)
    n_pages = sum(nb) + 3
    perm = torch.randperm(n_pages, generator=g).to(torch.int32)
    bt = torch.full((len(lens), max(nb)), -1, dtype=torch.int32)
    k = 0
    for b, n in enumerate(nb):
        bt[b, :n] = perm[k:k + n]
        k += n
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    x = torch.randn((L, sum(lens), 2, H, D), generator=g).to(torch.bfloat16)
    return x, cu, bt, (L, n_pages, 2, H, P, D)


def test_fused_append_wait_gives_up_then_recovers(dev, zero_wait_bound):
    x, cu, bt, pshape = _append_case(dev)
    pool = torch.zeros(pshape, dtype=torch.uint8, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    kv.kv_quant_append(x.to(dev), cu.to(dev), bt.to(dev), pool, err=err, single_pass=True)
    torch.cuda.synchronize()
    assert int(err.item()) & N.ZX_KERR_SPIN, "a zero wait bound must make the single pass give up"
    with pytest.raises(ValueError, match="wait"):
        kv.kv_quant_append(x.to(dev), cu.to(dev), bt.to(dev), pool, check=True, single_pass=True)
    kv.set_wait_bound_us(None)
    want = np.zeros(pshape, np.uint8)
    wsc, werr = O.kv_quant_append(bits16(x), cu.numpy(), None, bt.numpy(), want, pshape[4])
    assert werr == 0
    pool.zero_()
    sc = kv.kv_quant_append(x.to(dev), cu.to(dev), bt.to(dev), pool, check=True, single_pass=True)
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), wsc.view(np.uint32))
    np.testing.assert_array_equal(pool.cpu().numpy(), want)


def test_single_pass_quantiser_wait_gives_up_then_recovers(dev, zero_wait_bound):
    g = torch.Generator().manual_seed(5)
    x = torch.randn((3, 2, 4, 8192), generator=g).to(torch.bfloat16)
    xd = x.to(dev)
    with pytest.raises(ValueError, match="wait"):
        kv.fp8_quant_heads(xd, single_pass=True, check=True)
    kv.set_wait_bound_us(None)
    codes, scales = kv.fp8_quant_heads(xd, single_pass=True, check=True)
    wc, ws = O.fp8_quant_heads(bits16(x).reshape(3, 2, 4, 8192))
    np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint32), ws.view(np.uint32))
    np.testing.assert_array_equal(codes.cpu().numpy(), wc)


def test_quantizer_dropin_checks_its_single_pass(dev, zero_wait_bound):
    # 256 MiB of bf16: FP8KVQuantizer takes the single pass and checks it by default
    x = torch.ones((16, 2, 1, 8, 4096, 128), dtype=torch.bfloat16, device=dev)
    assert x.numel() * 2 >= kv.HEADS_SINGLE_PASS_BYTES
    q = FP8KVQuantizer(dev)
    with pytest.raises(ValueError, match="wait"):
        q.quantize(x)
    # a small input takes the two passes, which have no wait
    small = torch.randn((2, 2, 1, 4, 64, 64), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    codes, scales = q.quantize(small.to(dev))
    wc, ws = O.fp8_quant_heads(bits16(small).reshape(4, 1, 4, 64 * 64))
    np.testing.assert_array_equal(scales.cpu().numpy().reshape(-1).view(np.uint32), ws.reshape(-1).view(np.uint32))
    np.testing.assert_array_equal(codes.cpu().numpy().reshape(wc.shape), wc)
    del x
    torch.cuda.empty_cache()


def test_paged_cache_raises_and_rolls_back_an_aborted_append(dev, zero_wait_bound):
    x, cu, bt, pshape = _append_case(dev, seed=11)
    L, _, _, H, P, D = pshape
    lens = np.diff(cu.numpy()).tolist()
    cache = PagedFP8KVCache(L, H, D, num_pages=pshape[1] + 8, page_size=P, device=dev)
    free_before = list(cache._free)
    with pytest.raises(ValueError, match="wait"):
        cache.append(x, ["a", "b", "c"], lens, check=True, single_pass=True)
    assert cache.lengths == {} and cache.pages == {} and sorted(cache._free) == sorted(free_before)
    assert not cache.has_scales
    # unchecked: the error surfaces at the next check
    cache.append(x, ["a", "b", "c"], lens, single_pass=True)
    with pytest.raises(ValueError, match="wait"):
        cache.check_errors()
    cache.check_errors()  # the words were cleared by the raise
    for s in ("a", "b", "c"):
        cache.free(s)
    kv.set_wait_bound_us(None)
    cache.append(x, ["a", "b", "c"], lens, dynamic_scales=True, check=True, single_pass=True)
    tables = cache._tables(["a", "b", "c"]).cpu().numpy()
    want = np.zeros(tuple(cache.pool.shape), np.uint8)
    wsc, werr = O.kv_quant_append(bits16(x), cu.numpy(), None, tables, want, P)
    assert werr == 0
    np.testing.assert_array_equal(cache.scales.cpu().numpy().view(np.uint32), wsc.view(np.uint32))
    np.testing.assert_array_equal(cache.pool.cpu().numpy(), want)
