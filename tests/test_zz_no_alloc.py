"""zx_kv_quant_append_noalloc (the allocation-free variant of zx_kv_quant_append, for
callers that cannot allocate device memory) called through the C ABI: on two calls in a
row, the second smaller, its pool, scales and error word equal zx_kv_quant_append's on
the same inputs (the single-pass dynamic path, then the two-pass static path with an
overflow), bit for bit; a call needing more scratch than the library holds is refused
before anything runs."""
import pytest
import torch

from zenyx_amd import _native as N
from zenyx_amd import kv

pytestmark = pytest.mark.gpu


def _case(L, H, D, P, lens, seed, dev):
    g = torch.Generator().manual_seed(seed)
    nb = [(n + P - 1) // P for n in lens]
    n_pages = sum(nb) + 5
    perm = torch.randperm(n_pages, generator=g).to(torch.int32)
    bt = torch.full((len(lens), max(nb)), -1, dtype=torch.int32)
    k = 0
    for b, m in enumerate(nb):
        bt[b, :m] = perm[k:k + m]
        k += m
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    x = (torch.randn((L, sum(lens), 2, H, D), generator=g) * 3).to(torch.bfloat16)
    return x.to(dev), cu.to(dev), bt.to(dev), n_pages


def _noalloc(x, cu, bt, pool, scales, flags, err):
    L, T, _, H, D = x.shape
    n_pages, P = pool.shape[1], pool.shape[4]
    return N.load().zx_kv_quant_append_noalloc(
        N.ptr(x), T * 2 * H * D, L, T, H, D, N.ptr(cu), None, bt.shape[0], N.ptr(bt), bt.shape[1], P, N.ptr(pool),
        pool[0].numel(), n_pages, N.ptr(scales), flags, N.ptr(err), N.stream_ptr(x.device))


@pytest.mark.parametrize("static", [False, True])
def test_noalloc_append_equals_workspace_append(dev, static):
    L, H, D, P = 3, 8, 128, 16
    for call, lens in enumerate(([700, 33, 1500, 1], [40, 9])):  # the second call is smaller
        x, cu, bt, n_pages = _case(L, H, D, P, lens, seed=10 * call + static, dev=dev)
        pool_a = torch.zeros((L, n_pages, 2, H, P, D), dtype=torch.uint8, device=dev)
        pool_b = torch.full_like(pool_a, 0xAB)  # different old contents: pages outside the batch stay as they were
        pool_a.fill_(0xAB)
        if static:
            sc_a = torch.rand((L, 2, H), generator=torch.Generator().manual_seed(call)).to(dev) * 0.01 + 0.002
        else:
            sc_a = torch.empty((L, 2, H), dtype=torch.float32, device=dev)
        sc_b = sc_a.clone()
        err_a = torch.zeros(1, dtype=torch.int32, device=dev)
        err_b = torch.zeros(1, dtype=torch.int32, device=dev)
        # dynamic scales: the cooperative single pass, whose exchange slots live in the scratch
        kv.kv_quant_append(x, cu, bt, pool_a, scales=sc_a, static_scales=static, err=err_a, single_pass=not static)
        flags = N.ZX_APPEND_STATIC_SCALES if static else N.ZX_APPEND_SINGLE_PASS
        N.check(_noalloc(x, cu, bt, pool_b, sc_b, flags, err_b), "kv_quant_append_noalloc")
        torch.cuda.synchronize(dev)
        assert torch.equal(sc_a.view(torch.int32), sc_b.view(torch.int32)), f"call {call}: scales differ"
        assert torch.equal(pool_a, pool_b), f"call {call}: {(pool_a != pool_b).sum().item()} codes differ"
        assert int(err_a.item()) == int(err_b.item())
        if static:
            assert int(err_b.item()) == N.ZX_KERR_OVERFLOW  # scales of 0.002-0.012 under 3 x N(0,1) tokens


def test_noalloc_append_refuses_more_than_its_scratch(dev):
    x, cu, bt, n_pages = _case(1, 8, 128, 16, [20], seed=3, dev=dev)
    pool = torch.zeros((1, n_pages, 2, 8, 16, 128), dtype=torch.uint8, device=dev)
    sc = torch.empty((1, 2, 8), dtype=torch.float32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    lib = N.load()
    big = 2_000_000  # token offsets alone would need 16 MB
    assert lib.zx_kv_quant_append_workspace_bytes(1, big, 8, 128) > (8 << 20)
    rc = lib.zx_kv_quant_append_noalloc(
        N.ptr(x), big * 2 * 8 * 128, 1, big, 8, 128, N.ptr(cu), None, 1, N.ptr(bt), bt.shape[1], 16, N.ptr(pool),
        pool[0].numel(), n_pages, N.ptr(sc), 0, N.ptr(err), N.stream_ptr(dev))
    assert rc == N.ZX_ERR_WORKSPACE
    assert b"scratch" in lib.zx_last_error()
    torch.cuda.synchronize(dev)
    assert int(err.item()) == 0 and not pool.any()  # nothing ran


@pytest.mark.parametrize("mode", ["single_pass", "two_pass", "static"])
def test_noalloc_append_in_a_captured_graph(dev, mode):
    """The allocation-free append captured into a HIP graph (torch.cuda.CUDAGraph) after
    one eager call (which takes the scratch address and the occupancy figures), then
    replayed three times with eager work and synchronisations between the replays: each
    replay's pool, scales and error word equal zx_kv_quant_append's eager result bit for
    bit.  The cooperative single pass, the two passes and the static path all capture."""
    L, H, D, P = 3, 8, 128, 16
    x, cu, bt, n_pages = _case(L, H, D, P, [700, 33, 1500, 1], seed=5, dev=dev)
    static = mode == "static"
    flags = {"single_pass": N.ZX_APPEND_SINGLE_PASS, "two_pass": N.ZX_APPEND_TWO_PASS,
             "static": N.ZX_APPEND_STATIC_SCALES}[mode]
    pool_e = torch.zeros((L, n_pages, 2, H, P, D), dtype=torch.uint8, device=dev)
    if static:
        sc_e = torch.rand((L, 2, H), generator=torch.Generator().manual_seed(1)).to(dev) * 0.01 + 0.002
    else:
        sc_e = torch.empty((L, 2, H), dtype=torch.float32, device=dev)
    err_e = torch.zeros(1, dtype=torch.int32, device=dev)
    kv.kv_quant_append(x, cu, bt, pool_e, scales=sc_e, static_scales=static, two_pass=mode == "two_pass",
                       single_pass=mode == "single_pass", err=err_e)
    pool_g = torch.zeros_like(pool_e)
    sc_g = sc_e.clone()
    err_g = torch.zeros(1, dtype=torch.int32, device=dev)
    N.check(_noalloc(x, cu, bt, pool_g, sc_g, flags, err_g), "kv_quant_append_noalloc (eager)")
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side), torch.cuda.graph(graph, stream=side):
        rc = _noalloc(x, cu, bt, pool_g, sc_g, flags, err_g)
    assert rc == N.ZX_OK, N.load().zx_last_error()
    for rep in range(3):
        pool_g.zero_()  # the eager pool started from zeros too
        err_g.zero_()
        if not static:
            sc_g.fill_(-1.0)
        torch.cuda.synchronize(dev)
        graph.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(pool_g, pool_e), f"replay {rep}: {(pool_g != pool_e).sum().item()} codes differ"
        assert torch.equal(sc_g.view(torch.int32), sc_e.view(torch.int32)), f"replay {rep}: scales differ"
        assert int(err_g.item()) == int(err_e.item()), f"replay {rep}: error word differs"
        x.mul_(1.0)  # eager work between replays
