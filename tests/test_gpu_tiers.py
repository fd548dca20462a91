"""Three-tier Belady tiering on the GPU (README.md:150-154, HBM / DRAM / NVMe):
zx_belady_tier_plan against the oracle's explicit two-heap hierarchy (bit-exact per
position), and ThreeTierReplay moving real page bytes through a device pool, a pinned
host pool and a file, checked after every batch."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from zenyx_amd import kv
from zenyx_amd.train.belady_tiers import ThreeTierPlan, ThreeTierReplay

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _cases():
    rng = np.random.default_rng(11)
    out = []
    for n_pages, n in [(8, 100), (64, 2000), (500, 20000), (4000, 200000)]:
        out.append((rng.integers(0, n_pages, n).astype(np.int32), n_pages))
        hot = rng.integers(0, max(2, n_pages // 8), n)
        out.append((np.where(rng.random(n) < 0.7, hot, rng.integers(0, n_pages, n)).astype(np.int32), n_pages))
    out.append((O.ring_trace(3, 4, 8), 96))
    out.append((O.ring_trace(8, 8, 64), 8 * 8 * 64))
    return out


@pytest.mark.parametrize("case", range(10))
def test_tier_plan_matches_oracle(case):
    trace, n_pages = _cases()[case]
    print(f"tier plan case {case}: n={trace.size} pages={n_pages}", flush=True)
    rng = np.random.default_rng(case)
    t = torch.from_numpy(trace).to(DEV)
    for c0, c1 in [(max(1, n_pages // 5), n_pages // 4), (1, 1), (max(1, n_pages // 3), 0),
                   (int(rng.integers(1, n_pages)), int(rng.integers(0, n_pages)))]:
        want_src, want_v0, want_v1, _ = O.belady_tiers(trace, n_pages, c0, c1)
        sim0 = kv.BeladyTraceSim(t, n_pages, c0, record_misses=True)
        sim0.run()
        sim01 = kv.BeladyTraceSim(t, n_pages, c0 + c1, record_misses=True)
        sim01.run()
        src, v0, v1 = kv.belady_tier_plan(sim0, sim01, check=True)
        assert np.array_equal(src.cpu().numpy(), want_src), (c0, c1)
        assert np.array_equal(v0.cpu().numpy(), want_v0), (c0, c1)
        assert np.array_equal(v1.cpu().numpy(), want_v1), (c0, c1)


def test_three_tier_plan_slots_match_host_bookkeeping():
    trace, n_pages = _cases()[9]
    t = torch.from_numpy(trace).to(DEV)
    plan = ThreeTierPlan(t, n_pages, 700, 500, spare=64)
    src, v0, v1, _ = O.belady_tiers(trace, n_pages, 700, 500)
    nu, pu = O.next_use(trace, n_pages)
    ref = ThreeTierPlan.from_schedule(trace, n_pages, 700, 500, 64, src, v0, v1, nu, pu)
    for name in ("src", "v0", "v1", "adm0", "dep0", "adm1", "dep1", "slot0", "last_use"):
        assert np.array_equal(getattr(plan, name), getattr(ref, name)), name


def _pattern(pages: torch.Tensor, pb: int) -> torch.Tensor:
    """[len(pages), pb] uint8 bytes that identify each page."""
    k = torch.arange(pb, device=DEV, dtype=torch.int64)
    return ((k[None, :] * 7 + pages.to(torch.int64)[:, None] * 131 + 3) % 251).to(torch.uint8)


@pytest.mark.parametrize("which,c0,c1,spare,max_batch", [(8, 24, 16, 8, None), (9, 600, 400, 64, None),
                                                          (3, 20, 12, 4, 3), (5, 150, 0, 16, None)])
def test_three_tier_replay_keeps_bytes(tmp_path, which, c0, c1, spare, max_batch):
    trace, n_pages = _cases()[which]
    pb = 4096
    print(f"replay case {which}: n={trace.size} c0={c0} c1={c1} spare={spare}", flush=True)
    plan = ThreeTierPlan(torch.from_numpy(trace).to(DEV), n_pages, c0, c1, spare=spare)
    with ThreeTierReplay(plan, pb, str(tmp_path / "t2.bin"), device=DEV, io_threads=4) as rep:
        t0_rows = rep.t0.view(-1, pb)

        def create(pages, slots):
            t0_rows[torch.from_numpy(slots).to(DEV)] = _pattern(torch.from_numpy(pages).to(DEV), pb)

        checked = [0]

        def after_batch(a, b):
            pages = torch.from_numpy(plan.trace[a:b]).to(DEV)
            slots = torch.from_numpy(plan.slot0[a:b]).to(DEV)
            got = t0_rows[slots]
            assert torch.equal(got, _pattern(pages, pb)), f"bytes differ in batch [{a}, {b})"
            checked[0] += b - a

        out = rep.run(0, trace.size, create=create, after_batch=after_batch, max_batch=max_batch)
    assert rep.fd is None
    assert checked[0] == trace.size
    st = plan.stats()
    assert out["new_pages"] == st["new"] and out["t2_t0_pages"] == st["from_t2"]
    assert out["t1_t0_pages"] == st["from_t1"]
    if c1 > 0:
        assert out["t1_t0_pages"] > 0 or st["from_t1"] == 0
    assert out["t2_t0_pages"] > 0


@pytest.mark.parametrize("direction", ["h2d", "d2h", "d2d"])
def test_tier_move_pages(direction):
    pb, n_src, n_dst, n = 4096, 300, 200, 150
    g = torch.Generator().manual_seed(5)
    src_host = torch.randint(0, 256, (n_src * pb,), dtype=torch.uint8, generator=g)
    dst_host = torch.randint(0, 256, (n_dst * pb,), dtype=torch.uint8, generator=g)
    src = src_host.pin_memory() if direction == "h2d" else src_host.to(DEV)
    dst = dst_host.pin_memory() if direction == "d2h" else dst_host.to(DEV)
    so = torch.randperm(n_src, generator=g)[:n].to(torch.int64) * pb
    do = torch.randperm(n_dst, generator=g)[:n].to(torch.int64) * pb
    want = dst_host.clone().view(-1, pb)
    want[do // pb] = src_host.view(-1, pb)[so // pb]
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    kv.tier_move_pages(dst, src, do.pin_memory(), so.to(DEV), pb, max_workgroups=7, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert torch.equal(dst.cpu().view(-1, pb), want)


def test_tier_move_pages_flags_out_of_range():
    pb = 1024
    src = torch.arange(8 * pb, dtype=torch.int32, device=DEV).to(torch.uint8)
    dst = torch.zeros(4 * pb, dtype=torch.uint8, device=DEV)
    so = torch.tensor([0, pb, 7 * pb + 16], dtype=torch.int64, device=DEV)  # the last runs past src
    do = torch.tensor([0, 3 * pb + 8, pb], dtype=torch.int64, device=DEV)   # the second runs past dst
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    kv.tier_move_pages(dst, src, do, so, pb, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 1
    assert torch.equal(dst[:pb], src[:pb])            # the valid page moved
    assert torch.count_nonzero(dst[pb:]) == 0         # the others were skipped
