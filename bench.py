"""Benchmark of the KV-cache hot path on one MI355X.

Headline (``value``): configs[1] of the benchmark definition -- paged append with fused FP8 quantisation at
the Llama-3-8B KV shape (32 layers, 8 KV heads, head_dim 128, page 16, 16 sequences of
U[1k, 8k] tokens, 5% of each sequence's (layer, head) pairs x50), one step = one append
of every layer, inputs already resident in HBM.  Reported as algorithmic GB/s
(3 bytes per KV element + scales + block tables) and as a fraction of the 8 TB/s HBM3E
peak.  Also measured: configs[2] (paged gather + dequant, 64 x 32k decode, 300k-page
pool; plus decode attention computed straight from those FP8 pages), ring attention over FP8
pages (4 x 8k causal, ring degree 1 and 8: TFLOP/s against the bf16 matrix-core peak), configs[3]
(Belady tiering of a ring-attention trace: evictions/s, plus the
pinned-host tier moves of one layer overlapped with compute; and the same schedule over three
tiers, HBM / pinned DRAM / a file, planned on the GPU and replayed for three windows) and configs[4] (80-layer
70B-shape share streamed through 60 HBM layer slots and pinned DRAM: per-kernel append
and gather GB/s, D2H / H2D GB/s), and configs[0] (the reference's CPU-runnable cache:
quant + dequant on the GPU and in torch on the host cores).

The CPU baseline is the oracle's CPU restatement timed on this machine's host cores: for
the append and the gather its torch form (all of torch's threads, and one thread beside
it; bit-identical to the C oracle), elsewhere the C oracle; each on a bounded sample of
the same workload.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu]
                    [--only append|gather|decode|ring|belady|tiers|weights|configs4|configs4_16gb|stream|configs0|copy|all]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBPS = 8000.0
METRIC = "KV quant+append & gather+dequant GB/s (% HBM peak); evictions/sec"
# HBM bytes per launch of the dominant kernel, measured with rocprofv3 FETCH_SIZE and
# WRITE_SIZE and scaled by the same counters on a plain 4 GiB copy (profiles/*.md); keyed by
# (workload, seed) because the append's size depends on the seed.
MEASURED_TRAFFIC = {("append", 1): 14_860_676_704, ("gather", 2): 12_889_463_193}
TRAFFIC_SOURCE = ("profile figure, not measured in this run: rocprofv3 FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000 "
                  "per dispatch (profiles/kv_append_fused_configs1.md, profiles/gather_dequant_configs2.md)")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--skip-cpu", action="store_true", help="omit the CPU baseline leg")
    ap.add_argument("--only", choices=["append", "gather", "decode", "ring", "belady", "tiers", "weights", "configs4",
                                       "configs4_16gb", "stream",
                                       "configs0", "copy", "all"],
                    default="all")
    ap.add_argument("--seed", type=int, default=1)
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------------ workloads

def make_append_workload(torch, dev, seed=1):
    """32L, 8H, 128D, P=16, 16 seqs with T_b ~ U[1024, 8192]."""
    L, H, D, P, B = 32, 8, 128, 16, 16
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1024, 8193, (B,), generator=g).tolist()
    T = sum(lens)
    nb = [(n + P - 1) // P for n in lens]
    n_pages = sum(nb)
    max_blocks = max(nb)
    perm = torch.randperm(n_pages, generator=g).to(torch.int32)
    bt = torch.full((B, max_blocks), -1, dtype=torch.int32)
    k = 0
    for b in range(B):
        bt[b, :nb[b]] = perm[k:k + nb[b]]
        k += nb[b]
    cu = torch.zeros(B + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    # outliers: per sequence, 5% of its 256 (layer, head) pairs (13) scaled x50 on K and V
    outl = [torch.randperm(L * H, generator=g)[:13].tolist() for _ in range(B)]
    gd = torch.Generator(device=dev).manual_seed(seed)
    x = torch.empty((L, T, 2, H, D), dtype=torch.bfloat16, device=dev)
    for l in range(L):
        x[l].normal_(generator=gd)
    for b in range(B):
        for lh in outl[b]:
            l, h = divmod(lh, H)
            x[l, cu[b]:cu[b + 1], :, h] *= 50.0
    pool = torch.zeros((L, n_pages, 2, H, P, D), dtype=torch.uint8, device=dev)
    N = L * T * 2 * H * D
    alg_bytes = 3 * N + 4 * L * 2 * H + 4 * L * n_pages + 4 * (B + 1)
    return dict(x=x, cu=cu.to(dev), bt=bt.to(dev), pool=pool, lens=lens, T=T, n_pages=n_pages,
                N=N, alg_bytes=alg_bytes, L=L, H=H, D=D, P=P, B=B, cu_host=cu, bt_host=bt)


def make_gather_workload(torch, dev, seed=2):
    """64 seqs x 32768 tokens, 300k-page FP8 pool, fragmented tables."""
    n_pool, H, D, P, B, T, L = 300_000, 8, 128, 16, 64, 32768, 32
    g = torch.Generator().manual_seed(seed)
    max_blocks = T // P
    bt = torch.randperm(n_pool, generator=g)[: B * max_blocks].to(torch.int32).reshape(B, max_blocks)
    scales = (torch.rand((L, 2, H), generator=g) * (1 - 1e-3) + 1e-3).float()
    gd = torch.Generator(device=dev).manual_seed(seed)
    pool = torch.randint(0, 256, (n_pool, 2, H, P, D), dtype=torch.uint8, device=dev, generator=gd)
    pool[pool == 0x7F] = 0x7E
    pool[pool == 0xFF] = 0xFE
    seq_lens = torch.full((B,), T, dtype=torch.int32)
    layer = 7
    N = B * T * 2 * H * D
    alg_bytes = 3 * N + 4 * B * max_blocks + 4 * 2 * H + 4 * B
    return dict(pool=pool, scales=scales.to(dev), layer=layer, bt=bt.to(dev), seq_lens=seq_lens.to(dev),
                T=T, B=B, H=H, D=D, P=P, N=N, alg_bytes=alg_bytes, bt_host=bt, scales_host=scales)


# ------------------------------------------------------------------ timing

def time_steps(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    t0 = time.perf_counter()
    ev[0].record(st)
    for i in range(steps):
        fn()
        ev[i + 1].record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    return sum(per) / steps, per, wall


def _median_time(fn, reps=5):
    import statistics

    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline_append(W, budget_s=8.0):
    """CPU baseline of the append: the torch restatement (oracle.kv_quant_append_torch,
    bit-identical to the C oracle) on all of layer 0, with all of torch's threads and with
    one (median of 5 after a warm-up), plus the scalar C oracle on a bounded sample."""
    import numpy as np
    import torch

    from oracle import oracle as O

    x0 = W["x"][0].cpu()  # [T, 2, H, D] bf16
    lens, P, H, D = W["lens"], W["P"], W["H"], W["D"]
    cu, bt = W["cu_host"].numpy(), W["bt_host"].numpy()
    n_layer = x0.numel()
    threads = torch.get_num_threads()
    res = {}
    for nt in (threads, 1):
        torch.set_num_threads(nt)
        res[nt] = _median_time(lambda: O.kv_quant_append_torch(x0, cu, bt, W["n_pages"], P))
    torch.set_num_threads(threads)
    # the C oracle (scalar, one thread): whole sequences of layer 0 until about budget_s
    xb = x0.view(torch.int16).numpy().view(np.uint16)
    pool = np.zeros((1, W["n_pages"], 2, H, P, D), np.uint8)
    done_tok, elapsed, b = 0, 0.0, 0
    while b < len(lens) and elapsed < budget_s:
        xs = np.ascontiguousarray(xb[cu[b]:cu[b + 1]])[None]
        t0 = time.perf_counter()
        O.kv_quant_append(xs, np.array([0, lens[b]], np.int32), None, bt[b:b + 1], pool, P)
        elapsed += time.perf_counter() - t0
        done_tok += lens[b]
        b += 1
    gb = lambda sec: round(3 * n_layer / sec / 1e9, 4)  # noqa: E731
    return {"value": gb(res[threads]), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"torch restatement of the append (oracle.kv_quant_append_torch, bit-identical to the C "
                      f"oracle) on all of layer 0 ({W['T']} tokens, {n_layer} elements), {threads} threads, median "
                      f"of 5: {res[threads]:.3f} s",
            "one_thread": {"value": gb(res[1]), "seconds": round(res[1], 3)},
            "c_oracle_one_thread": {"value": round(3 * done_tok * 2 * H * D / elapsed / 1e9, 4),
                                    "sample": f"sequences 0..{b - 1} of layer 0, {elapsed:.1f} s"}}


def cpu_baseline_gather(W, n_seq=4):
    """CPU baseline of the gather: the torch restatement (oracle.kv_gather_dequant_torch)
    on n_seq whole sequences of the layer with all of torch's threads and on one with a
    single thread (median of 5 after a warm-up)."""
    import torch

    from oracle import oracle as O

    H, D, T = W["H"], W["D"], W["T"]
    bt = W["bt_host"][:n_seq]
    pages = torch.unique(bt.reshape(-1)).long()
    remap = torch.full((int(pages.max()) + 1,), -1, dtype=torch.int64)
    remap[pages] = torch.arange(len(pages))
    sub = W["pool"][pages.to(W["pool"].device)].cpu()  # only the sampled sequences' pages
    btl = remap[bt.long()]
    sc = W["scales_host"][W["layer"]]
    threads = torch.get_num_threads()
    t_all = _median_time(lambda: O.kv_gather_dequant_torch(sub, sc, btl, [T] * n_seq, T))
    torch.set_num_threads(1)
    t_one = _median_time(lambda: O.kv_gather_dequant_torch(sub, sc, btl[:1], [T], T))
    torch.set_num_threads(threads)
    n_all, n_one = n_seq * T * 2 * H * D, T * 2 * H * D
    return {"value": round(3 * n_all / t_all / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"torch restatement of the gather (oracle.kv_gather_dequant_torch, bit-identical to the C "
                      f"oracle), {n_seq} of {W['B']} sequences of one layer ({n_all} elements), {threads} threads, "
                      f"median of 5: {t_all:.3f} s",
            "one_thread": {"value": round(3 * n_one / t_one / 1e9, 4), "sample": "one sequence", "seconds":
                           round(t_one, 3)}}


def belady_leg(torch, dev, skip_cpu):
    """Belady tiering of a 1M-token, 80-layer ring schedule (degree 8), FP8
    pages of 64 tokens (128 KiB), 64 GB HBM budget, spill tier = pinned host DRAM."""
    from zenyx_amd.train.belayd_kv_cache_tiering import BeladyKVCacheTieringManager

    m = BeladyKVCacheTieringManager(num_devices=8, context_length=2**20, num_layers=80, num_kv_heads=8,
                                    head_dim=128, page_tokens=64, hbm_budget_bytes=64e9, device=dev)
    log(f"belady: {len(m.sequence)} accesses over {m.n_pages} pages, capacity {m.capacity}")
    m.plan()  # warm-up (kernel loading, allocator)
    stats = m.plan()
    sim_s, nu_s = m.timings["simulate_s"], m.timings["next_use_s"]
    ev = stats["evictions"]
    out = {"workload": "configs[3]: Belady MIN over a ring-attention schedule, 1M tokens, 80 layers, ring 8, "
                       "FP8 pages of 64 tokens (128 KiB), 64 GB HBM budget",
           "accesses": len(m.sequence), "pages": m.n_pages, "capacity_pages": m.capacity,
           "evictions": ev, "misses": stats["misses"], "hits": stats["hits"],
           "simulate_ms": round(sim_s * 1e3, 3), "next_use_ms": round(nu_s * 1e3, 3),
           "evictions_per_s": round(ev / sim_s, 1)}
    # the next-use tables alone (zx_belady_next_use: radix sort of the trace by page, then
    # neighbours), HIP events on the compute stream, median of 5 after a warm-up
    from zenyx_amd import kv
    trace_d = m.sim.trace
    kv.next_use(trace_d, m.n_pages)
    nu_ms = []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        kv.next_use(trace_d, m.n_pages)
        e1.record()
        torch.cuda.synchronize(dev)
        nu_ms.append(e0.elapsed_time(e1))
    out["next_use_kernels_ms"] = round(sorted(nu_ms)[2], 3)
    out["next_use_note"] = ("next_use_ms times the whole BeladyTraceSim set-up (tables, state, eviction lists) on the "
                            "host clock; next_use_kernels_ms the radix sort and neighbour kernels alone")
    log(f"belady: {ev} evictions in {sim_s * 1e3:.1f} ms -> {ev / sim_s / 1e6:.2f} M evictions/s "
        f"(set-up with next-use tables {nu_s * 1e3:.1f} ms; next-use kernels {out['next_use_kernels_ms']} ms)")
    # tier moves of one backward layer while a dequant-gather runs on the compute stream
    n = len(m.sequence)
    per_layer = n // 2 // 80
    t_a = n // 2 + 40 * per_layer
    pool = torch.randint(0, 126, (8192, 2, 8, 16, 128), dtype=torch.uint8, device=dev)
    bt = torch.randperm(8192, device=dev)[:64 * 128].to(torch.int32).view(64, 128)
    sl = torch.full((64,), 2048, dtype=torch.int32, device=dev)
    sc = torch.full((2, 8), 0.01, dtype=torch.float32, device=dev)

    def compute():
        for _ in range(20):
            kv.kv_gather_dequant(pool, sc, bt, sl, 2048)

    # two windows: the backward of layer 39 brings spilled pages back (H2D); the forward of
    # layer 50 evicts pages that the backward will use again (D2H)
    windows = {"backward_layer39": t_a, "forward_layer50": 50 * per_layer}
    m.replay_transfers(t_a, t_a + per_layer)  # warm-up: pinned pools, copy engines
    out["tier_moves"] = {}
    for name, a in windows.items():
        r = m.replay_transfers(a, a + per_layer, compute=compute)
        out["tier_moves"][name] = {
            "window": f"trace positions [{a}, {a + per_layer})", "d2h_pages": r["d2h_pages"],
            "h2d_pages": r["h2d_pages"], "d2h_GBps": round(r["d2h_GBps"], 2), "h2d_GBps": round(r["h2d_GBps"], 2),
            "overlapped_with": "20 paged gather+dequant kernels on the compute stream", "wall_ms": round(r["wall_ms"], 3)}
        log(f"tier moves, {name}: {r['d2h_pages']} D2H pages at {r['d2h_GBps']:.1f} GB/s, {r['h2d_pages']} H2D pages "
            f"at {r['h2d_GBps']:.1f} GB/s")
    out["tier_moves"]["both_directions"] = bidirectional_window(torch, dev, compute, skip_cpu)
    out["dropin_cache"] = dropin_belady_leg(torch, dev, m.capacity, len(m.sequence))
    out["curriculum"] = curriculum_leg(torch, dev, skip_cpu)
    if not skip_cpu:
        import numpy as np

        from oracle import oracle as O

        trace = m.sequence.trace("cpu").numpy()
        t0 = time.perf_counter()
        _, _, st = O.belady_simulate(trace, m.n_pages, m.capacity, evict_cap=1)
        dt = time.perf_counter() - t0
        assert st["evictions"] == ev, "GPU and CPU Belady disagree on the eviction count"
        out["cpu_baseline"] = {"value": round(ev / dt, 1), "unit": "evictions/s", "cores": 1, "kind": "port",
                               "sample": f"C oracle (indexed binary heap, 1 thread) over the full trace: "
                                         f"{ev} evictions in {dt:.2f} s"}
        # the reference's own algorithm: a linear scan of the resident set per victim (belady.py:46-50)
        cache = O.RefBeladyApproxCache(m.capacity)
        rng = np.random.default_rng(0)
        keys = rng.integers(0, n, m.capacity)
        for i in range(m.capacity):
            cache.update_future(i, int(keys[i]))
            cache._resident[i] = True
        t0 = time.perf_counter()
        k = 0
        while time.perf_counter() - t0 < 5.0:
            cache._select_victim()
            k += 1
        out["reference_linear_scan_evictions_per_s"] = round(k / (time.perf_counter() - t0), 3)
    del m
    return out


def bidirectional_window(torch, dev, compute, skip_cpu=True):
    """Tier moves in both directions at once: configs[3]'s geometry (ring 8 over 1M tokens,
    64-token FP8 pages of 128 KiB, 16,384 pages = 2 GiB per layer) for 3 layers under an
    HBM budget of 12,288 pages (1.5 GiB), smaller than one layer.  Inside layer 1's
    forward window the ring revisits its shards, so Belady writes back victims that are
    used again later (D2H) while pages it evicted earlier come back (H2D); the replay runs
    the two directions on the library's two copy streams at the same time, beside
    ``compute`` on the compute stream.  Also times the schedule itself: with a budget below
    one layer almost every window of the simulator has victims among the pages it has just
    seen, the regime where the next victim depends on the one before."""
    from zenyx_amd.train.belayd_kv_cache_tiering import BeladyKVCacheTieringManager

    pb = 64 * 8 * 128 * 2
    m = BeladyKVCacheTieringManager(num_devices=8, context_length=2**20, num_layers=3, num_kv_heads=8,
                                    head_dim=128, page_tokens=64, hbm_budget_bytes=12288 * pb, device=dev)
    m.plan()  # warm-up
    stats = m.plan()
    sim_s = m.timings["simulate_s"]
    sched = {"accesses": len(m.sequence), "evictions": stats["evictions"], "simulate_ms": round(sim_s * 1e3, 3),
             "evictions_per_s": round(stats["evictions"] / sim_s, 1)}
    log(f"small-budget schedule: {stats['evictions']} evictions over {len(m.sequence)} accesses in "
        f"{sim_s * 1e3:.1f} ms")
    if not skip_cpu:
        from oracle import oracle as O

        trace = m.sequence.trace("cpu").numpy()
        t0 = time.perf_counter()
        _, _, st = O.belady_simulate(trace, m.n_pages, m.capacity, evict_cap=1)
        dt = time.perf_counter() - t0
        assert st["evictions"] == stats["evictions"], "GPU and CPU Belady disagree on the eviction count"
        sched["cpu_baseline"] = {"value": round(st["evictions"] / dt, 1), "unit": "evictions/s", "cores": 1,
                                 "kind": "port", "sample": f"C oracle (indexed binary heap, 1 thread), the same "
                                                           f"trace: {dt * 1e3:.1f} ms"}
    per_layer = len(m.sequence) // 2 // 3
    a = per_layer
    m.replay_transfers(a, a + per_layer)  # warm-up: pinned pools, copy engines
    r = m.replay_transfers(a, a + per_layer, compute=compute)
    out = {"window": f"layer 1 forward, trace positions [{a}, {a + per_layer}), 3 layers x 16384 pages, "
                     f"HBM budget {m.capacity} pages (1.5 GiB)",
           "d2h_pages": r["d2h_pages"], "h2d_pages": r["h2d_pages"], "chunks": r["chunks"],
           "d2h_GBps": round(r["d2h_GBps"], 2), "h2d_GBps": round(r["h2d_GBps"], 2),
           "both_directions_GBps": round(r["both_GBps"], 2), "copy_span_ms": round(r["copy_span_ms"], 3),
           "d2h_ms": round(r["d2h_ms"], 3), "h2d_ms": round(r["h2d_ms"], 3),
           "overlapped_with": "20 paged gather+dequant kernels on the compute stream", "wall_ms": round(r["wall_ms"], 3),
           "schedule": sched}
    log(f"tier moves, both directions: {r['d2h_pages']} D2H pages at {r['d2h_GBps']:.1f} GB/s and {r['h2d_pages']} "
        f"H2D pages at {r['h2d_GBps']:.1f} GB/s in {r['chunks']} chunks; {r['both_GBps']:.1f} GB/s both ways over "
        f"the {r['copy_span_ms']:.1f} ms span")
    del m
    return out


def dropin_belady_leg(torch, dev, capacity, n_positions, seconds=1.5, distinct=2_000_000):
    """The drop-in BeladyApproxCache (belady.py:14-55's interface) at configs[3]'s resident
    set: ``capacity`` ids resident with random next uses, then a stream of new ids, each an
    update_future + touch that misses and evicts the farthest next use.  Evictions per
    second over ~``seconds`` (host bookkeeping, the slot-update and argmax kernels and one
    stream synchronisation per eviction), measured twice: right after the fill, and again
    once ``distinct`` ids in all have been given a next use (update_future only: the
    reference's next_use dictionary keeps every id it was told about), so the second rate
    shows whether the cost per eviction grows with the ids the cache has seen."""
    import numpy as np

    from zenyx_amd.streaming import BeladyApproxCache

    rng = np.random.default_rng(0)
    keys = rng.integers(0, n_positions, distinct + 400_000)
    cache = BeladyApproxCache(capacity, device=dev)
    for i in range(capacity):
        cache.update_future(i, int(keys[i]))
        cache.touch(i)
    nxt = capacity
    for _ in range(3):  # warm-up: the first miss uploads every slot
        cache.update_future(nxt, int(keys[nxt]))
        cache.touch(nxt)
        nxt += 1

    def window():
        nonlocal nxt
        t0 = time.perf_counter()
        k = 0
        while k % 64 or time.perf_counter() - t0 < seconds:
            cache.update_future(nxt, int(keys[nxt]))
            assert len(cache.touch(nxt)) == 1
            nxt += 1
            k += 1
        return k, time.perf_counter() - t0

    k1, dt1 = window()
    seen1 = nxt
    while nxt < distinct:  # ids told about but never touched
        cache.update_future(nxt, int(keys[nxt]))
        nxt += 1
    k2, dt2 = window()
    log(f"drop-in BeladyApproxCache at {capacity} resident ids: {k1 / dt1:.0f} evictions/s with {seen1} ids seen, "
        f"{k2 / dt2:.0f} with {nxt} ids seen")
    return {"workload": f"BeladyApproxCache(capacity={capacity}): {capacity} resident ids with random next uses, "
                        "then update_future + touch of new ids, each evicting one; timed again after "
                        f"{distinct} distinct ids have been given a next use",
            "evictions": k1, "seconds": round(dt1, 3), "evictions_per_s": round(k1 / dt1, 1),
            "ids_seen": seen1,
            "after_growth": {"ids_seen": nxt, "evictions": k2, "seconds": round(dt2, 3),
                             "evictions_per_s": round(k2 / dt2, 1)}}


def curriculum_leg(torch, dev, skip_cpu):
    """A ring curriculum across two phase changes (RingDegreeScheduler, README.md:162-165):
    one training step each at degree 2 / 256k tokens, 4 / 512k and 8 / 1M, 80 layers,
    FP8 pages of 64 tokens, the 64 GB HBM budget of configs[3].  The page trace is built
    on the GPU, then next-use tables and the Belady schedule over the whole run."""
    from zenyx_amd import kv
    from zenyx_amd.train.dynamic_ring_curriculum import CurriculumPhase, RingDegreeScheduler

    L, pt, page_bytes = 80, 64, 64 * 8 * 128 * 2
    s = RingDegreeScheduler([CurriculumPhase("ring2", 2, 1 << 18, 1), CurriculumPhase("ring4", 4, 1 << 19, 1),
                             CurriculumPhase("ring8", 8, 1 << 20)], num_devices=8)
    n_pages = L * s.layer_stride(pt)
    cap = int(64e9 // page_bytes)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    s.access_trace([0, 1, 2], 2, page_tokens=pt, device=dev)  # warm-up
    ev[0].record()
    trace = s.access_trace([0, 1, 2], L, page_tokens=pt, device=dev)
    ev[1].record()
    sim = kv.BeladyTraceSim(trace, n_pages, cap, evict_cap=1)
    ev[2].record()
    sim.run()
    ev[3].record()
    torch.cuda.synchronize(dev)
    st = sim.stats()
    t_trace, t_nu, t_sim = ev[0].elapsed_time(ev[1]), ev[1].elapsed_time(ev[2]), ev[2].elapsed_time(ev[3])
    out = {"workload": "3 training steps across two phase changes: ring 2 / 256k tokens, ring 4 / 512k, "
                       "ring 8 / 1M; 80 layers, FP8 pages of 64 tokens, 64 GB HBM budget",
           "accesses": int(trace.numel()), "pages": n_pages, "capacity_pages": cap, "evictions": st["evictions"],
           "misses": st["misses"], "trace_ms": round(t_trace, 3), "trace_GBps": round(4 * trace.numel() / t_trace / 1e6, 1),
           "next_use_ms": round(t_nu, 3), "simulate_ms": round(t_sim, 3),
           "evictions_per_s": round(st["evictions"] / (t_sim * 1e-3), 1)}
    log(f"curriculum: {trace.numel()} accesses, trace {t_trace:.2f} ms, next-use {t_nu:.2f} ms, simulate {t_sim:.1f} ms, "
        f"{st['evictions']} evictions")
    if not skip_cpu:
        from oracle import oracle as O

        t0 = time.perf_counter()
        want = O.ring_curriculum_trace([2, 4, 8], [4096, 8192, 16384], L, s.layer_stride(pt))
        t1 = time.perf_counter()
        _, _, cst = O.belady_simulate(want, n_pages, cap, evict_cap=1)
        t2 = time.perf_counter()
        assert cst["evictions"] == st["evictions"], "GPU and CPU Belady disagree over the curriculum"
        out["cpu_baseline"] = {"value": round(cst["evictions"] / (t2 - t1), 1), "unit": "evictions/s", "cores": 1,
                               "kind": "port", "sample": f"C oracle: trace {t1 - t0:.2f} s, heap Belady {t2 - t1:.2f} s "
                                                         f"over the same {want.size} accesses"}
    return out


def weights_leg(torch, dev):
    """Layer-weight streaming on the KV tiers' transfer engine (LayerWeightStreamer,
    parameter_streamer.py:32-87): 16 layers of 256 MiB in pinned DRAM, at most 2 resident;
    per layer prefetch(i + 1), get(i), then ~5 ms of paged gather+dequant kernels.
    Reports the copy rate alone, the compute alone and the pipelined loop."""
    from zenyx_amd import kv
    from zenyx_amd.streaming import LayerWeightStreamer, ParameterStore

    n_layers, numel = 16, 128 << 20  # bf16: 256 MiB per layer
    store = ParameterStore()
    for i in range(n_layers):
        store.register(f"layer{i}", torch.full((numel,), float(i), dtype=torch.bfloat16))
    pool = torch.randint(0, 126, (8192, 2, 8, 16, 128), dtype=torch.uint8, device=dev)
    bt = torch.randperm(8192, device=dev)[:64 * 128].to(torch.int32).view(64, 128)
    sl = torch.full((64,), 2048, dtype=torch.int32, device=dev)
    sc = torch.full((2, 8), 0.01, dtype=torch.float32, device=dev)

    def compute(reps):
        for _ in range(reps):
            kv.kv_gather_dequant(pool, sc, bt, sl, 2048)

    def timed(fn):
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize(dev)
        return time.perf_counter() - t0

    compute(4)
    one = timed(lambda: compute(10)) / 10
    reps = max(1, int(round(5e-3 / one)))
    t_compute = timed(lambda: [compute(reps) for _ in range(n_layers)])

    def copies_only():
        s = LayerWeightStreamer(store, dev, max_resident_layers=2)
        for i in range(n_layers):
            s.get(f"layer{i}")

    def pipelined():
        s = LayerWeightStreamer(store, dev, max_resident_layers=2)
        for i in range(n_layers):
            if i + 1 < n_layers:
                s.prefetch(f"layer{i + 1}")
            s.get(f"layer{i}")
            compute(reps)

    copies_only()  # warm-up
    t_copy = timed(copies_only)
    pipelined()
    t_pipe = timed(pipelined)
    layer_bytes = numel * 2
    hidden = (t_copy + t_compute - t_pipe) / min(t_copy, t_compute)
    out = {"workload": f"{n_layers} layers x 256 MiB bf16 weights, 2 resident, prefetch-next, "
                       f"{reps} gather+dequant kernels (~5 ms) per layer",
           "h2d_GBps": round(n_layers * layer_bytes / t_copy / 1e9, 2), "copy_ms": round(t_copy * 1e3, 2),
           "compute_ms": round(t_compute * 1e3, 2), "pipelined_ms": round(t_pipe * 1e3, 2),
           "overlap_frac": round(hidden, 3)}
    log(f"weights: copies {t_copy * 1e3:.1f} ms ({out['h2d_GBps']} GB/s), compute {t_compute * 1e3:.1f} ms, "
        f"pipelined {t_pipe * 1e3:.1f} ms (overlap {hidden:.2f})")
    return out


def tiers_leg(torch, dev):
    """configs[3]'s schedule over three tiers (README.md:150-154: HBM / DRAM / NVMe): T0 =
    the 64 GB HBM budget, T1 = 32 GiB of pinned host DRAM, T2 = a file.  The whole trace
    is planned on the GPU (two Belady runs + the plan kernel, then host slot bookkeeping);
    three windows are replayed with real page bytes, each overlapped with 20 paged
    gather+dequant kernels on the compute stream: the forward of layer 50 (T0 -> T1 and
    T1 -> T2 moves), the backward of layer 40 (T1 -> T0) and the backward of layer 20
    (T2 -> T0; its pages are written to the file first, untimed)."""
    import shutil

    import numpy as np

    from zenyx_amd import kv
    from zenyx_amd.train.belady_tiers import ThreeTierPlan, ThreeTierReplay
    from zenyx_amd.train.belayd_kv_cache_tiering import BeladyKVCacheTieringManager

    m = BeladyKVCacheTieringManager(num_devices=8, context_length=2**20, num_layers=80, num_kv_heads=8,
                                    head_dim=128, page_tokens=64, hbm_budget_bytes=64e9, device=dev)
    spare = 4096
    t1_pages = (32 << 30) // m.page_bytes - spare  # T1 pool (with spare slots) = 32 GiB
    trace = m.sequence.trace(dev)
    ThreeTierPlan(trace[:65536].contiguous(), m.n_pages, 1024, 1024, spare=64)  # warm-up
    plan = ThreeTierPlan(trace, m.n_pages, m.capacity, t1_pages, spare=spare)
    st = plan.stats()
    log(f"three tiers: plan {st['gpu_plan_s'] * 1e3:.0f} ms on the GPU + {st['host_slots_s']:.2f} s of host slots; "
        f"{st['from_t1']} pages back from DRAM, {st['from_t2']} from the file")
    out = {"workload": "configs[3] schedule over T0 = 64 GB HBM, T1 = 32 GiB pinned DRAM, T2 = file",
           "t0_pages": m.capacity, "t1_pages": t1_pages, "spare_slots": spare, "plan": st}
    tmpdir = os.environ.get("TMPDIR", "/tmp")
    if shutil.disk_usage(tmpdir).free < (12 << 30):
        out["replay"] = f"skipped: less than 12 GiB free under {tmpdir}"
        return out
    path = os.path.join(tmpdir, f"zx_t2_{os.getpid()}.bin")
    pool = torch.randint(0, 126, (8192, 2, 8, 16, 128), dtype=torch.uint8, device=dev)
    bt = torch.randperm(8192, device=dev)[:64 * 128].to(torch.int32).view(64, 128)
    sl = torch.full((64,), 2048, dtype=torch.int32, device=dev)
    sc = torch.full((2, 8), 0.01, dtype=torch.float32, device=dev)

    def compute():
        for _ in range(20):
            kv.kv_gather_dequant(pool, sc, bt, sl, 2048)

    n = plan.trace.size
    per_layer = n // 2 // 80
    windows = {"forward_layer50": (50 * per_layer, 51 * per_layer),
               "backward_layer40": (n // 2 + 39 * per_layer, n // 2 + 40 * per_layer),
               "backward_layer20": (n // 2 + 59 * per_layer, n // 2 + 60 * per_layer)}
    rep = ThreeTierReplay(plan, m.page_bytes, path, device=dev)
    try:
        a, b = windows["backward_layer20"]
        pages = plan.moves(a, b)["t2_t0"][0]
        if len(pages):  # the window reads these pages from the file: put them there first
            rep._pwrite(rep._t1_np, (np.arange(len(pages)) % (plan.c1 + spare)) * m.page_bytes, pages)
        a, b = windows["backward_layer40"]
        rep.run(a, a + 8192)  # warm-up: staging buffers, copy engines
        res = {}
        for name, (a, b) in windows.items():
            r = rep.run(a, b, compute=compute)
            keep = ("batches", "wall_s", "t0_t1_pages", "t1_t0_pages", "t2_t0_pages", "t1_t2_pages", "t0_t2_pages",
                    "d2h_GBps", "h2d_GBps", "disk_write_GBps", "disk_read_GBps", "direct_io")
            res[name] = {k: (round(r[k], 3) if isinstance(r[k], float) else r[k]) for k in keep}
            log(f"three tiers {name}: " + ", ".join(f"{k} {res[name][k]}" for k in keep))
        out["replay"] = res
        out["overlapped_with"] = "20 paged gather+dequant kernels on the compute stream per window"
    finally:
        rep.close()
        os.remove(path)
    return out


C5 = dict(L=80, H=8, D=128, P=16, B=4, Tb=131072, hbm_layers=60)


def configs0_leg(torch, dev, steps, warmup):
    """the reference's CPU-runnable case -- the README toy model's cache
    [12 layers, K/V, B=1, 12 heads, 4096 tokens, 64], seed 0, quantised per (layer, kv,
    head) and dequantised: FP8 e4m3 per head (FP8KVQuantizer, README.md:157) and the
    legacy int8 per-tensor functions of precision.py:8-16 applied per slab.  GPU: the HIP
    kernels; CPU: the same semantics in torch on the host (all of torch's threads and one
    thread, median of 5 after a warm-up)."""
    import platform
    import statistics

    from zenyx_amd import kv

    torch.manual_seed(0)
    x = torch.randn([12, 2, 1, 12, 4096, 64], dtype=torch.float32).to(torch.bfloat16)
    n = x.numel()
    xd = x.to(dev).reshape(24, 1, 12, 4096 * 64)

    def gpu_fp8():
        c, s = kv.fp8_quant_heads(xd)
        return c, s, kv.fp8_dequant_heads(c, s)

    slabs = [xd[o, 0, h] for o in range(24) for h in range(12)]
    xs = xd.reshape(24, 12, 4096 * 64).reshape(288, 4096 * 64)  # slab (l, kv, h) = row 12 (2 l + kv) + h

    def gpu_int8_loop():  # the reference's per-tensor API called per slab
        return [kv.int8_legacy_dequant(*kv.int8_legacy_quant(t)) for t in slabs]

    def gpu_int8():  # the same per-slab functions in one launch each
        return kv.int8_legacy_dequant_slabs(*kv.int8_legacy_quant_slabs(xs))

    ms_f, _, _ = time_steps(torch, gpu_fp8, steps, warmup)
    ms_i, _, _ = time_steps(torch, gpu_int8, steps, warmup)
    ms_il, _, _ = time_steps(torch, gpu_int8_loop, max(1, steps // 4), 1)

    def cpu_fp8(x):
        xf = x.reshape(24, 1, 12, 4096 * 64).float()
        sc = xf.abs().amax(dim=(1, 3)).clamp_min(1e-8) / 448.0
        codes = (xf / sc[:, None, :, None]).to(torch.float8_e4m3fn)
        return codes, sc, (codes.float() * sc[:, None, :, None]).to(torch.bfloat16)

    def cpu_int8(x):
        out = []
        for o in range(24):
            for h in range(12):
                t = x[o // 2, o % 2, 0, h]
                scale = t.abs().amax().clamp_min(1e-8) / 127.0  # in t's dtype (bf16), as precision.py
                q = torch.clamp(torch.round(t / scale), -127, 127).to(torch.int8)
                out.append((q.float() * scale).to(torch.bfloat16))
        return out

    def med(fn, reps=5):
        fn(x)
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn(x)
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    threads = torch.get_num_threads()
    cpu = {}
    for nt in (threads, 1):
        torch.set_num_threads(nt)
        cpu[nt] = (med(cpu_fp8), med(cpu_int8))
    torch.set_num_threads(threads)
    # parity of this very run: GPU codes / scales / dequant against the CPU restatement
    gc, gs, gy = gpu_fp8()
    cc, cs, cy = cpu_fp8(x)
    same = (torch.equal(gc.cpu(), cc.view(torch.uint8)) and torch.equal(gs.cpu().view(torch.int32), cs.view(torch.int32))
            and torch.equal(gy.cpu().view(torch.int16), cy.reshape(gy.shape).view(torch.int16)))
    gi8 = gpu_int8().cpu()
    same_i8 = all(torch.equal(gi8[i].reshape(-1).view(torch.int16), c.reshape(-1).view(torch.int16))
                  for i, c in enumerate(cpu_int8(x)))
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    gb = lambda sec: round(2 * 3 * n / sec / 1e9, 3)  # noqa: E731  quant + dequant, 3 B/element each
    res = {"workload": "configs[0]: [12,2,1,12,4096,64] bf16 (seed 0), per (layer, kv, head) quant then dequant; "
                       "FP8 e4m3 per head and the legacy int8 per-tensor functions per slab",
           "elements": n,
           "gpu": {"fp8_heads_ms": round(ms_f, 4), "fp8_heads_GBps": gb(ms_f * 1e-3),
                   "int8_legacy_slabs_ms": round(ms_i, 4), "int8_legacy_GBps": gb(ms_i * 1e-3),
                   "int8_legacy_per_tensor_loop_ms": round(ms_il, 3),
                   "note": "int8 per slab in one launch each (zx_int8_legacy_quant_slabs / _dequant_slabs); the "
                           "loop figure calls the reference's per-tensor API once per slab (576 launches)"},
           "cpu": {"nproc": os.cpu_count(), "model": model, "machine": platform.machine(),
                   f"threads_{threads}": {"fp8_s": round(cpu[threads][0], 4), "int8_s": round(cpu[threads][1], 4),
                                          "fp8_GBps": gb(cpu[threads][0]), "int8_GBps": gb(cpu[threads][1])},
                   "threads_1": {"fp8_s": round(cpu[1][0], 4), "int8_s": round(cpu[1][1], 4),
                                 "fp8_GBps": gb(cpu[1][0]), "int8_GBps": gb(cpu[1][1])},
                   "kind": "torch ATen on the host, same semantics (median of 5 after a warm-up)"},
           "gpu_equals_cpu": {"fp8_codes_scales_dequant": bool(same), "int8_all_288_slabs": bool(same_i8)}}
    # the same functions at size: one 1 Gi-element bf16 tensor (2 GiB), per tensor (the
    # reference's precision.py API) and per head (FP8, 64 x 4 x 8 slabs of 512 K elements)
    big = torch.randn((64, 4, 8, 1 << 19), device=dev, generator=torch.Generator(device=dev).manual_seed(4))
    big = big.to(torch.bfloat16)
    nb = big.numel()
    q8, s8 = kv.int8_legacy_quant(big)
    ms_lq, _, _ = time_steps(torch, lambda: kv.int8_legacy_quant(big), steps, warmup)
    ms_ld, _, _ = time_steps(torch, lambda: kv.int8_legacy_dequant(q8, s8), steps, warmup)
    del q8
    c8, sc8 = kv.fp8_quant_heads(big)
    ms_hq, _, _ = time_steps(torch, lambda: kv.fp8_quant_heads(big), steps, warmup)
    ms_hq2, _, _ = time_steps(torch, lambda: kv.fp8_quant_heads(big, two_pass=True), steps, warmup)
    ms_hd, _, _ = time_steps(torch, lambda: kv.fp8_dequant_heads(c8, sc8), steps, warmup)
    del c8, big
    torch.cuda.empty_cache()
    tb = lambda b_el, ms: round(b_el * nb / (ms * 1e-3) / 1e12, 3)  # noqa: E731
    res["at_size"] = {
        "elements": nb, "dtype": "bf16",
        "int8_legacy_quant": {"ms": round(ms_lq, 4), "TBps_alg": tb(3, ms_lq), "TBps_moved": tb(5, ms_lq)},
        "int8_legacy_dequant": {"ms": round(ms_ld, 4), "TBps_alg": tb(3, ms_ld)},
        "fp8_quant_heads": {"ms": round(ms_hq, 4), "TBps_alg": tb(3, ms_hq),
                            "frac": round(tb(3, ms_hq) * 1e3 / HBM_PEAK_GBPS, 4),
                            "path": "single pass (heads_fused_kernel): 3 B/el moved"},
        "fp8_quant_heads_two_pass": {"ms": round(ms_hq2, 4), "TBps_alg": tb(3, ms_hq2), "TBps_moved": tb(5, ms_hq2)},
        "fp8_dequant_heads": {"ms": round(ms_hd, 4), "TBps_alg": tb(3, ms_hd)},
        "note": "3 B/el algorithmic everywhere; the int8 legacy quant and the FP8 two-pass quant move 5 B/el "
                "(amax pass 2 B/el + quant pass 2 B/el read, 1 written), the FP8 single pass 3 B/el; times are "
                "whole calls (HIP events), kernel-only figures in profiles/fp8_heads_single_pass.md"}
    log(f"configs[0] functions at 1 Gi elements: int8 quant {ms_lq:.3f} ms, dequant {ms_ld:.3f} ms; fp8 heads quant "
        f"{ms_hq:.3f} ms (two passes {ms_hq2:.3f} ms), dequant {ms_hd:.3f} ms")
    log(f"configs[0]: GPU fp8 {ms_f:.4f} ms, int8 per slab {ms_i:.4f} ms (loop {ms_il:.3f} ms); CPU {threads} threads fp8 "
        f"{cpu[threads][0]:.3f} s, 1 thread {cpu[1][0]:.3f} s; GPU == CPU: {same}, {same_i8}")
    return res


MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16 on MI355X


def make_ring_workload(torch, dev, seed=7):
    """4 sequences x 8,192 tokens at the Llama-3-8B attention shape (32 query heads over 8 KV
    heads, D = 128, page 16): random FP8 codes (no NaN codes), pages at random in the pool,
    fp32 scales, N(0,1) bf16 queries, every sequence's queries at positions 0..8191."""
    B, T, Hq, H, D, P = 4, 8192, 32, 8, 128, 16
    n_pages = B * T // P
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 256, (n_pages, 2, H, P, D), dtype=torch.uint8, generator=g)
    codes[(codes & 0x7F) == 0x7F] = 0x3A  # no NaN codes, as the quantizer writes none
    bt_h = torch.randperm(n_pages, generator=g).to(torch.int32).view(B, T // P)
    sc_h = torch.rand((2, H), generator=g) * 0.01 + 0.001
    q_h = torch.randn((B * T, Hq, D), generator=g).to(torch.bfloat16)
    return dict(B=B, T=T, Hq=Hq, H=H, D=D, P=P, codes=codes, bt_host=bt_h, scales_host=sc_h, q_host=q_h,
                pool=codes.to(dev), bt=bt_h.to(dev), scales=sc_h.to(dev), q=q_h.to(dev),
                cu=torch.arange(0, B * T + 1, T, dtype=torch.int32, device=dev),
                q_pos0=torch.zeros(B, dtype=torch.int32, device=dev),
                kv_len=torch.full((B,), T, dtype=torch.int32, device=dev))


def ring_attention_leg(torch, dev, steps, warmup, skip_cpu):
    """Ring attention straight from the FP8 pages (QuantizedRingAttention's compute,
    README.md:344): 4 sequences x 8,192 tokens, causal, 32 query heads over 8 KV heads,
    D = 128, page 16, pages at random in the pool; ring degree 1 (one step over all keys)
    and 8 (eight key shards merged through the running log-sum-exp, as the ring's steps
    would run on one GPU)."""
    import numpy as np
    from oracle import oracle as O
    from zenyx_amd import kv

    R = make_ring_workload(torch, dev)
    B, T, Hq, D = R["B"], R["T"], R["Hq"], R["D"]
    codes, bt_h, sc_h, q_h = R["codes"], R["bt_host"], R["scales_host"], R["q_host"]
    pool, bt, sc, q, cu, qp, kl = R["pool"], R["bt"], R["scales"], R["q"], R["cu"], R["q_pos0"], R["kv_len"]
    out = torch.empty_like(q)
    flops = 4.0 * B * Hq * D * (T * (T + 1) / 2)  # QK^T and PV over the causal (row, key) pairs
    res = {"workload": "ring attention from FP8 pages: 4 seqs x 8192 tokens causal, 32 query heads over 8 KV "
                       "heads, D=128, page 16 (Llama-3-8B attention shape); kernel paged_prefill_mfma",
           "useful_flop_per_step": flops,
           "note": "peak: the 2.5 PFLOP/s dense bf16/fp16 MFMA figure; with precision 'exact' P.V runs twice "
                   "(P as bf16 hi + lo), so the matrix cores execute 1.5x the useful flops"}
    p_desc = {"f16": "P x 2^7 rounded once to fp16, V fp16 (error <= 1 ulp + 2^-10 max|V|)",
              "bf16": "P rounded once to bf16 (error <= 1 ulp + 2^-7 max|V|)",
              "exact": "P as bf16 hi + lo, two products (error <= 1 ulp + 2^-15 max|V|; measured within 2^-17)"}
    for key, ring, single, prec in (("ring1", 1, True, "f16"), ("ring8", 8, True, "f16"),
                                    ("ring8_steps", 8, False, "f16"), ("ring1_exact", 1, True, "exact"),
                                    ("ring8_exact", 8, True, "exact"), ("ring1_bf16p", 1, True, "bf16")):
        fn = lambda: kv.ring_attention_fp8(q, cu, qp, pool, sc, bt, kl, ring_degree=ring, causal=True,  # noqa: E731
                                           single_launch=single, precision=prec, max_q_per_seq=T)
        # the first ~15-25 launches of a leg run slower while the GPU's clock rises: each
        # launch takes the same number of cycles (GRBM_GUI_ACTIVE ~44 M summed over the
        # XCDs) while the duration falls from ~3.0 ms to ~2.4 ms (about 1.86 -> 2.28 GHz per
        # XCD); at least 25 warm-up calls, so the timed calls run at the settled clock
        ms, _, _ = time_steps(torch, fn, steps, max(warmup, 25))
        tf = flops / (ms * 1e-3) / 1e12
        how = "one launch walking the shards" if single else "one launch per shard, merged through HBM"
        log(f"ring attention degree {ring} ({how}; {p_desc[prec]}): {ms:.3f} ms/step, {tf:.1f} TFLOP/s "
            f"({100 * tf / MFMA_BF16_PEAK_TFLOPS:.1f}% of the bf16 MFMA peak)")
        res[key] = {"ms_per_step": round(ms, 4), "TFLOPs": round(tf, 1), "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                    "launches": "1" if single else str(ring), "precision": prec, "p_in_pv": p_desc[prec]}
    if not skip_cpu:
        # the C oracle (double precision, one thread) on the last 16 query rows of sequence 0
        # (about 20 s on one host core)
        rows = 16
        qs = q_h[T - rows:T].contiguous().view(torch.int16).numpy().view(np.uint16)
        t0 = time.perf_counter()
        O.paged_attention_prefill(qs, np.array([0, rows], np.int32), np.array([T - rows], np.int32),
                                  codes.numpy(), sc_h.numpy(), bt_h[:1].numpy(), np.zeros(1, np.int32),
                                  np.full(1, T, np.int32), True, float(np.float32(1.0 / np.sqrt(D))))
        dt = time.perf_counter() - t0
        f_s = 4.0 * Hq * D * sum(T - rows + r + 1 for r in range(rows))
        res["cpu_baseline"] = {"value": round(f_s / dt / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
                               "sample": f"oracle zxo_paged_attention_prefill, last {rows} query rows of one "
                                         f"sequence (keys 0..8191, 32 heads): {dt:.2f} s"}
        log(f"CPU oracle: {res['cpu_baseline']['value']:.6f} TFLOP/s ({dt:.2f} s)")
    del pool, q, out, R
    torch.cuda.empty_cache()
    return res


def make_c5_layer(torch, dev, layer, out, seed=5, chunk=65536):
    """configs[4] KV of one layer, [B*Tb, 2, H, D] bf16 written into ``out``: Student-t
    (nu = 3) draws times a per-(kv, head, channel) scale 10**U(-2, 2), generated on the
    device from seed (seed, layer)."""
    g = torch.Generator(device=dev).manual_seed(seed * 1000 + layer)
    ch = 10.0 ** (torch.rand((2, C5["H"], C5["D"]), device=dev, generator=g) * 4 - 2)
    T = out.shape[0]
    for t0 in range(0, T, chunk):
        n = min(chunk, T - t0)
        shape = (n, 2, C5["H"], C5["D"])
        z = torch.randn(shape, device=dev, generator=g)
        chi2 = torch.randn((3,) + shape, device=dev, generator=g).square_().sum(0)  # chi-square, 3 dof
        out[t0:t0 + n] = (z * torch.rsqrt(chi2 / 3.0) * ch).to(torch.bfloat16)
    return out


def configs4_setup(torch, dev, timing=False, hbm_layers=None, layers=None, tokens=None):
    """configs[4]'s buffers: block tables (seed 5), the per-layer input, the gather outputs
    and the 80-layer cache streamed through ``hbm_layers`` (default 60) HBM slots and
    pinned DRAM.  ``layers`` and ``tokens`` (per sequence) override the layer count and
    the 131,072 tokens of each of the 4 sequences."""
    from zenyx_amd.train.kv_layer_stream import LayerStreamedKVCache

    L, H, D, P, B, Tb, S = (C5[k] for k in ("L", "H", "D", "P", "B", "Tb", "hbm_layers"))
    S = hbm_layers or S
    L = layers or L
    Tb = tokens or Tb
    T = B * Tb
    n_pages = T // P
    g = torch.Generator().manual_seed(5)
    bt_h = torch.randperm(n_pages, generator=g).to(torch.int32).view(B, Tb // P)
    return dict(bt_host=bt_h, bt=bt_h.to(dev), cu=torch.arange(0, T + 1, Tb, dtype=torch.int32, device=dev),
                sl=torch.full((B,), Tb, dtype=torch.int32, device=dev),
                x=torch.empty((T, 2, H, D), dtype=torch.bfloat16, device=dev),
                kout=torch.empty((B, H, Tb, D), dtype=torch.bfloat16, device=dev),
                vout=torch.empty((B, H, Tb, D), dtype=torch.bfloat16, device=dev),
                cache=LayerStreamedKVCache(L, S, n_pages, H, D, P, device=dev, timing=timing),
                T=T, n_pages=n_pages, L=L, Tb=Tb)


def configs4_step(torch, dev, c, on_gather=None):
    """One configs[4] step: forward (generate layer l's KV on the device, append it) for
    l = 0 .. 79, then backward (gather + dequant) for l = 79 .. 0, through the streamed
    cache; ``on_gather(l, k, v)`` runs on the compute stream after each gather."""
    cache = c["cache"]
    cache.reset()
    for l in range(c["L"]):
        make_c5_layer(torch, dev, l, c["x"])
        cache.append_layer(l, c["x"], c["cu"], c["bt"])
    for l in range(c["L"] - 1, -1, -1):
        k, v = cache.gather_layer(l, c["bt"], c["sl"], c["Tb"], out=(c["kout"], c["vout"]))
        if on_gather is not None:
            on_gather(l, k, v)


def configs4_leg(torch, dev, hbm_layers=None, tokens=None):
    """70B-shape share, 80 layers x (4 x 128k tokens), streamed through 60 HBM
    layer slots and pinned DRAM (zenyx_amd.train.kv_layer_stream.LayerStreamedKVCache).
    ``hbm_layers`` and ``tokens`` (per sequence) change the slot count and the layer size:
    with few slots most layers go out and come back, PCIe sets the pace and the step's wall
    time is to be compared with the copies alone.
    Forward: each layer's KV is generated, appended (dynamic per-head FP8) into its slot;
    layers 0-19 (the Belady victims of the backward sweep) are written back to pinned host
    memory on a side stream right after their own append, and layer l >= 60 reuses layer
    l - 60's slot once that copy is done.  Backward (79 -> 0): every layer is gathered +
    dequantised; the slot a gather frees immediately receives the H2D prefetch of the
    spilled layer 60 positions later in the sweep.  Per-kernel times come from HIP events
    on the compute stream; tier moves from events on the side stream."""
    L, H, D, P, B, Tb, S = (C5[k] for k in ("L", "H", "D", "P", "B", "Tb", "hbm_layers"))
    S = hbm_layers or S
    Tb = tokens or Tb
    c = configs4_setup(torch, dev, timing=True, hbm_layers=S, tokens=Tb)
    T, n_pages, cache = c["T"], c["n_pages"], c["cache"]
    N = T * 2 * H * D
    alg_append = 3 * N + 4 * 2 * H + 4 * n_pages + 4 * (B + 1)
    alg_gather = 3 * N + 4 * n_pages + 4 * 2 * H + 4 * B

    log(f"configs[4]: {S} HBM slots, 4 x {Tb} tokens; warm-up step (80 layers forward + backward)")
    configs4_step(torch, dev, c)
    torch.cuda.synchronize(dev)
    cache.check_errors()
    log("configs[4]: timed step")
    t0 = time.perf_counter()
    configs4_step(torch, dev, c)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    ms = lambda evs: [a.elapsed_time(b) for a, b in evs]  # noqa: E731
    app_ms, gat_ms = ms(cache.events["append"]), ms(cache.events["gather"])
    # the library's choice: one pass when a CU's share of a slab (16-byte vectors) is between
    # half and twice the 5 x 960 its registers hold and the call has >= 32 slabs
    share = -(-T // torch.cuda.get_device_properties(dev).multi_processor_count) * (D // 8)
    append_path = ("two-pass (one layer, 16 slabs per call)" if 2 * H < 32 else
                   "single pass" if 2 * share >= 5 * 960 and share <= 2 * 5 * 960 else "two-pass")
    d2h_ms, h2d_ms = ms(cache.events["d2h"]), ms(cache.events["h2d"])
    a_gbps = L * alg_append / (sum(app_ms) * 1e-3) / 1e9
    g_gbps = L * alg_gather / (sum(gat_ms) * 1e-3) / 1e9
    moved = (L - S) * cache.layer_bytes
    med = lambda v: sorted(v)[len(v) // 2]  # noqa: E731
    out = {"workload": f"configs[4]: 80 layers, 8 KV heads, D=128, 4 x {Tb} tokens, Student-t(3) KV x "
                       f"per-channel 10**U(-2,2); {S} layer slots in HBM ({S * cache.layer_bytes / 1e9:.1f} GB), "
                       f"{L - S} layers spilled to pinned DRAM ({L * cache.layer_bytes / 1e9:.1f} GB of FP8 KV in all)",
           "append_GBps": round(a_gbps, 2), "append_frac": round(a_gbps / HBM_PEAK_GBPS, 4),
           "append_ms_per_layer": round(sum(app_ms) / L, 4), "append_path": append_path,
           "gather_GBps": round(g_gbps, 2), "gather_frac": round(g_gbps / HBM_PEAK_GBPS, 4),
           "gather_ms_per_layer": round(sum(gat_ms) / L, 4),
           "append_ms_median": round(med(app_ms), 4), "append_ms_min": round(min(app_ms), 4),
           "gather_ms_median": round(med(gat_ms), 4), "gather_ms_min": round(min(gat_ms), 4),
           "d2h_GBps": round(moved / (sum(d2h_ms) * 1e-3) / 1e9, 2),
           "h2d_GBps": round(moved / (sum(h2d_ms) * 1e-3) / 1e9, 2),
           "tier_bytes_each_way": moved, "step_wall_s": round(wall, 3),
           "copies_only_s": round((sum(d2h_ms) + sum(h2d_ms)) * 1e-3, 3),
           "hbm_slot_bytes": S * cache.layer_bytes, "cache_bytes": L * cache.layer_bytes,
           "streaming_ratio": round(L / S, 2), "kernels_s": round((sum(app_ms) + sum(gat_ms)) * 1e-3, 4),
           "note": "KV generation (Student-t sampling) runs inside the step and is not in the kernel times"}
    log(f"configs[4]: append {a_gbps:.1f} GB/s ({100 * a_gbps / HBM_PEAK_GBPS:.1f}%), gather {g_gbps:.1f} GB/s "
        f"({100 * g_gbps / HBM_PEAK_GBPS:.1f}%), D2H {out['d2h_GBps']} GB/s, H2D {out['h2d_GBps']} GB/s, "
        f"step {wall:.2f} s; per layer append median {med(app_ms):.3f} ms (min {min(app_ms):.3f}), gather median "
        f"{med(gat_ms):.3f} ms (min {min(gat_ms):.3f})")
    del c, cache
    torch.cuda.empty_cache()
    return out


def decode_loop_leg(torch, dev, steps=100, warmup=5, n_seqs=64, ctx=32768, n_layers=4):
    """Decode loop through the drop-in classes (PagedFP8KVCache + QuantizedRingAttention):
    ``n_seqs`` sequences prefilled to ``ctx`` tokens, then ``steps`` decode steps, each one
    append of one token per sequence (all layers, static scales) plus decode attention
    for every layer (32 query heads over 8 KV heads, D = 128).  Reports the wall time per
    step, the host time to issue a step (the drop-in's bookkeeping and launches; the
    calls do not synchronise) and the device time per step from HIP events (whole steps,
    kernels back to back when the host keeps ahead).  ``n_layers`` of the model's 32 keep
    the cache at ~17 GB; every layer adds the same work per step."""
    from zenyx_amd.train.fp8_kv_quantization import PagedFP8KVCache, QuantizedRingAttention

    H, D, P, Hq = 8, 128, 16, 32
    per_seq = -(-(ctx + warmup + steps + 10) // P)
    cache = PagedFP8KVCache(n_layers, H, D, num_pages=n_seqs * per_seq, page_size=P, device=dev,
                            overflow="saturate")
    seqs = list(range(n_seqs))
    g = torch.Generator(device=dev).manual_seed(17)
    x = torch.randn((n_layers, n_seqs * ctx, 2, H, D), device=dev, generator=g, dtype=torch.bfloat16)
    t0 = time.perf_counter()
    cache.append(x, seqs, [ctx] * n_seqs, check=True)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    del x
    torch.cuda.empty_cache()
    xs = torch.randn((warmup + steps + 10, n_layers, n_seqs, 2, H, D), device=dev, generator=g, dtype=torch.bfloat16)
    qs = torch.randn((warmup + steps + 10, n_layers, n_seqs, Hq, D), device=dev, generator=g, dtype=torch.bfloat16)
    att = QuantizedRingAttention(cache, check=False)
    ones = [1] * n_seqs

    def step(i):
        cache.append(xs[i], seqs, ones)
        for layer in range(n_layers):
            att.decode(qs[i, layer], layer, seqs)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    t0 = time.perf_counter()
    ev[0].record(st)
    host = 0.0
    for i in range(steps):
        h0 = time.perf_counter()
        step(warmup + i)
        host += time.perf_counter() - h0
        ev[i + 1].record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    # the host's own cost of a step: issued right after a synchronisation, so no launch
    # waits for room in the device's queue (in the loop above the host runs ahead of the
    # device until the queue is full, and from then on every launch waits for the device)
    issue = []
    for i in range(warmup + steps, warmup + steps + 10):
        torch.cuda.synchronize()
        h0 = time.perf_counter()
        step(i)
        issue.append(time.perf_counter() - h0)
    torch.cuda.synchronize()
    issue.sort()
    cache.check_errors()
    out = {"workload": f"decode loop through PagedFP8KVCache + QuantizedRingAttention.decode: {n_seqs} seqs "
                       f"prefilled to {ctx} tokens, {n_layers} layers (8 KV heads, D=128, page 16, 32 query "
                       f"heads), {steps} steps of append(1 token per seq) + decode attention per layer",
           "wall_ms_per_step": round(1e3 * wall / steps, 4), "device_ms_per_step": round(sum(gpu) / steps, 4),
           "device_ms_per_step_min": round(min(gpu), 4),
           "host_issue_ms_per_step": round(1e3 * issue[len(issue) // 2], 4),
           "host_ms_per_step_in_loop": round(1e3 * host / steps, 4),
           "prefill_append_s": round(prefill_s, 3), "saturated_appends": cache.saturated_appends}
    log(f"decode loop: {out['wall_ms_per_step']:.3f} ms/step wall, device {out['device_ms_per_step']:.3f} ms/step, "
        f"host issue {out['host_issue_ms_per_step']:.3f} ms/step ({n_layers} layers)")
    del cache, xs, qs, att
    torch.cuda.empty_cache()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: the KV hot path is benchmarked on a "
                          "single MI355X (how the path shards over GPUs is designed, not run)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from zenyx_amd import kv

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    out = {"metric": METRIC, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
           "data": "synthetic (seeded N(0,1) bf16 KV, random page tables)"}

    if args.only == "copy":
        # Counter calibration: one plain device-to-device copy of exactly 4 GiB per step, so
        # rocprofv3's FETCH_SIZE / WRITE_SIZE per dispatch can be compared with known bytes.
        src = torch.randint(0, 255, (4 << 30,), dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        ms_c, _, _ = time_steps(torch, lambda: dst.copy_(src), args.steps, args.warmup)
        out.update({"value": round(2 * src.numel() / (ms_c * 1e-3) / 1e9, 2), "ms_per_step": round(ms_c, 4),
                    "config": {"workload": "calibration: torch copy_ of 4 GiB (4 GiB read + 4 GiB written)"}})
        print(json.dumps(out), flush=True)
        return

    if args.only in ("append", "all"):
        log("building configs[1] append workload")
        W = make_append_workload(torch, dev, seed=args.seed)
        scales = torch.empty((W["L"], 2, W["H"]), dtype=torch.float32, device=dev)

        def step():
            kv.kv_quant_append(W["x"], W["cu"], W["bt"], W["pool"], scales=scales)

        log(f"append: {W['T']} tokens x 32 layers = {W['N']} elements; timing {args.steps} steps")
        ms, per, wall = time_steps(torch, step, args.steps, args.warmup)
        gbps = W["alg_bytes"] / (ms * 1e-3) / 1e9
        log(f"append: {ms:.3f} ms/step, {gbps:.1f} GB/s ({100 * gbps / HBM_PEAK_GBPS:.1f}% of peak)")
        out.update({
            "value": round(gbps, 2), "ms_per_step": round(ms, 4),
            "config": {"workload": "configs[1]: paged append + fused FP8 e4m3 quant, Llama-3-8B KV shape "
                                   "(32 layers, 8 KV heads, D=128, page 16, 16 seqs U[1k,8k], 5% heads x50)",
                       "n_tok": W["T"], "elements": W["N"], "n_pages_per_layer": W["n_pages"],
                       "algorithmic_bytes_per_step": W["alg_bytes"], "seed": args.seed},
            "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4),
                         "traffic": MEASURED_TRAFFIC.get(("append", args.seed)),
                         "traffic_source": TRAFFIC_SOURCE if ("append", args.seed) in MEASURED_TRAFFIC else None,
                         "kernel": "kv_append_fused_kernel (HIP events around the whole zx_kv_quant_append "
                                   "call: token offsets + fills + the fused kernel)"},
        })
        if not args.skip_cpu:
            log("CPU baseline (append)")
            out["cpu_baseline"] = cpu_baseline_append(W)
        del W
        torch.cuda.empty_cache()

    if args.only in ("gather", "all"):
        log("building configs[2] gather workload")
        G = make_gather_workload(torch, dev)
        k = torch.empty((G["B"], G["H"], G["T"], G["D"]), dtype=torch.bfloat16, device=dev)
        v = torch.empty_like(k)
        sc = G["scales"][G["layer"]].contiguous()

        def gstep():
            kv.kv_gather_dequant(G["pool"], sc, G["bt"], G["seq_lens"], G["T"], out=(k, v))

        ms_g, _, _ = time_steps(torch, gstep, args.steps, args.warmup)
        gb_g = G["alg_bytes"] / (ms_g * 1e-3) / 1e9
        log(f"gather: {ms_g:.3f} ms/step, {gb_g:.1f} GB/s ({100 * gb_g / HBM_PEAK_GBPS:.1f}% of peak)")
        gather = {"GBps": round(gb_g, 2), "ms_per_step": round(ms_g, 4), "frac": round(gb_g / HBM_PEAK_GBPS, 4),
                  "traffic": MEASURED_TRAFFIC.get(("gather", 2)), "traffic_source": TRAFFIC_SOURCE,
                  "workload": "configs[2]: paged gather + dequant, 64 seqs x 32768, 300k-page pool, one layer K+V",
                  "algorithmic_bytes_per_step": G["alg_bytes"]}
        if not args.skip_cpu:
            log("CPU baseline (gather)")
            gather["cpu_baseline"] = cpu_baseline_gather(G)
        # decode attention straight from the same FP8 pages (one query token per sequence,
        # 32 query heads over the 8 KV heads, as Llama-3-8B)
        Hq = 32
        qd = torch.randn((G["B"], Hq, G["D"]), device=dev, generator=torch.Generator(device=dev).manual_seed(3))
        qd = qd.to(torch.bfloat16)
        od = torch.empty_like(qd)
        astep = lambda: kv.paged_attention_decode(qd, G["pool"], sc, G["bt"], G["seq_lens"], out=od)
        # its first few dozen launches after the gather leg run ~10% slower (measured
        # 0.885 ms at 3 warm-up steps, 0.786 ms at 40): time the steady state
        ms_a, _, _ = time_steps(torch, astep, args.steps, max(args.warmup, 40))
        alg_a = G["N"] + 4 * G["B"] * (G["T"] // G["P"]) + 4 * 2 * G["H"] + 2 * 2 * G["B"] * Hq * G["D"]
        gb_a = alg_a / (ms_a * 1e-3) / 1e9
        log(f"attention decode from FP8 pages: {ms_a:.3f} ms/step, {gb_a:.1f} GB/s ({100 * gb_a / HBM_PEAK_GBPS:.1f}% "
            f"of peak)")
        gather["attention_decode"] = {
            "GBps": round(gb_a, 2), "ms_per_step": round(ms_a, 4), "frac": round(gb_a / HBM_PEAK_GBPS, 4),
            "algorithmic_bytes_per_step": alg_a,
            "workload": "paged_decode_mfma/combine: 64 seqs x 32768 positions, 32 query heads over 8 KV heads, "
                        "D=128, reading the configs[2] pool (1 B per K/V element)"}
        del qd, od
        out["gather_dequant"] = gather
        if "value" not in out:
            out.update({"value": round(gb_g, 2), "ms_per_step": round(ms_g, 4),
                        "config": {"workload": gather["workload"]}})
        del G, k, v
        torch.cuda.empty_cache()

    if args.only in ("decode", "all"):
        out["decode_loop"] = decode_loop_leg(torch, dev)
        if "value" not in out:
            d = out["decode_loop"]
            out.update({"value": round(1e3 / d["wall_ms_per_step"], 2), "unit": "steps/s",
                        "ms_per_step": d["wall_ms_per_step"], "config": {"workload": d["workload"]}})

    if args.only in ("configs0", "all"):
        out["configs0"] = configs0_leg(torch, dev, args.steps, args.warmup)
        if "value" not in out:
            c = out["configs0"]
            out.update({"value": c["gpu"]["fp8_heads_GBps"], "ms_per_step": c["gpu"]["fp8_heads_ms"],
                        "config": {"workload": c["workload"]}})

    if args.only in ("ring", "all"):
        out["ring_attention"] = ring_attention_leg(torch, dev, args.steps, args.warmup, args.skip_cpu)
        if "value" not in out:
            r = out["ring_attention"]
            out.update({"value": r["ring1"]["TFLOPs"], "unit": "TFLOP/s", "ms_per_step": r["ring1"]["ms_per_step"],
                        "dtype": "bf16", "config": {"workload": r["workload"]},
                        "roofline": {"bound": "mfma", "achieved": r["ring1"]["TFLOPs"],
                                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": r["ring1"]["frac"],
                                     "traffic": None, "kernel": "paged_prefill_mfma_kernel<4>"}})
            if "cpu_baseline" in r:
                out["cpu_baseline"] = r["cpu_baseline"]

    if args.only in ("belady", "all"):
        out["belady"] = belady_leg(torch, dev, args.skip_cpu)
        if "value" not in out:
            b = out["belady"]
            out.update({"value": b["evictions_per_s"], "unit": "evictions/s",
                        "ms_per_step": b["simulate_ms"], "config": {"workload": b["workload"]}})

    if args.only in ("weights", "all"):
        out["weight_streaming"] = weights_leg(torch, dev)
        if "value" not in out:
            w = out["weight_streaming"]
            out.update({"value": w["h2d_GBps"], "ms_per_step": w["pipelined_ms"],
                        "config": {"workload": w["workload"]}})

    if args.only == "tiers":
        out["three_tier"] = tiers_leg(torch, dev)
    elif args.only == "all":
        # in a child process: 64 GB of T0 slots and 32 GiB of pinned T1 slots
        import subprocess

        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--only", "tiers", "--skip-cpu"],
                           stdout=subprocess.PIPE, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"three-tier leg failed with exit code {r.returncode}")
        out["three_tier"] = json.loads(r.stdout.strip().splitlines()[-1])["three_tier"]

    if args.only == "configs4_16gb":
        # Switched off: its first run (65 pinned host buffers of 1 GiB, 15 HBM slots) ended in
        # a segmentation fault of the process during the warm-up step, and the cause has not
        # been shown; configs4_leg(torch, dev, hbm_layers=15) is the code it ran.
        raise SystemExit("configs4_16gb is switched off: its first run crashed (segmentation fault) and the cause "
                         "is not known")
    if args.only == "stream":
        # configs[4]'s 80-layer step at a streaming ratio of 40:1 (README.md:154 claims 32:1):
        # layers of 4 x 32,768 tokens (268 MB), 2 HBM slots, 78 layers through pinned DRAM
        # (21 GB, the pinned footprint of the 60-slot configs[4] leg)
        out["stream"] = configs4_leg(torch, dev, hbm_layers=2, tokens=32768)
    elif args.only == "all":
        import subprocess  # a child process, like configs[4]: 21 GB of pinned memory

        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--only", "stream", "--skip-cpu"],
                           stdout=subprocess.PIPE, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"streaming leg failed with exit code {r.returncode}")
        out["stream"] = json.loads(r.stdout.strip().splitlines()[-1])["stream"]
    if args.only == "configs4":
        out["configs4"] = configs4_leg(torch, dev)
    elif args.only == "all":
        # in a child process: the leg allocates 64 GB of slots plus 21.5 GB of pinned memory,
        # and after the other legs' allocations its kernels measured ~10% slower in-process
        import subprocess

        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--only", "configs4", "--skip-cpu"],
                           stdout=subprocess.PIPE, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"configs[4] leg failed with exit code {r.returncode}")
        out["configs4"] = json.loads(r.stdout.strip().splitlines()[-1])["configs4"]
    if args.only == "tiers" and "value" not in out:
        t = out["three_tier"]
        out.update({"value": round(t["plan"]["accesses"] / (t["plan"]["gpu_plan_s"] + t["plan"]["host_slots_s"]), 1),
                    "unit": "accesses planned/s", "ms_per_step": round(1e3 * t["plan"]["gpu_plan_s"], 3),
                    "config": {"workload": t["workload"]}})
    if args.only == "configs4_16gb" and "value" not in out:
        c = out["configs4_16gb"]
        out.update({"value": c["append_GBps"], "ms_per_step": round(1e3 * c["step_wall_s"], 3),
                    "config": {"workload": c["workload"]}})
    if args.only == "stream" and "value" not in out:
        c = out["stream"]
        out.update({"value": round(2 * c["tier_bytes_each_way"] / c["step_wall_s"] / 1e9, 2),
                    "unit": "GB/s through PCIe (both ways, whole step)", "ms_per_step": round(1e3 * c["step_wall_s"], 3),
                    "config": {"workload": c["workload"]}})
    if args.only in ("configs4", "all"):
        if "value" not in out:
            c = out["configs4"]
            out.update({"value": c["append_GBps"], "ms_per_step": round(c["append_ms_per_layer"] * C5["L"], 4),
                        "config": {"workload": c["workload"]}})

    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
