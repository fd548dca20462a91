"""Parity at the benchmark's full sizes, on the exact workloads bench.py times.

* configs[1] (seed 1: 32 layers x 74,902 tokens, 8 KV heads, D = 128, page 16, outlier
  heads x50): one fused append of all layers; all 512 scales bit-exact against the C
  oracle's amax over each whole layer, and every layer's pool (every code of all 32
  layers) against the oracle's torch restatement of the append.
* configs[2] (64 x 32,768 positions, 300,000-page pool): the full gather, every gathered
  bf16 of all 64 sequences (K and V) bit-exact against the oracle's torch restatement.
* the decode attention over the same pool, two whole sequences checked against the
  oracle within the stated tolerance (one bf16 ulp plus 2^-17 max|V|).
* ring attention at bench.py's ring workload (4 x 8,192 causal): 128 rows (blocks of 8
  consecutive rows spread over the causal range of every sequence) against the oracle
  at ring degree 1 and 8, and ring 8 against ring 1 on every output.
* configs[3] (1M tokens, 80 layers, ring 8, 64 GB budget: 20,971,520 accesses): the whole
  Belady schedule of the GPU simulator -- every eviction's position and page, and the
  miss flags of every access -- against the C heap oracle.
* the ring curriculum of bench.py (ring 2 / 256k, 4 / 512k, 8 / 1M tokens, 80 layers:
  27,525,120 accesses): the GPU-built page trace against the oracle's, and the whole
  Belady schedule over it against the C heap oracle.
"""
import numpy as np
import pytest
import torch

import bench
from oracle import oracle as O
from zenyx_amd import kv
from test_gpu_attention import assert_within_bound, assert_within_one_ulp

pytestmark = pytest.mark.gpu


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def test_configs1_full_append(dev):
    """all 32 layers' 16 scales against the C oracle's amax over each whole
    layer, and every layer's pool (4,688 pages, every code) against the torch restatement
    of the append (bit-identical to the C oracle, tests/test_oracle.py)."""
    W = bench.make_append_workload(torch, dev, seed=1)
    print(f"configs[1]: {W['T']} tokens x {W['L']} layers", flush=True)
    sc = kv.kv_quant_append(W["x"], W["cu"], W["bt"], W["pool"], check=True)
    torch.cuda.synchronize()
    L, H, P = W["L"], W["H"], W["P"]
    cu, bt = W["cu_host"].numpy(), W["bt_host"].numpy()
    got_sc = sc.cpu().numpy()
    for layer in range(L):
        x_l = W["x"][layer].cpu()  # [T, 2, H, D]
        wsc = O.kv_scales(x_l.view(torch.int16).numpy().view(np.uint16)[None])[0]
        np.testing.assert_array_equal(got_sc[layer].view(np.uint32), wsc.view(np.uint32))
        wsc_t, wpool = O.kv_quant_append_torch(x_l, cu, bt, W["n_pages"], P)
        np.testing.assert_array_equal(got_sc[layer].view(np.uint32), wsc_t.numpy().view(np.uint32))
        gpool = W["pool"][layer].cpu()
        assert torch.equal(gpool, wpool), f"layer {layer}: {(gpool != wpool).sum().item()} codes differ"
    print(f"all {L * 2 * H} scales and every code of all {L} layers ({W['pool'].numel()} bytes) bit-exact",
          flush=True)


def test_configs2_full_gather_and_attention(dev):
    G = bench.make_gather_workload(torch, dev)
    B, H, D, P, T = G["B"], G["H"], G["D"], G["P"], G["T"]
    sc = G["scales"][G["layer"]].contiguous()
    k, v = kv.kv_gather_dequant(G["pool"], sc, G["bt"], G["seq_lens"], T, check=True)
    torch.cuda.synchronize()
    bt = G["bt_host"].numpy()
    scl = G["scales_host"][G["layer"]].numpy()
    pool_host = G["pool"].cpu()
    lens = G["seq_lens"].cpu().numpy()
    for b in range(B):  # every gathered value, one sequence at a time
        wk, wv = O.kv_gather_dequant_torch(pool_host, torch.from_numpy(scl), bt[b:b + 1], lens[b:b + 1], T)
        for name, got, want in (("K", k[b], wk[0]), ("V", v[b], wv[0])):
            g_ = got.cpu().view(torch.int16)
            w_ = want.view(torch.int16)
            assert torch.equal(g_, w_), f"sequence {b} {name}: {(g_ != w_).sum().item()} values differ"
    print(f"gather: all {B} sequences x {T} positions (K and V, {2 * k.numel()} values) bit-exact", flush=True)
    del k, v, pool_host
    torch.cuda.empty_cache()

    dec = O.e4m3_decode(np.arange(256, dtype=np.uint8))
    Hq = 32
    q = torch.randn((B, Hq, D), generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    out = kv.paged_attention_decode(q.to(dev), G["pool"], sc, G["bt"], G["seq_lens"], check=True)
    torch.cuda.synchronize()
    for b in (0, 40):
        pages = np.unique(bt[b])
        sub = G["pool"][torch.from_numpy(pages.astype(np.int64)).to(dev)].cpu().numpy()
        remap = np.full(bt.max() + 1, -1, np.int64)
        remap[pages] = np.arange(len(pages))
        bt_b = remap[bt[b]][None].astype(np.int32)
        qb = bits16(q[b:b + 1])
        sm = float(np.float32(1.0 / np.sqrt(D)))
        want, err = O.paged_attention_decode(qb, sub, scl, bt_b, np.array([T], np.int32), sm)
        assert err == 0
        vcodes = sub[:, 1]  # [pages, H, P, D]
        vmax = np.abs(dec[vcodes].astype(np.float64)).max(axis=(0, 2)) * scl[1][:, None]  # [H, D]
        vmax_q = np.repeat(vmax, Hq // H, axis=0)[None]  # [1, Hq, D]
        assert_within_one_ulp(bits16(out[b:b + 1]), want, vmax_q)
    print("attention: 2 sequences x 32 heads within tolerance", flush=True)


def test_ring_attention_bench_shape(dev):
    """The ring-attention workload bench.py times (4 x 8,192 causal, 32 query heads over 8
    KV heads): rows at both ends of the causal range against the oracle for ring degree 1
    and 8 in the default precision (P in fp16: within 2 bf16 ulps + 2^-10 max|V| of the
    oracle) and ring 1 in the exact one (one ulp + 2^-17 max|V|), and every element of ring
    8 against ring 1 (within twice the default bound of each other)."""
    R = bench.make_ring_workload(torch, dev)
    T, Hq, H, D, P = R["T"], R["Hq"], R["H"], R["D"], R["P"]
    outs = {}
    for ring in (1, 8):
        outs[ring] = kv.ring_attention_fp8(R["q"], R["cu"], R["q_pos0"], R["pool"], R["scales"], R["bt"],
                                           R["kv_len"], ring_degree=ring, causal=True, check=True)
    # ring 8 as eight launches merged through the fp32 running output (the multi-GPU unit)
    outs["8s"] = kv.ring_attention_fp8(R["q"], R["cu"], R["q_pos0"], R["pool"], R["scales"], R["bt"], R["kv_len"],
                                       ring_degree=8, causal=True, check=True, single_launch=False)
    outs["1x"] = kv.ring_attention_fp8(R["q"], R["cu"], R["q_pos0"], R["pool"], R["scales"], R["bt"], R["kv_len"],
                                       ring_degree=1, causal=True, check=True, precision="exact")
    torch.cuda.synchronize()
    codes, bt, sc = R["codes"].numpy(), R["bt_host"].numpy(), R["scales_host"].numpy()
    dec = np.abs(O.e4m3_decode(np.arange(256, dtype=np.uint8)).astype(np.float64))
    sm = float(np.float32(1.0 / np.sqrt(D)))
    grp = Hq // H
    # per sequence and KV head: running max over keys of |V| per channel
    vmax = np.zeros((R["B"], H, T, D))
    t = np.arange(T)
    for b in range(R["B"]):
        pages = bt[b, t // P]
        for h in range(H):
            vmax[b, h] = np.maximum.accumulate(dec[codes[pages, 1, h, t % P, :]], axis=0) * float(sc[1, h])
    q_bits = bits16(R["q_host"])
    blocks = [(b, r0) for b in range(R["B"]) for r0 in (0, 1000 + 1500 * b, 4096 + 700 * b, T - 8)]
    for b, r0 in blocks:  # 4 blocks of 8 consecutive rows per sequence: 128 rows
        i = b * T + r0
        rows = np.arange(r0, r0 + 8)
        want, _, err = O.paged_attention_prefill(q_bits[i:i + 8], np.array([0, 8], np.int32),
                                                 np.array([r0], np.int32), codes, sc, bt[b:b + 1],
                                                 np.zeros(1, np.int32), np.full(1, T, np.int32), True, sm)
        assert err == 0
        vm = np.repeat(vmax[b][:, rows], grp, axis=0).transpose(1, 0, 2)  # [8, Hq, D]
        for ring in (1, 8, "8s"):
            assert_within_bound(bits16(outs[ring][i:i + 8]), want, vm, 2.0 ** -10, ulps=2)
        assert_within_one_ulp(bits16(outs["1x"][i:i + 8]), want, vm)
    print(f"ring 1, ring 8 (one launch) and ring 8 (eight launches), and ring 1 exact: {8 * len(blocks)} rows x "
          "32 heads within tolerance of the oracle", flush=True)
    for other in (8, "8s"):
        for b in range(R["B"]):  # one sequence at a time (float32 is exact for bf16 values and their differences)
            a = outs[1][b * T:(b + 1) * T].float().cpu().numpy()
            c = outs[other][b * T:(b + 1) * T].float().cpu().numpy()
            vm_b = np.repeat(vmax[b], grp, axis=0).transpose(1, 0, 2).astype(np.float32)  # [T, Hq, D]
            mag = np.maximum(np.maximum(np.abs(a), np.abs(c)), np.float32(2.0 ** -100))
            tol = 4 * np.exp2(np.floor(np.log2(mag)) - 7) + np.float32(2.0 ** -9) * vm_b
            bad = np.abs(a - c) > tol
            assert not bad.any(), f"sequence {b}: {bad.sum()} elements of ring {other} differ from ring 1"
        print(f"ring {other} == ring 1 within tolerance on all 33.5 M outputs", flush=True)


def test_configs3_full_belady_schedule(dev):
    from zenyx_amd.train.belayd_kv_cache_tiering import BeladyKVCacheTieringManager

    m = BeladyKVCacheTieringManager(num_devices=8, context_length=2**20, num_layers=80, num_kv_heads=8,
                                    head_dim=128, page_tokens=64, hbm_budget_bytes=64e9, device=dev)
    print(f"configs[3]: {len(m.sequence)} accesses, {m.n_pages} pages, capacity {m.capacity}", flush=True)
    stats = m.plan()
    trace = O.ring_trace(80, 8, m.pages_per_shard)
    np.testing.assert_array_equal(m.sim.trace.cpu().numpy(), trace)
    pos, page, st, miss = O.belady_simulate(trace, m.n_pages, m.capacity, miss_flags=True)
    assert {k: stats[k] for k in ("evictions", "misses", "hits", "resident")} == st
    gpos, gpage = m.sim.evictions()
    np.testing.assert_array_equal(gpos.numpy(), pos)
    np.testing.assert_array_equal(gpage.numpy(), page)
    np.testing.assert_array_equal(m.sim.miss_flags.cpu().numpy(), miss)


def test_curriculum_full_trace_and_schedule(dev):
    from zenyx_amd.train.dynamic_ring_curriculum import CurriculumPhase, RingDegreeScheduler

    L, pt, page_bytes = 80, 64, 64 * 8 * 128 * 2
    s = RingDegreeScheduler([CurriculumPhase("ring2", 2, 1 << 18, 1), CurriculumPhase("ring4", 4, 1 << 19, 1),
                             CurriculumPhase("ring8", 8, 1 << 20)], num_devices=8)
    n_pages, cap = L * s.layer_stride(pt), int(64e9 // page_bytes)
    trace = s.access_trace([0, 1, 2], L, page_tokens=pt, device=dev)
    want = O.ring_curriculum_trace([2, 4, 8], [4096, 8192, 16384], L, s.layer_stride(pt))
    print(f"curriculum: {want.size} accesses, {n_pages} pages, capacity {cap}", flush=True)
    np.testing.assert_array_equal(trace.cpu().numpy(), want)
    sim = kv.BeladyTraceSim(trace, n_pages, cap, record_misses=True)
    sim.run()
    pos, page, st, miss = O.belady_simulate(want, n_pages, cap, miss_flags=True)
    assert sim.stats() == st
    gpos, gpage = sim.evictions()
    np.testing.assert_array_equal(gpos.numpy(), pos)
    np.testing.assert_array_equal(gpage.numpy(), page)
    np.testing.assert_array_equal(sim.miss_flags.cpu().numpy(), miss)
