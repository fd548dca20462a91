"""configs[4] (70B-shape share, 4 x 131,072 tokens per layer) parity on sampled layers,
appended and gathered on their own, and the whole streamed step bench.py times (80 layers
through 60 HBM slots and pinned DRAM) checked after the backward gather.

Each sampled layer is generated on the device exactly as bench.py's configs[4] leg does
(Student-t(3) x per-channel 10**U(-2, 2)), appended with dynamic scales (the library takes
the two-pass path at this size) and gathered back.  Checks against the C oracle:
  * all 16 scales of the layer, bit-exact (oracle amax over the full layer);
  * the pool bytes of 4,096 sampled token rows (every kv, head and channel), bit-exact:
    the oracle appends the same rows into a compact pool with the oracle's scales;
  * the gathered bf16 of those positions, bit-exact to the oracle's dequant of the codes.
"""
import numpy as np
import pytest
import torch

import bench
from oracle import oracle as O
from zenyx_amd import kv

pytestmark = pytest.mark.gpu


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("layer", [0, 39, 79])
def test_configs4_sampled_layer(dev, layer):
    C = bench.C5
    H, D, P, B, Tb = C["H"], C["D"], C["P"], C["B"], C["Tb"]
    T = B * Tb
    n_pages = T // P
    g = torch.Generator().manual_seed(100 + layer)
    bt = torch.randperm(n_pages, generator=g).to(torch.int32).view(B, Tb // P)
    cu = torch.arange(0, T + 1, Tb, dtype=torch.int32)
    x = torch.empty((T, 2, H, D), dtype=torch.bfloat16, device=dev)
    bench.make_c5_layer(torch, dev, layer, x)
    pool = torch.zeros((n_pages, 2, H, P, D), dtype=torch.uint8, device=dev)
    sc = kv.kv_quant_append(x, cu.to(dev), bt.to(dev), pool, check=True)
    k, v = kv.kv_gather_dequant(pool, sc[0], bt.to(dev), torch.full((B,), Tb, dtype=torch.int32, device=dev),
                                Tb, check=True)

    xb = bits16(x)  # [T, 2, H, D]
    del x
    wsc = O.kv_scales(xb[None])
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), wsc.view(np.uint32))

    rng = np.random.default_rng(layer)
    S = 4096
    tok = np.sort(rng.choice(T, S, replace=False))
    b, pos = tok // Tb, tok % Tb
    page = bt.numpy()[b, pos // P]
    got = pool.cpu().numpy()[page, :, :, pos % P, :]  # [S, 2, H, D]
    compact = np.zeros((1, S // P, 2, H, P, D), np.uint8)
    _, werr = O.kv_quant_append(np.ascontiguousarray(xb[tok])[None], np.array([0, S], np.int32), None,
                                np.arange(S // P, dtype=np.int32)[None], compact, P, scales=wsc)
    assert werr == 0
    want = compact[0].transpose(0, 3, 1, 2, 4).reshape(S, 2, H, D)
    np.testing.assert_array_equal(got, want)

    # gathered values at the sampled positions vs the oracle's dequant of the codes
    codes = np.ascontiguousarray(want.transpose(1, 2, 0, 3)).reshape(2, 1, H, S * D)
    deq = O.fp8_dequant_heads(codes, wsc[0]).reshape(2, H, S, D)
    gk = bits16(k[torch.from_numpy(b).to(dev), :, torch.from_numpy(pos).to(dev)])  # [S, H, D]
    gv = bits16(v[torch.from_numpy(b).to(dev), :, torch.from_numpy(pos).to(dev)])
    for got_kv, want_kv in ((gk, deq[0].transpose(1, 0, 2)), (gv, deq[1].transpose(1, 0, 2))):
        g_nan = (got_kv & 0x7FFF) > 0x7F80
        w_nan = (want_kv & 0x7FFF) > 0x7F80
        np.testing.assert_array_equal(g_nan, w_nan)
        np.testing.assert_array_equal(got_kv[~g_nan], want_kv[~w_nan])


def _oracle_rows(xb, wsc, tok, P):
    """Oracle codes [S, 2, H, D] of token rows xb[tok] under the layer scales wsc [1, 2, H]
    (appended into a compact pool, one position per sampled row) and their dequantised
    bf16 bits [2, H, S, D]."""
    S = len(tok)
    _, _, H, D = xb.shape
    compact = np.zeros((1, S // P, 2, H, P, D), np.uint8)
    _, werr = O.kv_quant_append(np.ascontiguousarray(xb[tok])[None], np.array([0, S], np.int32), None,
                                np.arange(S // P, dtype=np.int32)[None], compact, P, scales=wsc)
    assert werr == 0
    want = compact[0].transpose(0, 3, 1, 2, 4).reshape(S, 2, H, D)
    codes = np.ascontiguousarray(want.transpose(1, 2, 0, 3)).reshape(2, 1, H, S * D)
    return want, O.fp8_dequant_heads(codes, wsc[0]).reshape(2, H, S, D)


def _assert_bf16_bits(got, want):
    g_nan = (got & 0x7FFF) > 0x7F80
    w_nan = (want & 0x7FFF) > 0x7F80
    np.testing.assert_array_equal(g_nan, w_nan)
    np.testing.assert_array_equal(got[~g_nan], want[~w_nan])


def test_configs4_streamed_step(dev):
    """bench.py's configs[4] step end to end (bench.configs4_step over
    LayerStreamedKVCache): layers 0-19 are written back to pinned DRAM after their append,
    their slots reused by layers 60-79, and prefetched back into slots the backward
    gathers freed; layers 20-79 stay resident.  After the backward gather:
      * all 80 layers' 16 scales bit-exact against fp32(max(amax, 1e-8) / 448) of the
        layer's input (amax by torch on the device, exact for bf16; the division by numpy
        in IEEE fp32);
      * the whole gathered K and V of layer 7 (spilled and prefetched back) and layer 60
        (resident): every value bit-exact against the oracle's torch restatement of the
        append followed by its gather;
      * 2,048 sampled (sequence, position) rows of layers 0, 19 and 79 against the C
        oracle."""
    C = bench.C5
    L, H, D, P, B, Tb = C["L"], C["H"], C["D"], C["P"], C["B"], C["Tb"]
    c = bench.configs4_setup(torch, dev)
    cache = c["cache"]
    assert cache.n_spill == 20 and cache.S == 60
    whole = (7, 60)
    sample = (0, 19, 79)
    rng = np.random.default_rng(17)
    S = 2048
    picks = {l: (rng.integers(0, B, S), rng.integers(0, Tb, S)) for l in sample}
    got, got_whole = {}, {}

    def on_gather(layer, k, v):
        if layer in picks:
            b, pos = (torch.from_numpy(a).to(dev) for a in picks[layer])
            got[layer] = (k[b, :, pos].clone(), v[b, :, pos].clone())  # [S, H, D]
        if layer in whole:
            got_whole[layer] = (k.cpu(), v.cpu())  # [B, H, Tb, D] each

    print("configs[4] streamed step: 80 layers forward + backward", flush=True)
    bench.configs4_step(torch, dev, c, on_gather)
    torch.cuda.synchronize()
    cache.check_errors()
    scales = cache.scales.cpu().numpy()
    x = c["x"]
    for layer in range(L):
        bench.make_c5_layer(torch, dev, layer, x)
        amax = x.abs().amax(dim=(0, 3)).float().cpu().numpy()  # [2, H], exact
        want = np.maximum(amax, np.float32(1e-8)).astype(np.float32) / np.float32(448.0)
        np.testing.assert_array_equal(scales[layer].view(np.uint32), want.view(np.uint32))
    print(f"all {L} layers' scales bit-exact", flush=True)
    # identity tables: the gathered values do not depend on which pages hold the codes
    seq_tables = np.arange(B * Tb // P, dtype=np.int32).reshape(B, Tb // P)
    cu = np.arange(0, B * Tb + 1, Tb, dtype=np.int32)
    for layer in whole:
        bench.make_c5_layer(torch, dev, layer, x)
        wsc, wpool = O.kv_quant_append_torch(x.cpu(), cu, seq_tables, B * Tb // P, P)
        np.testing.assert_array_equal(scales[layer].view(np.uint32), wsc.numpy().view(np.uint32))
        wk, wv = O.kv_gather_dequant_torch(wpool, wsc, seq_tables, np.full(B, Tb, np.int32), Tb)
        for name, g_, w_ in (("K", got_whole[layer][0], wk), ("V", got_whole[layer][1], wv)):
            gi, wi = g_.view(torch.int16), w_.view(torch.int16)
            assert torch.equal(gi, wi), f"layer {layer} {name}: {(gi != wi).sum().item()} values differ"
        where = "spilled to pinned DRAM and prefetched back" if layer < cache.n_spill else "resident"
        print(f"layer {layer} ({where}): every gathered value ({2 * wk.numel()}) bit-exact", flush=True)
        del wpool, wk, wv
    for layer in sample:
        bench.make_c5_layer(torch, dev, layer, x)
        xb = bits16(x)
        wsc = O.kv_scales(xb[None])
        np.testing.assert_array_equal(scales[layer].view(np.uint32), wsc[0].view(np.uint32))
        b, pos = picks[layer]
        _, deq = _oracle_rows(xb, wsc, b * Tb + pos, P)
        gk, gv = (bits16(t) for t in got[layer])
        _assert_bf16_bits(gk, deq[0].transpose(1, 0, 2))
        _assert_bf16_bits(gv, deq[1].transpose(1, 0, 2))
        where = "spilled to pinned DRAM and prefetched back" if layer < cache.n_spill else "resident"
        print(f"layer {layer} ({where}): scales and {S} gathered rows bit-exact", flush=True)
    del c, cache, x, got, got_whole
    torch.cuda.empty_cache()


def test_streamed_step_through_two_slots(dev):
    """The streamed cache at a high streaming ratio: 12 layers through 2 HBM layer slots
    (10 of 12 layers written back to pinned DRAM and prefetched back; 6:1), small layers
    (4 x 2,048 tokens), two sweeps on the same buffers.  Every gathered K and V value of
    every layer in both sweeps bit-exact against the oracle's torch restatement of the
    append followed by its gather, and every scale against fp32(max(amax, 1e-8) / 448)."""
    L, S, Tb = 12, 2, 2048
    C = bench.C5
    H, D, P, B = C["H"], C["D"], C["P"], C["B"]
    c = bench.configs4_setup(torch, dev, hbm_layers=S, layers=L, tokens=Tb)
    cache = c["cache"]
    assert cache.n_spill == L - S and cache.S == S
    seq_tables = np.arange(B * Tb // P, dtype=np.int32).reshape(B, Tb // P)
    cu = np.arange(0, B * Tb + 1, Tb, dtype=np.int32)
    want = {}
    x = c["x"]
    for layer in range(L):
        bench.make_c5_layer(torch, dev, layer, x)
        wsc, wpool = O.kv_quant_append_torch(x.cpu(), cu, seq_tables, B * Tb // P, P)
        wk, wv = O.kv_gather_dequant_torch(wpool, wsc, seq_tables, np.full(B, Tb, np.int32), Tb)
        want[layer] = (wsc.numpy(), wk.view(torch.int16), wv.view(torch.int16))
    for sweep in range(2):
        got = {}
        bench.configs4_step(torch, dev, c, lambda l, k, v: got.__setitem__(l, (k.cpu(), v.cpu())))
        torch.cuda.synchronize()
        cache.check_errors()
        scales = cache.scales.cpu().numpy()
        for layer in range(L):
            np.testing.assert_array_equal(scales[layer].view(np.uint32), want[layer][0].view(np.uint32))
            for name, g_, w_ in (("K", got[layer][0], want[layer][1]), ("V", got[layer][1], want[layer][2])):
                gi = g_.view(torch.int16)
                assert torch.equal(gi, w_), f"sweep {sweep} layer {layer} {name}: {(gi != w_).sum().item()} differ"
        print(f"sweep {sweep}: all {L} layers bit-exact through {S} slots", flush=True)
    del c, cache
    torch.cuda.empty_cache()
