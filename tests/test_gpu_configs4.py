"""configs[4] (70B-shape share, 4 x 131,072 tokens per layer) parity on sampled layers.

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
