"""GPU parity over a seeded sweep of attention shapes: the MFMA kernel through
tsa_attn_gqa_fwd (grouped K/V heads, with and without the output gate) and the VALU opponent
through tsa_attn_fwd (Hkv = Hq, no gate), against the oracle (naive_attn_kernel restated,
src/attn_sm75.cu:55-94; the gated GQA layer defined on it) on every row.  Shapes mix batches,
head groupings, ragged S (one key to past ten 64-key tiles, so diagonal and tail tiles land at
every offset), D in {64, 128, 256}, causal and not, and N(0, 1) or N(0, 0.5) inputs with 1 %
outliers x8 (the long-context configuration's input form), so that the kernels' masks, tile
walks and head maps meet shapes the hand-picked cases do not.

Gate: max-abs < 0.02 on fp16 outputs (src/attn_sm75.cu:501-502); the tighter 5e-3 of
test_gpu_attn.py guards regressions.
"""
import numpy as np
import pytest

import tsa

pytestmark = pytest.mark.gpu
GATE, TIGHT = 2e-2, 5e-3


def _cases(n=24, seed=2027):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        B = int(rng.integers(1, 3))
        Hkv = int(rng.integers(1, 4))
        grp = int(rng.choice([1, 1, 2, 3, 6]))
        S = int(rng.choice([1, 2, 63, 64, 65, 127, 128, 129]) if i % 3 == 0 else rng.integers(130, 700))
        D = [64, 128, 256][i % 3]
        causal = bool(i % 2 == 0)
        gated = bool(grp > 1 and i % 4 != 3)
        outliers = bool(i % 5 == 2)
        cases.append((i, B, Hkv * grp, Hkv, S, D, causal, gated, outliers))
    return cases


def _tensor(rng, shape, outliers):
    if not outliers:
        return rng.standard_normal(shape).astype(np.float16)
    x = 0.5 * rng.standard_normal(shape)
    m = rng.random(shape) < 0.01
    x[m] *= 8
    return x.astype(np.float16)


@pytest.mark.parametrize("case", _cases(), ids=lambda c: "c{}_B{}Hq{}Hkv{}S{}D{}{}{}{}".format(
    c[0], c[1], c[2], c[3], c[4], c[5], "_causal" if c[6] else "", "_gate" if c[7] else "",
    "_outliers" if c[8] else ""))
def test_attention_sweep(dev, orc, case):
    import torch
    i, B, Hq, Hkv, S, D, causal, gated, outliers = case
    print(f"attention sweep case {i}: B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} causal={causal} "
          f"gate={gated} outliers={outliers}", flush=True)
    rng = np.random.default_rng(3000 + i)
    q = _tensor(rng, (B, Hq, S, D), outliers)
    k, v = _tensor(rng, (B, Hkv, S, D), outliers), _tensor(rng, (B, Hkv, S, D), outliers)
    gate = (2.0 * rng.standard_normal((B, Hq, S, D))).astype(np.float16) if gated else None
    rows, ref = orc.attn_gqa_rows(q, k, v, gate, np.arange(B * Hq * S), causal)
    tq, tk, tv = (torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in (q, k, v))
    tg = torch.from_numpy(gate).to(dev) if gated else None
    o = tsa.attn_gqa_fwd(tq, tk, tv, tg, causal=causal)
    torch.cuda.synchronize()
    e = float(np.abs(o.cpu().numpy().astype(np.float64).reshape(-1, D)[rows] - ref).max())
    print(f"  mfma: max-abs {e:.2e}", flush=True)
    assert e < min(TIGHT, GATE)
    if Hkv == Hq and not gated:
        ov = tsa.attn_fwd(tq, tk, tv, causal=causal, valu=True)
        torch.cuda.synchronize()
        ev = float(np.abs(ov.cpu().numpy().astype(np.float64).reshape(-1, D)[rows] - ref).max())
        print(f"  valu: max-abs {ev:.2e}", flush=True)
        assert ev < min(TIGHT, GATE)
