"""A seeded sweep of the prefill context gather (qmla_gather) against the oracle's restatement of
gather_cache_torch (ops/mla_gather.py:28-76), bit for bit: FP8 rows with each rms format and bf16
rows, latent ranks 256-1792 with rope 64 / 116 / 232 (the plugin's deployed layouts put the rms tail
at offsets that are not multiples of 8, as the reference's FP8 test gathers them,
tests/test_fp8_kv.py:111-122), pages of 1-784 tokens, whole sequences or chunks that start inside
them. Columns past the decoded row and rows past the chunk keep their sentinel.
"""
import random

import numpy as np
import pytest
import torch

from tests.mla_cases import make_case, ora
from tests.test_gpu_gather import SENT, _meta, _oracle, _run

pytestmark = pytest.mark.gpu

LAYOUTS = [(512, 64, 24), (256, 232, 24), (768, 116, 12), (1792, 64, 24), (1792, 232, 24)]
RMS = {"log8": ("log8", ora.RMS_LOG8), "bf16_bytes": ("bf16", ora.RMS_BF16_BYTES), "e4m3": ("e4m3", ora.RMS_E4M3)}


def _draw(seed):
    r = random.Random(seed)
    kv = "fp8" if seed % 4 else "bf16"
    rms = r.choice(sorted(RMS)) if kv == "fp8" else "bf16"
    d_c, rope, heads = LAYOUTS[seed % len(LAYOUTS)]
    page = r.choice((1, 16, 64, 784))
    lens = [r.randint(1, 1500) for _ in range(r.randint(1, 4))]
    sliced = r.random() < 0.5
    starts = [r.randint(0, L - 1) for L in lens] if sliced else None
    clen = [r.randint(0, L - st) for L, st in zip(lens, starts)] if sliced else list(lens)
    if sum(clen) == 0:
        clen[0] = lens[0] - (starts[0] if starts else 0)
    return dict(kv=kv, rms=rms, d_c=d_c, rope=rope, heads=heads, page=page, lens=lens, starts=starts, clen=clen)


@pytest.mark.parametrize("seed", range(100))
def test_gather_sweep(gpu, seed):
    a = _draw(seed)
    print(f"[gather sweep {seed}] {a['kv']} {a['rms']} d_c {a['d_c']} rope {a['rope']} heads {a['heads']} "
          f"page {a['page']} lens {a['lens']} starts {a['starts']} chunk {a['clen']}", flush=True)
    c = make_case(batch=len(a["lens"]), heads=a["heads"], d_c=a["d_c"], rope_w=a["rope"], page_size=a["page"],
                  lens=a["lens"], kv=a["kv"], rms_mode=a["rms"], seed=2000 + seed, device=gpu, rms="spread", amp=4.0)
    cu, t2s, ss, n = _meta(a["clen"], a["starts"])
    if a["kv"] == "fp8":
        mode, omode = RMS[a["rms"]]
        got = _run(gpu, c, "fp8", (c.rms_offset, c.heads, mode), cu, t2s, ss, n, c.row)
        exp = _oracle(c, cu, t2s, ss, n, "fp8", omode)
        k = c.rms_offset + c.heads
    else:
        got = _run(gpu, c, "auto", None, cu, t2s, ss, n, c.row)
        exp = _oracle(c, cu, t2s, ss, n, "bf16", ora.RMS_NONE)
        k = c.row
    bad = np.argwhere(got[:n, :k] != exp[:, :k])
    assert bad.size == 0, (bad[:5].tolist(), len(bad))
    assert np.all(got[:n, k:] == SENT) and np.all(got[n:] == SENT)
