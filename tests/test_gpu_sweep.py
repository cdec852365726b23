"""A seeded sweep over the supported decode families against the CPU oracle: every case draws a
family, page size, batch, ragged lengths (empty requests included), verify tokens and split mode
from its seed, so combinations no targeted test picks are covered too. Tolerances as in
tests/test_gpu_decode.py (max-abs 1e-2 bf16 / 3e-2 fp8 beyond the output's own bf16 rounding; lse
1e-2, -inf exactly where a row sees no token).
"""
import random

import pytest
import torch

from tests.mla_cases import make_case, run_oracle

pytestmark = pytest.mark.gpu

REL = 2.0 ** -7
# (kv, rms mode, d_c, heads, verify tokens allowed, groups)
FAMILIES = [
    ("fp8", "log8", 512, 24, (1,), 1),           # warp-specialized, transposed rms reads
    ("fp8", "log8", 512, 16, (1, 2), 1),         # warp-specialized, rms read per row
    ("fp8", "log8", 512, 8, (1, 2, 4), 1),
    ("fp8", "log8", 512, 24, (1, 2, 4), 2),      # GLA-g2
    ("fp8", "e4m3", 512, 24, (1, 4), 1),         # per-group kernel
    ("fp8", "bf16_bytes", 512, 24, (1,), 1),
    ("bf16", "bf16", 512, 24, (1, 4), 1),
    ("bf16", "bf16", 1792, 24, (1,), 1),         # column-split kernel
]
PAGES = (1, 16, 40, 64, 784)


def _draw(seed):
    r = random.Random(seed)
    kv, rms, d_c, heads, qopts, groups = FAMILIES[seed % len(FAMILIES)]
    qrows = r.choice(qopts)
    page = r.choice(PAGES)
    batch = r.randint(1, 6)
    lens = [r.choice((0, 1, 2, 3, r.randint(4, 400), r.randint(400, 2500))) for _ in range(batch)]
    if all(L == 0 for L in lens):
        lens[0] = 17
    splits = r.choice((0, 0, 1, 3, 16))
    nwg = r.choice((0, 2, 7, 33)) if splits == 0 else 0
    return dict(kv=kv, rms=rms, d_c=d_c, heads=heads, qrows=qrows, groups=groups, page=page, lens=lens,
                splits=splits, nwg=nwg)


@pytest.mark.parametrize("seed", range(40))
def test_sweep(gpu, seed):
    import qmla
    a = _draw(seed)
    print(f"[sweep {seed}] {a}", flush=True)
    c = make_case(batch=len(a["lens"]), heads=a["heads"], d_c=a["d_c"], rope_w=64, page_size=a["page"], lens=a["lens"],
                  kv=a["kv"], rms_mode=a["rms"], seed=1000 + seed, device=gpu, qrows=a["qrows"], groups=a["groups"],
                  rms="spread", amp=2.0)
    kw = dict(kv_fp8=True, fp8_rms={"bf16_bytes": "bf16"}.get(a["rms"], a["rms"]), k_scale=c.k_scale) \
        if a["kv"] == "fp8" else {}
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, d_c=a["d_c"], page_size=a["page"],
                          sm_scale=c.sm_scale, qrows=a["qrows"], groups=a["groups"], num_splits=a["splits"],
                          num_workgroups=a["nwg"], **kw)
    torch.cuda.synchronize()
    ro, rl = run_oracle(c)
    tol = 3e-2 if a["kv"] == "fp8" else 1e-2
    d = (o.float().cpu() - ro).abs()
    excess = (d - REL * ro.abs()).max().item()
    lg = lse.float().cpu()
    empty = torch.isneginf(rl)
    assert torch.equal(torch.isneginf(lg), empty), "rows without tokens differ"
    lerr = (lg[~empty] - rl[~empty]).abs().max().item() if (~empty).any() else 0.0
    print(f"   max-abs {d.max().item():.3e} beyond rounding {excess:.3e} (tol {tol}) lse {lerr:.3e}", flush=True)
    assert excess < tol and lerr < 1e-2
