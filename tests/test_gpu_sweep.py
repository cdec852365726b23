"""A seeded sweep over the supported decode families against the CPU oracle: every case draws a
family (kernel family, cache format, rms format, latent rank, heads, rope width, logit cap), page
size, batch, ragged lengths (empty requests included), verify tokens, split mode and the output
element type (bf16, fp16 or fp32; outputs start as NaN) from its seed, so combinations no targeted
test picks are covered too. Bound: plain max-abs 1e-2 (bf16 cache) / 3e-2 (fp8 cache) against the
float32 oracle, or, where the reference kernel's own roundings already exceed that on the same
inputs, C_REF times their error; lse within 1e-2 (beyond an fp16 lse's rounding), -inf exactly
where a row sees no token.
"""
import random

import pytest
import torch

from tests.mla_cases import C_REF, TOL, make_case, run_oracle

pytestmark = pytest.mark.gpu

# (kv, rms mode, d_c, heads, rope width, verify tokens allowed, groups, logit cap)
FAMILIES = [
    ("fp8", "log8", 512, 24, 64, (1,), 1, 0.0),            # warp-specialized, transposed rms reads
    ("fp8", "log8", 512, 16, 64, (1, 2), 1, 0.0),          # warp-specialized, rms read per row
    ("fp8", "log8", 512, 8, 64, (1, 2, 4), 1, 0.0),
    ("fp8", "log8", 512, 24, 64, (1, 2, 4), 2, 0.0),       # GLA-g2
    ("fp8", "e4m3", 512, 24, 64, (1, 4), 1, 0.0),          # per-group kernel
    ("fp8", "bf16_bytes", 512, 24, 64, (1,), 1, 0.0),
    ("bf16", "bf16", 512, 24, 64, (1, 4), 1, 0.0),
    ("bf16", "bf16", 1792, 24, 64, (1,), 1, 0.0),          # column-split kernel
    ("fp8", "log8", 512, 24, 64, (1,), 1, 30.0),           # tanh logit cap
    ("bf16", "bf16", 512, 24, 64, (1,), 1, 30.0),
    ("fp8", "log8", 256, 24, 232, (1,), 1, 0.0),           # the plugin's deployed partial-rope layouts
    ("fp8", "e4m3", 768, 12, 116, (1,), 1, 0.0),
    ("bf16", "bf16", 256, 12, 116, (1,), 1, 0.0),
    ("bf16", "bf16", 768, 24, 232, (1,), 1, 0.0),          # ... rank 768 in the column-split kernel
    ("fp8", "log8", 1792, 24, 232, (1,), 1, 0.0),          # ... rank 1792 (padded rope windows)
    ("fp8", "bf16_bytes", 1792, 12, 116, (1, 2, 4), 1, 0.0),
    ("fp8", "log8", 1792, 24, 64, (1,), 1, 0.0),           # FP8 wide latent, rows split over workgroups
]
# seeds from FOLD_SEED0 on: spec-verify rows folded on every cache format and deployed layout (the
# rows of a request split over up to four workgroups sharing its token range)
FOLD_SEED0 = 2000
FOLD_FAMILIES = [
    ("fp8", "e4m3", 512, 24, 64, (2, 4), 1, 0.0),
    ("fp8", "bf16_bytes", 512, 24, 64, (2, 4), 1, 0.0),
    ("bf16", "bf16", 512, 24, 64, (2, 3, 4), 1, 30.0),
    ("fp8", "log8", 256, 24, 232, (2, 4), 1, 0.0),
    ("fp8", "bf16_bytes", 768, 24, 232, (2, 4), 1, 0.0),
    ("bf16", "bf16", 768, 24, 232, (2, 4), 1, 0.0),
    ("bf16", "bf16", 1792, 24, 64, (2, 4), 1, 0.0),
    ("fp8", "log8", 1792, 24, 232, (2, 4), 1, 0.0),
]
PAGES = (1, 16, 40, 64, 784)


def _draw(seed):
    r = random.Random(seed)
    fams = FAMILIES if seed < FOLD_SEED0 else FOLD_FAMILIES
    kv, rms, d_c, heads, rope, qopts, groups, cap = fams[seed % len(fams)]
    qrows = r.choice(qopts)
    page = r.choice(PAGES)
    batch = r.randint(1, 6)
    lens = [r.choice((0, 1, 2, 3, r.randint(4, 400), r.randint(400, 2500))) for _ in range(batch)]
    if all(L == 0 for L in lens):
        lens[0] = 17
    splits = r.choice((0, 0, 1, 3, 16))
    nwg = r.choice((0, 2, 7, 33)) if splits == 0 else 0
    odt = r.choice(("bf16", "bf16", "f16", "f32"))   # output and lse element type (drawn last)
    return dict(kv=kv, rms=rms, d_c=d_c, heads=heads, rope=rope, qrows=qrows, groups=groups, cap=cap, page=page,
                lens=lens, splits=splits, nwg=nwg, odt=odt)


def run_case(gpu, seed):
    """Run sweep case `seed` on the GPU; returns its plain errors against the float32 oracle and the
    error of the reference's own roundings (the oracle's emulation, output rounded to the same
    element type) on the same inputs."""
    import qmla
    a = _draw(seed)
    print(f"[sweep {seed}] {a}", flush=True)
    c = make_case(batch=len(a["lens"]), heads=a["heads"], d_c=a["d_c"], rope_w=a["rope"], page_size=a["page"],
                  lens=a["lens"], kv=a["kv"], rms_mode=a["rms"], seed=1000 + seed, device=gpu, qrows=a["qrows"],
                  groups=a["groups"], rms="spread", amp=2.0)
    kw = dict(kv_fp8=True, fp8_rms={"bf16_bytes": "bf16"}.get(a["rms"], a["rms"]), k_scale=c.k_scale) \
        if a["kv"] == "fp8" else {}
    dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[a["odt"]]
    rows = c.q_nope.shape[0]
    o = torch.full((rows, a["heads"], a["d_c"] // a["groups"]), float("nan"), dtype=dt, device=gpu)
    lse = torch.full((rows, a["heads"]), float("nan"), dtype=torch.float32 if dt == torch.bfloat16 else dt,
                     device=gpu)
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, d_c=a["d_c"], page_size=a["page"],
                          sm_scale=c.sm_scale, qrows=a["qrows"], groups=a["groups"], num_splits=a["splits"],
                          num_workgroups=a["nwg"], logit_cap=a["cap"], out=o, lse=lse, **kw)
    torch.cuda.synchronize()
    ro, rl = run_oracle(c, logit_cap=a["cap"])
    eo, _ = run_oracle(c, logit_cap=a["cap"], reference_rounding=True, num_splits=max(a["splits"], 1),
                       align=16 if a["page"] % 16 == 0 else 0)
    lg = lse.float().cpu()
    empty = torch.isneginf(rl)
    lrel = 2.0 ** -11 if lse.dtype == torch.float16 else 0.0
    lerr = ((lg[~empty] - rl[~empty]).abs() - lrel * rl[~empty].abs()).max().item() if (~empty).any() else 0.0
    return dict(kv=a["kv"], err=(o.float().cpu() - ro).abs().max().item(),
                ref_err=(eo.to(dt).float() - ro).abs().max().item(), lerr=lerr,
                empty_ok=torch.equal(torch.isneginf(lg), empty))


# 1231: bf16 d_c 1792, one split, lengths [2102, 205, 2] on 784-token pages, inputs x2 -- the one
# case of an earlier 2,800-seed sweep whose plain error (3.2e-2) exceeded the bound of its time
@pytest.mark.parametrize("seed", list(range(200)) + [1231] + list(range(FOLD_SEED0, FOLD_SEED0 + 48)))
def test_sweep(gpu, seed):
    r = run_case(gpu, seed)
    tol = TOL[r["kv"]]
    bound = max(tol, C_REF * r["ref_err"])
    print(f"   max-abs {r['err']:.3e} (tol {tol}, reference roundings {r['ref_err']:.3e}, bound {bound:.3e}) "
          f"lse {r['lerr']:.3e}", flush=True)
    assert r["empty_ok"], "rows without tokens differ"
    assert r["err"] < bound and r["lerr"] < 1e-2
