"""NaN inputs: one NaN element in one head's query row, and one NaN code (e4m3 0x7F, or a bf16 NaN)
in one cached latent element of another request. The softmax of the warp-specialized, row-owner and
column-split kernels is compiled without NaN semantics (no canonicalizing v_max before each fmaxf),
so this pins what reaches the outputs:

  * the head whose query holds the NaN outputs NaN (every column), as the reference's Triton decode
    does (its q.k, maximum and exp propagate NaN);
  * every head of the request whose cache holds the NaN outputs NaN (the latent is every head's key
    and value; with GLA-g2 every head of the latent group the column belongs to);
  * every other row, of those requests and of the others, is finite and meets the parity bound.

The lse of a row whose inputs hold a NaN is NaN, as in the reference, but not pinned here.
Each family in the balanced mode (split requests merged by the combine) and with fixed splits.
"""
import pytest
import torch

from tests.mla_cases import C_REF, TOL, make_case, run_oracle_requests

pytestmark = pytest.mark.gpu

# (name, kv, rms, d_c, heads, groups, qrows)
FAMILIES = [
    ("ws", "fp8", "log8", 512, 24, 1, 1),        # warp-specialized (the headline kernel)
    ("ro", "fp8", "log8", 512, 24, 2, 4),        # row-owner GLA-g2
    ("group", "bf16", "bf16", 512, 24, 1, 1),    # per-group kernel
    ("cs", "bf16", "bf16", 1792, 24, 1, 1),      # column-split wide latent
]
LENS = [900, 1500, 700, 1200]
QREQ, QHEAD, QCOL = 1, 5, 100        # request, head and column of the NaN query element
CREQ, CTOK, CCOL = 2, 333, 42        # request, token and latent column of the NaN cached element


@pytest.mark.parametrize("splits", [0, 4])
@pytest.mark.parametrize("fam", FAMILIES, ids=lambda f: f[0])
def test_nan_inputs_stay_in_their_rows(gpu, fam, splits):
    import qmla
    name, kv, rms, d_c, heads, groups, qrows = fam
    c = make_case(batch=len(LENS), heads=heads, d_c=d_c, rope_w=64, page_size=64, lens=LENS, kv=kv, rms_mode=rms,
                  seed=61, device=gpu, qrows=qrows, groups=groups, rms="spread", amp=2.0)
    # the NaN query element: head QHEAD of the first verify row of request QREQ
    qn = c.q_nope.clone()
    qn[QREQ * qrows, QHEAD, QCOL] = float("nan")
    # the NaN cached element: latent column CCOL of token CTOK of request CREQ
    page = int(c.block_table[CREQ * qrows + qrows - 1, CTOK // c.page_size])
    if kv == "fp8":
        c.cache[page, CTOK % c.page_size, 0, CCOL] = 0x7F                       # e4m3fn NaN
    else:
        c.cache.view(torch.int16)[page, CTOK % c.page_size, 0, CCOL] = 0x7FC0    # bf16 NaN
    kw = dict(kv_fp8=True, fp8_rms=rms, k_scale=c.k_scale) if kv == "fp8" else {}
    o, lse = qmla.forward(qn, c.q_pe, c.cache, c.block_table, c.seq_lens, d_c=d_c, page_size=c.page_size,
                          sm_scale=c.sm_scale, qrows=qrows, groups=groups, num_splits=splits, num_workgroups=3,
                          **kw)
    torch.cuda.synchronize()
    o = o.float().cpu()
    print(f"[nan {name} S={splits}]", flush=True)
    # the query NaN: that head of that row is NaN in every column
    assert torch.isnan(o[QREQ * qrows, QHEAD]).all(), "NaN query did not reach its row"
    # the cache NaN: every row of that request that sees the token is NaN in every head that reads
    # the column (GLA-g2: the heads of its latent group)
    crows = [CREQ * qrows + j for j in range(qrows) if LENS[CREQ] - (qrows - 1 - j) > CTOK]
    hpg = heads // groups
    g = CCOL // (d_c // groups)
    cheads = slice(g * hpg, (g + 1) * hpg)
    assert torch.isnan(o[crows][:, cheads]).all(), "NaN cache element did not reach its request's rows"
    # everything else: finite and within the bound of the oracle on the clean inputs of those rows
    clean = torch.ones(o.shape[:2], dtype=torch.bool)
    clean[QREQ * qrows, QHEAD] = False
    clean[crows, cheads] = False
    assert torch.isfinite(o[clean]).all(), "a NaN leaked into other rows"
    reqs = [b for b in range(len(LENS)) if b != CREQ]
    ro, rl, rows = run_oracle_requests(c, reqs)          # c.q_nope is the clean query
    eo, _, _ = run_oracle_requests(c, reqs, reference_rounding=True, num_splits=max(splits, 1))
    got = o[rows]
    keep = clean[rows]
    err = (got[keep] - ro[keep]).abs().max().item()
    ref_err = (eo.to(torch.bfloat16).float()[keep] - ro[keep]).abs().max().item()
    bound = max(TOL[kv], C_REF * ref_err)
    assert torch.isfinite(lse.float().cpu()[rows][keep]).all()
    print(f"   other rows: max-abs {err:.3e} (tol {TOL[kv]}, reference roundings {ref_err:.3e}, bound {bound:.3e})",
          flush=True)
    assert err < bound
