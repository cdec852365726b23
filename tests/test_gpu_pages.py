"""Block-table entries outside the cache's pages, on the GPU: each kernel family (warp-specialized FP8
+ log8, per-group bf16, column-split d_c 1792) checks every entry it reads against the page count
the wrapper passes, reads page 0 instead of the bad page, and stores QMLA_ERR_PAGE into the status
word; the requests whose entries are all valid still match the oracle, in the balanced and the
fixed-split modes. The reference trusts the table (a bad entry is an out-of-bounds read there)."""
import pytest
import torch

from tests.mla_cases import TOL, make_case, run_oracle

pytestmark = pytest.mark.gpu

FAMILIES = {
    "ws_fp8_log8": dict(d_c=512, kv="fp8", rms_mode="log8", lens=[700, 1500, 300]),
    "partial_bf16": dict(d_c=512, kv="bf16", rms_mode="bf16", lens=[700, 1500, 300]),
    "cs_bf16_1792": dict(d_c=1792, kv="bf16", rms_mode="bf16", lens=[300, 900, 200]),
}


@pytest.mark.parametrize("splits", [0, 4])
@pytest.mark.parametrize("family", sorted(FAMILIES))
def test_out_of_range_page_ids(gpu, family, splits):
    import qmla
    from qmla import _lib
    f = FAMILIES[family]
    c = make_case(batch=3, heads=24, d_c=f["d_c"], rope_w=64, page_size=64, lens=f["lens"], kv=f["kv"],
                  rms_mode=f["rms_mode"], seed=71, device=gpu)
    n_pages = c.cache.shape[0]
    bt = c.block_table.clone()
    bt[1, 2] = n_pages + 7      # past the cache
    bt[1, 5] = -3               # negative
    print(f"[pages {family} splits {splits}] {n_pages} pages, request 1 entries 2 and 5 invalid", flush=True)

    def run(table):
        status = torch.zeros(1, dtype=torch.int32, device=gpu)
        o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, table, c.seq_lens, d_c=c.d_c, page_size=c.page_size,
                              sm_scale=c.sm_scale, kv_fp8=c.kv == "fp8", fp8_rms="log8", k_scale=c.k_scale,
                              num_splits=splits, num_workgroups=0 if splits else 6, status=status)
        torch.cuda.synchronize()
        return o, lse, int(status.item())

    o, lse, st = run(bt)
    assert st == _lib.ERR_PAGE
    assert torch.isfinite(o.float()).all() and torch.isfinite(lse).all()
    ro, rl = run_oracle(c, rows=[0, 2])
    err = (o.float().cpu()[[0, 2]] - ro).abs().max().item()
    lerr = (lse.cpu()[[0, 2]] - rl).abs().max().item()
    print(f"  valid requests: max-abs {err:.3e} lse {lerr:.3e}", flush=True)
    assert err < TOL[c.kv] and lerr < 1e-2
    # the intact table leaves the status word untouched
    _, _, st = run(c.block_table)
    assert st == 0
