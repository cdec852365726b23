"""Page-table and cache-layout cases on the GPU.

Block-table entries outside the cache's pages: each kernel family (warp-specialized FP8 + log8,
per-group bf16, column-split d_c 1792) checks every entry it reads against the page count the
wrapper passes, reads page 0 instead of the bad page, and stores QMLA_ERR_PAGE into the status word;
the requests whose entries are all valid still match the oracle, in the balanced and the fixed-split
modes. The reference trusts the table (a bad entry is an out-of-bounds read there).

A cache whose token stride is wider than its rows (bytes past every row set to NaN) matches the
oracle in the warp-specialized, row-owner and per-group kernels."""
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


# A cache whose token stride is wider than the row (a view of a wider tensor): the kernels take the
# per-lane page-lookup path instead of one buffer range per tile.
PADDED = {
    "ws_fp8_log8": dict(d_c=512, kv="fp8", rms_mode="log8", qrows=1, groups=1),
    "ro_gla_fp8_log8": dict(d_c=512, kv="fp8", rms_mode="log8", qrows=4, groups=2),
    "partial_bf16": dict(d_c=512, kv="bf16", rms_mode="bf16", qrows=1, groups=1),
}


@pytest.mark.parametrize("splits", [0, 4])
@pytest.mark.parametrize("family", sorted(PADDED))
def test_padded_token_stride(gpu, family, splits):
    import qmla
    f = PADDED[family]
    c = make_case(batch=3, heads=24, d_c=f["d_c"], rope_w=64, page_size=64, lens=[700, 1500, 33], kv=f["kv"],
                  rms_mode=f["rms_mode"], seed=73, device=gpu, qrows=f["qrows"], groups=f["groups"],
                  rms="spread")
    pages, P, one, row = c.cache.shape
    pad = 32 if f["kv"] == "fp8" else 16   # elements: 32 bytes past every row
    wide = torch.full((pages, P, one, row + pad), 0x7F if f["kv"] == "fp8" else float("nan"),
                      dtype=c.cache.dtype, device=gpu)
    wide[..., :row] = c.cache
    view = wide[..., :row]
    assert view.stride(1) == row + pad
    print(f"[padded stride {family} splits {splits}] row {row}, token stride {row + pad}", flush=True)
    o, lse = qmla.forward(c.q_nope, c.q_pe, view, c.block_table, c.seq_lens, d_c=c.d_c, page_size=c.page_size,
                          sm_scale=c.sm_scale, kv_fp8=c.kv == "fp8", fp8_rms="log8", k_scale=c.k_scale,
                          qrows=c.qrows, groups=c.groups, num_splits=splits, num_workgroups=0 if splits else 5)
    torch.cuda.synchronize()
    ro, rl = run_oracle(c)
    err = (o.float().cpu() - ro).abs().max().item()
    lerr = (lse.cpu() - rl).abs().max().item()
    print(f"  max-abs {err:.3e} lse {lerr:.3e}", flush=True)
    assert err < TOL[c.kv] and lerr < 1e-2
