"""GPU parity of the wide-latent decode (d_c = 1792, rope 64, 24 heads) against the CPU oracle: the
reference routes these widths to its two-pass path (ops/mla_decode_attention.py:778-849); the library
computes them in one pass, with the same partial layout and split bounds. bf16 caches (one workgroup
holds the 24 heads), FP8 caches with log8 codes (16 rows per workgroup: the heads are split over two
workgroups that read the same tokens), 4-token verify rows (96 rows over three workgroups), and the
plugin's deployed FP8 layouts (rope 232 / 116 in padded windows) in balanced mode and with verify
rows.

Bound: tests.mla_cases.check_decode (plain max-abs 1e-2 for a bf16 cache / 3e-2 for an FP8 cache
against the float32 oracle, or C_REF times the reference roundings' own error where that is
larger), lse 1e-2.
"""
import pytest
import torch

from tests.mla_cases import check_decode, check_partials, make_case

pytestmark = pytest.mark.gpu

DC = 1792


@pytest.mark.parametrize("page_size,splits", [(1600, 16), (40, 3)])
def test_wide_reference_surface(gpu, page_size, splits):
    """decode_attention_fwd with fixed splits: 1600-token pages (one page per 16-token tile) and
    40-token pages (pages change inside a tile); partials in the reference layout."""
    import qmla
    lens = [1, 1700, 5000, 333]
    c = make_case(batch=len(lens), heads=24, d_c=DC, rope_w=64, page_size=page_size, lens=lens, kv="bf16",
                  seed=3, device=gpu, rms="spread")
    B, H = c.q_nope.shape[:2]
    q = torch.zeros(B, H, c.row, dtype=torch.bfloat16, device=gpu)
    q[..., :DC] = c.q_nope
    q[..., DC:DC + 64] = c.q_pe
    q[..., DC + 64:] = 5.0      # tail columns are not part of the scores
    o = torch.full((B, H, DC), float("nan"), dtype=torch.bfloat16, device=gpu)
    lse = torch.zeros(B, H, dtype=torch.float32, device=gpu)
    logits = torch.full((B, H, splits, DC + 1), float("nan"), dtype=torch.float32, device=gpu)
    qmla.decode_attention_fwd(q, c.cache, c.cache[..., :DC], o, lse, c.block_table, c.seq_lens, logits, splits,
                              c.sm_scale, page_size, is_mla=True, rms_offset=DC + 64)
    torch.cuda.synchronize()
    align = 16 if page_size % 16 == 0 else 0
    check_decode(f"wide P={page_size} S={splits}", c, o, lse, num_splits=splits, align=align)
    check_partials(f"wide P={page_size} S={splits}", c, logits, num_splits=splits, align=align)


@pytest.mark.parametrize("page_size", [64, 40])
def test_wide_balanced(gpu, page_size):
    """Balanced split mode over ragged lengths, a few workgroups so requests span several."""
    import qmla
    lens = [33, 900, 4100, 16, 2500]
    c = make_case(batch=len(lens), heads=24, d_c=DC, rope_w=64, page_size=page_size, lens=lens, kv="bf16",
                  seed=8, device=gpu, rms="spread")
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, page_size=page_size,
                          sm_scale=c.sm_scale, num_workgroups=9)
    torch.cuda.synchronize()
    check_decode(f"wide balanced P={page_size}", c, o, lse)


def test_wide_no_rms(gpu):
    """No rms tail (rms_offset < 0): plain scores."""
    import qmla
    lens = [700, 1999]
    c = make_case(batch=len(lens), heads=24, d_c=DC, rope_w=64, page_size=64, lens=lens, kv="bf16",
                  rms_mode="none", seed=9, device=gpu)
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, page_size=64, rms_offset=-1,
                          sm_scale=c.sm_scale, num_workgroups=4)
    torch.cuda.synchronize()
    check_decode("wide no-rms", c, o, lse)


@pytest.mark.parametrize("page_size,splits", [(64, 16), (40, 0)])
def test_wide_fp8(gpu, page_size, splits):
    """FP8 rows with log8 codes: fixed splits on 64-token pages and the balanced mode on 40-token
    pages (pages change inside a 32-token tile)."""
    import qmla
    lens = [1, 2100, 5000, 333]
    c = make_case(batch=len(lens), heads=24, d_c=DC, rope_w=64, page_size=page_size, lens=lens, kv="fp8",
                  rms_mode="log8", seed=21, device=gpu, rms="spread", amp=4.0)
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, page_size=page_size,
                          sm_scale=c.sm_scale, kv_fp8=True, fp8_rms="log8", k_scale=c.k_scale, num_splits=splits,
                          num_workgroups=0 if splits else 11)
    torch.cuda.synchronize()
    check_decode(f"wide fp8 P={page_size} S={splits}", c, o, lse)


def test_wide_verify_rows(gpu):
    """4 verify tokens per request (row j sees L - 3 + j tokens) x 24 heads, no rms tail, passed to the
    C entry unfolded (96 rows per request: three workgroups per token range), balanced mode."""
    import qmla
    from qmla import _lib
    from qmla.decode import Workspace, build_params, workspace_bytes
    lens = [5, 1500, 3333]
    c = make_case(batch=len(lens), heads=24, d_c=DC, rope_w=64, page_size=64, lens=lens, kv="bf16",
                  rms_mode="none", seed=22, device=gpu, qrows=4)
    rows = c.q_nope.shape[0]
    out = torch.empty(rows, 24, DC, dtype=torch.bfloat16, device=gpu)
    lse = torch.empty(rows, 24, dtype=torch.float32, device=gpu)
    a = dict(q_nope=c.q_nope, q_pe=c.q_pe, kv_cache=c.cache, block_table=c.block_table, seq_lens=c.seq_lens,
             out=out, lse=lse, d_c=DC, rope_w=64, rms_offset=-1, rms_mode=_lib.RMS_NONE, kv=_lib.KV_BF16,
             page_size=64, sm_scale=c.sm_scale, qrows=4, groups=1, num_splits=0, num_workgroups=5)
    ws = Workspace().reserve(workspace_bytes(build_params(**a)), gpu)
    p = build_params(workspace=ws, **a)
    rc = qmla.lib().qmla_decode(p, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    check_decode("wide verify x4", c, out, lse)


@pytest.mark.parametrize("heads,rope,rms,qrows,splits", [
    (24, 232, "log8", 1, 0),          # deployed layout, balanced mode, 784-token pages
    (12, 116, "e4m3", 4, 0),          # 4 verify tokens, folded in pairs: 24 rows over two workgroups along z
    (12, 116, "bf16_bytes", 2, 8),    # 2 verify tokens, fixed splits
])
def test_wide_fp8_partial_rope(gpu, heads, rope, rms, qrows, splits):
    """The plugin's deployed FP8 layouts at rank 1792 (padded rope windows, unaligned rms tails)
    through `forward`: balanced and fixed splits, verify rows."""
    import qmla
    lens = [3, 1500, 4100, 790]
    c = make_case(batch=len(lens), heads=heads, d_c=DC, rope_w=rope, page_size=784, lens=lens, kv="fp8",
                  rms_mode=rms, seed=23 + heads + qrows, device=gpu, rms="spread", amp=4.0, qrows=qrows)
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, page_size=784, sm_scale=c.sm_scale,
                          kv_fp8=True, fp8_rms={"bf16_bytes": "bf16"}.get(rms, rms), k_scale=c.k_scale,
                          qrows=qrows, num_splits=splits, num_workgroups=0 if splits else 9)
    torch.cuda.synchronize()
    check_decode(f"wide fp8 rope {rope} {rms} q{qrows} S={splits}", c, o, lse, num_splits=max(splits, 1))


@pytest.mark.parametrize("page_size", [1, 40, 100])
@pytest.mark.parametrize("rms,qrows,splits", [("log8", 1, 0), ("e4m3", 4, 0), ("bf16_bytes", 2, 8)])
def test_wide_fp8_rope232_odd_pages(gpu, page_size, rms, qrows, splits):
    """The deployed FP8 rank-1792 rope-232 rows with 24 heads (16-token tiles of 32 rows) on pages
    that are not a multiple of the tile: tiles straddle pages, so every row's page is looked up per
    lane instead of one resource per tile."""
    import qmla
    lens = [3, 700, 1301, 260]
    c = make_case(batch=len(lens), heads=24, d_c=DC, rope_w=232, page_size=page_size, lens=lens, kv="fp8",
                  rms_mode=rms, seed=31 + page_size + qrows, device=gpu, rms="spread", amp=4.0, qrows=qrows)
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, page_size=page_size,
                          sm_scale=c.sm_scale, kv_fp8=True, fp8_rms={"bf16_bytes": "bf16"}.get(rms, rms),
                          k_scale=c.k_scale, qrows=qrows, num_splits=splits, num_workgroups=0 if splits else 7)
    torch.cuda.synchronize()
    check_decode(f"wide fp8 rope 232 {rms} q{qrows} S={splits} pages {page_size}", c, o, lse,
                 num_splits=max(splits, 1))
