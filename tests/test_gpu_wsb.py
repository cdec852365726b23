"""Shapes that stress the wide-row warp-specialized decode's bookkeeping rather than its arithmetic,
on each of its row formats (bf16 rows; the plugin's deployed FP8 rows at rank 768 with rope 232 and
24 heads, with rope 116 and 12 heads, and at rank 256 with bf16-byte rms), against the float32
oracle (tests.mla_cases.check_decode):

* hundreds of short requests, empty ones among them, over two workgroups: more pieces than one
  planning window holds (64), so each workgroup walks several windows and most tiles end a request;
* 1-token pages: every tile's rows come from 32 pages (per-lane page lookup), and a request needs
  more pages than one window holds (256), so its range is cut at page boundaries into windows;
* 40-token pages: tiles straddle pages;
* 256-token pages and 32 fixed splits on the reference layout;
* two long requests over 64 workgroups: each split into ~32 pieces that the combine merges.
"""
import pytest
import torch

from tests.mla_cases import check_decode, make_case

pytestmark = pytest.mark.gpu

# (name, kv, rms, d_c, rope, heads)
FAMILIES = [
    ("bf16", "bf16", "bf16", 512, 64, 24),
    ("fp8-r768-tp1", "fp8", "log8", 768, 232, 24),
    ("fp8-r768-tp2", "fp8", "e4m3", 768, 116, 12),
    ("fp8-r256-bb", "fp8", "bf16_bytes", 256, 232, 24),
]


def _case(gpu, fam, lens, page_size, seed, amp=2.0):
    _, kv, rms, d_c, rope, heads = fam
    return make_case(batch=len(lens), heads=heads, d_c=d_c, rope_w=rope, page_size=page_size, lens=lens, kv=kv,
                     rms_mode=rms, seed=seed, device=gpu, rms="spread", amp=amp)


def _forward(c, **kw):
    import qmla
    if c.kv == "fp8":
        kw.update(kv_fp8=True, fp8_rms={"bf16_bytes": "bf16"}.get(c.rms_mode, c.rms_mode), k_scale=c.k_scale)
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, d_c=c.d_c, rope_w=c.rope_w,
                          rms_offset=c.rms_offset, page_size=c.page_size, sm_scale=c.sm_scale, qrows=c.qrows, **kw)
    torch.cuda.synchronize()
    return o, lse


def _routes_to_wide_row_kernel(c):
    """The shape is served by the wide-row kernel (its plan switch charge is the warp-specialized one)."""
    import ctypes
    from qmla import _lib
    from qmla.decode import build_params
    mode = {"bf16": _lib.RMS_BF16, "log8": _lib.RMS_LOG8, "bf16_bytes": _lib.RMS_BF16_BYTES,
            "e4m3": _lib.RMS_E4M3}[c.rms_mode]
    p = build_params(q_nope=c.q_nope, q_pe=c.q_pe, kv_cache=c.cache, block_table=c.block_table,
                     seq_lens=c.seq_lens, out=c.q_nope, lse=None, d_c=c.d_c, rope_w=c.rope_w,
                     rms_offset=c.rms_offset, rms_mode=mode, kv=_lib.KV_FP8 if c.kv == "fp8" else _lib.KV_BF16,
                     page_size=c.page_size, sm_scale=c.sm_scale)
    return _lib.lib().qmla_plan_switch_tiles(ctypes.byref(p)) == 2


@pytest.mark.parametrize("fam", FAMILIES, ids=lambda f: f[0])
def test_many_short_requests_two_workgroups(gpu, fam):
    g = torch.Generator().manual_seed(51)
    lens = torch.randint(1, 100, (300,), generator=g)
    lens[::17] = 0                                  # empty requests among them
    lens = [int(x) for x in lens]
    c = _case(gpu, fam, lens, 64, seed=51)
    assert _routes_to_wide_row_kernel(c)
    o, lse = _forward(c, num_workgroups=2)
    check_decode(f"{fam[0]}: 300 short requests, 2 workgroups", c, o, lse)


@pytest.mark.parametrize("fam", FAMILIES, ids=lambda f: f[0])
def test_one_token_pages_several_windows(gpu, fam):
    c = _case(gpu, fam, [700, 45, 300], 1, seed=52)
    o, lse = _forward(c, num_workgroups=2)
    check_decode(f"{fam[0]}: 1-token pages", c, o, lse)


@pytest.mark.parametrize("fam", FAMILIES, ids=lambda f: f[0])
def test_straddling_pages(gpu, fam):
    c = _case(gpu, fam, [1000, 77, 333], 40, seed=53)
    o, lse = _forward(c, num_workgroups=5)
    check_decode(f"{fam[0]}: 40-token pages", c, o, lse)


@pytest.mark.parametrize("splits", [0, 32])
@pytest.mark.parametrize("fam", FAMILIES, ids=lambda f: f[0])
def test_large_pages(gpu, fam, splits):
    c = _case(gpu, fam, [5000, 257, 4096, 1], 256, seed=54)
    o, lse = _forward(c, num_splits=splits) if splits else _forward(c, num_workgroups=7)
    check_decode(f"{fam[0]}: 256-token pages, splits {splits}", c, o, lse, num_splits=max(splits, 1))


@pytest.mark.parametrize("fam", FAMILIES, ids=lambda f: f[0])
def test_long_requests_many_pieces(gpu, fam):
    c = _case(gpu, fam, [30000, 29001], 64, seed=55, amp=1.0)
    o, lse = _forward(c, num_workgroups=64)
    check_decode(f"{fam[0]}: 2 x 30k over 64 workgroups", c, o, lse)
