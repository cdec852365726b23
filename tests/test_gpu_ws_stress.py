"""Shapes that stress the warp-specialized decode's bookkeeping rather than its arithmetic, against
the CPU oracle (same tolerances as tests/test_gpu_ws.py):

* hundreds of short requests, empty ones among them, over two workgroups: more pieces than one
  planning window holds (64), so each workgroup walks several windows, and most tiles end a request;
* two 60k-token requests over 64 workgroups: each request is split into ~32 pieces whose partials
  the combine merges in batches;
* 256-token pages (tiles never straddle a page) and 32 fixed splits on the reference layout.
"""
import pytest
import torch

from tests.mla_cases import make_case
from tests.test_gpu_ws import _check, _forward

pytestmark = pytest.mark.gpu


def test_many_short_requests_two_workgroups(gpu):
    g = torch.Generator().manual_seed(41)
    lens = torch.randint(1, 100, (300,), generator=g)
    lens[::17] = 0                                  # empty requests among them
    lens = [int(x) for x in lens]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv="fp8", rms_mode="log8",
                  seed=41, device=gpu, rms="spread", amp=4.0)
    o, lse = _forward(c, num_workgroups=2)
    _check("300 short requests, 2 workgroups", c, o, lse)


def test_long_requests_many_pieces(gpu):
    lens = [60000, 59001]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv="fp8", rms_mode="log8",
                  seed=42, device=gpu, rms="spread")
    o, lse = _forward(c, num_workgroups=64)
    _check("2 x 60k over 64 workgroups", c, o, lse)


@pytest.mark.parametrize("splits", [0, 32])
def test_large_pages(gpu, splits):
    lens = [5000, 257, 4096, 1]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=256, lens=lens, kv="fp8", rms_mode="log8",
                  seed=43, device=gpu, rms="spread", amp=4.0)
    o, lse = _forward(c, num_splits=splits) if splits else _forward(c, num_workgroups=7)
    _check(f"256-token pages, splits {splits}", c, o, lse)
