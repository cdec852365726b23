"""Output and lse element types: the decode writes bf16, fp16 or fp32 outputs and lse (the
reference's stage 2 stores fp16 when the output is fp16, ops/mla_decode_attention.py:1125-1131)
from every store path: the kernels' own final rows (one split, or a request one workgroup finished),
the fixed-split combine and the balanced combine. Each kernel family once, against the oracle;
outputs start as NaN so an unwritten element fails.
"""
import pytest
import torch

from tests.mla_cases import check_decode, make_case

pytestmark = pytest.mark.gpu

# (kv, rms, d_c, heads, qrows, groups, rope_w); wide_fp8: the plugin's FP8 rank-1792 row (rope 232 in a
# 256-column window, 32x32 P.V, fp16 partials through the 8-column combine)
FAMILIES = {
    "ws": ("fp8", "log8", 512, 24, 1, 1, 64),
    "gla": ("fp8", "log8", 512, 24, 4, 2, 64),
    "partial": ("bf16", "bf16", 512, 24, 1, 1, 64),
    "wide": ("bf16", "bf16", 1792, 24, 1, 1, 64),
    "wide_fp8": ("fp8", "log8", 1792, 24, 1, 1, 232),
}
DTYPES = {"f16": torch.float16, "f32": torch.float32}


@pytest.mark.parametrize("splits", [0, 1, 4])
@pytest.mark.parametrize("dt", sorted(DTYPES))
@pytest.mark.parametrize("family", sorted(FAMILIES))
def test_output_types(gpu, family, dt, splits):
    import qmla
    kv, rms, d_c, heads, qrows, groups, rope_w = FAMILIES[family]
    lens = [0, 900, 2500, 5]
    c = make_case(batch=len(lens), heads=heads, d_c=d_c, rope_w=rope_w, page_size=64, lens=lens, kv=kv, rms_mode=rms,
                  seed=71, device=gpu, qrows=qrows, groups=groups, rms="spread")
    rows = c.q_nope.shape[0]
    o = torch.full((rows, heads, d_c // groups), float("nan"), dtype=DTYPES[dt], device=gpu)
    lse = torch.full((rows, heads), float("nan"), dtype=DTYPES[dt], device=gpu)
    kw = dict(kv_fp8=True, fp8_rms=rms, k_scale=c.k_scale) if kv == "fp8" else {}
    qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, d_c=d_c, page_size=64, sm_scale=c.sm_scale,
                 qrows=qrows, groups=groups, num_splits=splits, num_workgroups=5 if splits == 0 else 0, out=o, lse=lse,
                 **kw)
    torch.cuda.synchronize()
    got, gl = o.float().cpu(), lse.float().cpu()
    assert not torch.isnan(got).any() and not torch.isnan(gl).any(), "unwritten elements"
    check_decode(f"{family} {dt} S={splits}", c, o, lse, num_splits=max(splits, 1))
