"""Each benchmarked workload, checked at its own size against the oracle through the exact call the
bench times (`bench.decode_call`: qmla_decode, balanced split mode, or 16 fixed splits plus the
combine for the wide latent):

  bf16_b64   bf16 cache, B 64, ctx U[4k, 32k], 64-token pages, seed 1
  fp8_b128   FP8 + log8, B 128, ctx lognormal (median 16k, sigma 0.5) in [1k, 64k], inputs x4, seed 2
  wide_b32   bf16, d_c 1792, B 32 x 65536 tokens, 1600-token pages, 16 fixed splits, seed 3
  gla_b48    GLA-g2 FP8 + log8, B 48 x 4 causal verify rows, ctx U[8k, 32k], seed 4
  verify_b64x4  FP8 + log8, B 64 x 4 causal verify rows x 24 heads, ctx lognormal(16k, 0.5), seed 5
  verify_bf16_b64x4  the same on bf16 rows
  fp8_r768_b128  the plugin's FP8 row at TP 1 (rank 768, rope 232, 24 log8 codes: 1024 bytes), the
                 headline's batch and lengths

The oracle runs on every 8th request plus the longest and the shortest (whole 4-row requests for
GLA-g2). The bound is the plain one: max-abs 1e-2 on the output for a bf16 cache and 3e-2 for an
FP8 cache against the float32 oracle, lse within 1e-2. The error of the reference's own roundings
(the oracle's emulation of them) is printed beside it.
"""
import pytest
import torch

import bench
from tests.mla_cases import run_oracle_requests

pytestmark = pytest.mark.gpu

TOL = {"bf16": 1e-2, "fp8": 3e-2}


def _picks(case):
    n_req = case.seq_lens.shape[0] // case.qrows
    L = case.seq_lens.view(n_req, case.qrows)[:, -1].cpu()
    picks = set(range(0, n_req, 8)) | {int(L.argmax()), int(L.argmin())}
    return sorted(picks)


@pytest.mark.parametrize("workload", ["bf16_b64", "fp8_b128", "wide_b32", "gla_b48", "verify_b64x4",
                                      "verify_bf16_b64x4", "fp8_r768_b128"])
def test_config_workload(gpu, workload):
    import qmla
    from qmla import _lib
    print(f"[config {workload}] building", flush=True)
    case, _ = bench.make_workload(workload, gpu)
    splits = bench.WORKLOADS[workload].get("splits", 0)
    p, out, lse, keep = bench.decode_call(case, splits, gpu)
    out.fill_(float("nan"))
    lse.fill_(float("nan"))
    _lib.check("qmla_decode", qmla.lib().qmla_decode(p, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    picks = _picks(case)
    print(f"[config {workload}] oracle on {len(picks)} requests", flush=True)
    ro, rl, rows = run_oracle_requests(case, picks)
    eo, _, _ = run_oracle_requests(case, picks, reference_rounding=True, num_splits=max(splits, 1))
    o = out.float().cpu()[rows]
    lg = lse.float().cpu()[rows]
    assert not torch.isnan(out.float()).any() and not torch.isnan(lse).any(), "unwritten output rows"
    err = (o - ro).abs().max().item()
    ref_err = (eo.to(torch.bfloat16).float() - ro).abs().max().item()
    lerr = (lg - rl).abs().max().item()
    tol = TOL[case.kv]
    print(f"[config {workload}] max-abs {err:.3e} (tol {tol}; reference roundings {ref_err:.3e}) lse {lerr:.3e}",
          flush=True)
    assert err < tol and lerr < 1e-2


def test_bf16_config_fp32_output(gpu):
    """The bf16 workload (B 64, ctx U[4k, 32k]) with its output written as fp32: the kernel's own error
    without the bf16 output rounding, beside the error of the reference's own roundings (keys as
    stored, P rounded to bf16 before P.V, its split-K merge) before any output cast. At bf16 output
    both sit at the output's rounding floor (about 5e-4), which hides which is smaller."""
    import qmla
    from qmla import _lib
    case, _ = bench.make_workload("bf16_b64", gpu)
    p, out, lse, keep = bench.decode_call(case, 0, gpu)
    out32 = torch.full(out.shape, float("nan"), dtype=torch.float32, device=gpu)
    p.out, p.out_dtype = out32.data_ptr(), _lib.DT_F32
    p.out_stride_row, p.out_stride_head = out32.stride(0), out32.stride(1)
    _lib.check("qmla_decode", qmla.lib().qmla_decode(p, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    picks = _picks(case)
    ro, rl, rows = run_oracle_requests(case, picks)
    eo, _, _ = run_oracle_requests(case, picks, reference_rounding=True)
    err = (out32.cpu()[rows] - ro).abs().max().item()
    ref_err = (eo - ro).abs().max().item()
    print(f"[config bf16_b64 fp32 output] max-abs {err:.3e}, reference roundings {ref_err:.3e} "
          f"(ratio {err / ref_err:.2f})", flush=True)
    assert not torch.isnan(out32).any()
    assert err < TOL["bf16"] and err <= 1.25 * ref_err
