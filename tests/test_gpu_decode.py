"""GPU parity: the HIP decode against the CPU oracle on the same seeded inputs.

Tolerances (max-abs on the output, fp32 oracle): 1e-2 for a bf16 cache, 3e-2 for an fp8 cache.
LSE (natural log) within 1e-2.
"""
import math

import pytest
import torch

from tests.mla_cases import make_case, ora, run_oracle, uniform_lens

pytestmark = pytest.mark.gpu

TOL = {"bf16": 1e-2, "fp8": 3e-2}
# The output is bf16 (and P is rounded to bf16 before P.V, as in the reference kernel), so besides
# the absolute bound an element may carry rounding of up to 2^-7 of its own magnitude; this only
# matters for very short contexts where |o| is O(1).
REL = 2.0 ** -7


def _report(name, o, lse, ro, rl, tol):
    d = (o.float().cpu() - ro).abs()
    err = d.max().item()
    excess = (d - REL * ro.abs()).max().item()
    lerr = (lse.float().cpu() - rl).abs().max().item()
    print(f"[{name}] max-abs {err:.3e} (beyond bf16 rounding {excess:.3e}, tol {tol}) lse {lerr:.3e}", flush=True)
    return excess, lerr


@pytest.mark.parametrize("kv,rms_mode", [("bf16", "bf16"), ("fp8", "log8"), ("fp8", "bf16_bytes"), ("fp8", "e4m3")])
def test_forward_balanced(gpu, kv, rms_mode):
    import qmla
    lens = [1, 63, 64, 65, 700, 2047, 3000, 129]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv=kv,
                  rms_mode=rms_mode, seed=5, device=gpu, rms="spread", amp=2.0 if kv == "fp8" else 1.0)
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, page_size=c.page_size,
                          sm_scale=c.sm_scale, kv_fp8=kv == "fp8", fp8_rms={"log8": "log8", "bf16_bytes": "bf16",
                                                                          "e4m3": "e4m3", "bf16": "log8"}[rms_mode],
                          k_scale=c.k_scale, num_workgroups=5)
    torch.cuda.synchronize()
    ro, rl = run_oracle(c)
    err, lerr = _report(f"balanced {kv}/{rms_mode}", o, lse, ro, rl, TOL[kv])
    assert err < TOL[kv] and lerr < 1e-2


@pytest.mark.parametrize("splits", [1, 3, 8])
@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_reference_surface(gpu, kv, splits):
    """decode_attention_fwd: q = [latent | rope | tail], attn_logits partials, in-place outputs."""
    import qmla
    lens = [900, 77, 1600, 513]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv=kv, seed=7,
                  device=gpu, rms="spread")
    B, H = c.q_nope.shape[:2]
    q = torch.zeros(B, H, c.row - 0, dtype=torch.bfloat16, device=gpu)
    q[..., :512] = c.q_nope
    q[..., 512:576] = c.q_pe
    q[..., 576:] = 7.0          # tail columns must be ignored (Lk = rms_offset)
    o = torch.full((B, H, 512), float("nan"), dtype=torch.bfloat16, device=gpu)
    lse = torch.zeros(B, H, dtype=torch.float32, device=gpu)
    logits = torch.full((B, H, splits, 513), float("nan"), dtype=torch.float32, device=gpu)
    cache = c.cache if kv == "bf16" else c.cache.view(torch.float8_e4m3fn)
    qmla.decode_attention_fwd(q, cache, cache[..., :512], o, lse, c.block_table, c.seq_lens, logits, splits,
                              c.sm_scale, c.page_size, k_scale=c.k_scale, is_mla=True, rms_offset=576,
                              rms_log8=kv == "fp8")
    torch.cuda.synchronize()
    ro, rl = run_oracle(c)
    err, lerr = _report(f"ref-surface {kv} S={splits}", o, lse, ro, rl, TOL[kv])
    assert err < TOL[kv] and lerr < 1e-2
    if splits > 1:
        # the partials follow the reference bounds and layout exactly
        from tests.mla_cases import cache_bytes, ORACLE_RMS
        ks = float(c.k_scale.cpu()) if c.k_scale is not None else 1.0
        att = ora.mla_decode_partials(c.q_nope.cpu().float(), c.q_pe.cpu().float(), cache_bytes(c),
                                      c.block_table.cpu(), c.seq_lens.cpu(), num_splits=splits, align=16,
                                      page_size=c.page_size, d_c=512, rope_w=64, rms_offset=576, kv=kv,
                                      rms_mode=ORACLE_RMS[c.rms_mode], k_scale=ks, sm_scale=c.sm_scale)
        got = logits.cpu()
        written = ~torch.isnan(att[..., 0])
        assert torch.equal(written, ~torch.isnan(got[..., 0])), "split bounds differ from the reference"
        perr = ((got[written] - att[written]).abs() - REL * att[written].abs()).max().item()
        print(f"  partial max-abs beyond rounding {perr:.3e}")
        assert perr < TOL[kv]


def test_small_pages_config1(gpu):
    """B=4, ctx 2048, 16-token pages with a random-permutation block table, bf16 (config 1 shape)."""
    import qmla
    c = make_case(batch=4, heads=24, d_c=512, rope_w=64, page_size=16, lens=[2048] * 4, kv="bf16", seed=0,
                  device=gpu)
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, page_size=16,
                          sm_scale=c.sm_scale, num_workgroups=7)
    torch.cuda.synchronize()
    ro, rl = run_oracle(c)
    err, lerr = _report("config1 P16", o, lse, ro, rl, 1e-2)
    assert err < 1e-2 and lerr < 1e-2


def test_gla_verify(gpu):
    """GLA-g2 (2 x 256 latent, 12 heads per group) with 4-token causal verify rows, fp8 + log8."""
    import qmla
    lens = [300, 1000, 64, 2100, 5]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv="fp8",
                  rms_mode="log8", seed=4, device=gpu, qrows=4, groups=2, rms="spread")
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, d_c=512, page_size=64,
                          sm_scale=c.sm_scale, kv_fp8=True, fp8_rms="log8", k_scale=c.k_scale, qrows=4,
                          groups=2, num_workgroups=6)
    torch.cuda.synchronize()
    ro, rl = run_oracle(c)
    err, lerr = _report("gla-g2 verify", o, lse, ro, rl, 3e-2)
    assert err < 3e-2 and lerr < 1e-2


@pytest.mark.parametrize("kv,rms,d_c,qrows", [("fp8", "log8", 512, 1), ("fp8", "e4m3", 512, 1), ("bf16", "bf16", 512, 4),
                                              ("bf16", "bf16", 1792, 1)])
def test_single_split_empty_requests(gpu, kv, rms, d_c, qrows):
    """One split (final rows written by the decode kernel itself, no combine): requests of length 0
    still get a zero output and -inf lse, as every combine writes them. Outputs start as NaN."""
    import qmla
    lens = [0, 700, 0, 3, 1]
    c = make_case(batch=len(lens), heads=24, d_c=d_c, rope_w=64, page_size=64, lens=lens, kv=kv, rms_mode=rms,
                  seed=61, device=gpu, qrows=qrows, rms="spread")
    rows = c.q_nope.shape[0]
    o = torch.full((rows, 24, d_c), float("nan"), dtype=torch.bfloat16, device=gpu)
    lse = torch.full((rows, 24), float("nan"), dtype=torch.float32, device=gpu)
    kw = dict(kv_fp8=True, fp8_rms=rms, k_scale=c.k_scale) if kv == "fp8" else {}
    qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, page_size=64, sm_scale=c.sm_scale, qrows=qrows,
                 num_splits=1, out=o, lse=lse, **kw)
    torch.cuda.synchronize()
    ro, rl = run_oracle(c)
    assert not torch.isnan(o.float()).any() and not torch.isnan(lse).any(), "unwritten rows"
    err, _ = _report(f"one split {kv} {rms} d_c {d_c} q{qrows}", o, lse, ro, rl, TOL[kv])
    lg = lse.cpu()
    empty = torch.isneginf(rl)
    assert torch.equal(torch.isneginf(lg), empty)
    assert (lg[~empty] - rl[~empty]).abs().max().item() < 1e-2 and err < TOL[kv]
