"""GPU parity of the wide-latent decode (d_c = 1792, bf16 cache, rope 64, 24 heads) against the CPU
oracle: the reference routes these widths to its two-pass path (ops/mla_decode_attention.py:778-849);
the library computes them in one pass, with the same partial layout and split bounds.

Tolerance: max-abs 1e-2 on the output (bf16 cache) beyond the output's own bf16 rounding, lse 1e-2.
"""
import pytest
import torch

from tests.mla_cases import ORACLE_RMS, cache_bytes, make_case, ora, run_oracle

pytestmark = pytest.mark.gpu

TOL = 1e-2
REL = 2.0 ** -7
DC = 1792


def _report(name, o, lse, ro, rl):
    d = (o.float().cpu() - ro).abs()
    excess = (d - REL * ro.abs()).max().item()
    lerr = (lse.float().cpu() - rl).abs().max().item()
    print(f"[{name}] max-abs {d.max().item():.3e} (beyond bf16 rounding {excess:.3e}, tol {TOL}) "
          f"lse {lerr:.3e}", flush=True)
    return excess, lerr


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
    ro, rl = run_oracle(c)
    err, lerr = _report(f"wide P={page_size} S={splits}", o, lse, ro, rl)
    assert err < TOL and lerr < 1e-2
    align = 16 if page_size % 16 == 0 else 0
    att = ora.mla_decode_partials(c.q_nope.cpu().float(), c.q_pe.cpu().float(), cache_bytes(c),
                                  c.block_table.cpu(), c.seq_lens.cpu(), num_splits=splits, align=align,
                                  page_size=page_size, d_c=DC, rope_w=64, rms_offset=DC + 64, kv="bf16",
                                  rms_mode=ORACLE_RMS[c.rms_mode], sm_scale=c.sm_scale)
    got = logits.cpu()
    written = ~torch.isnan(att[..., 0])
    assert torch.equal(written, ~torch.isnan(got[..., 0])), "split bounds differ from the reference"
    perr = ((got[written] - att[written]).abs() - REL * att[written].abs()).max().item()
    print(f"  partial max-abs beyond rounding {perr:.3e}", flush=True)
    assert perr < TOL


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
    ro, rl = run_oracle(c)
    err, lerr = _report(f"wide balanced P={page_size}", o, lse, ro, rl)
    assert err < TOL and lerr < 1e-2


def test_wide_no_rms(gpu):
    """No rms tail (rms_offset < 0): plain scores."""
    import qmla
    lens = [700, 1999]
    c = make_case(batch=len(lens), heads=24, d_c=DC, rope_w=64, page_size=64, lens=lens, kv="bf16",
                  rms_mode="none", seed=9, device=gpu)
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, page_size=64, rms_offset=-1,
                          sm_scale=c.sm_scale, num_workgroups=4)
    torch.cuda.synchronize()
    ro, rl = run_oracle(c)
    err, lerr = _report("wide no-rms", o, lse, ro, rl)
    assert err < TOL and lerr < 1e-2
