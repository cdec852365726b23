"""Test helpers: synthetic cases (from qmla.synth) and the oracle run on the same inputs."""
from __future__ import annotations

import pathlib
import sys

import torch

REPO = pathlib.Path(__file__).resolve().parent.parent
for p in (REPO, REPO / "qwen-mla-vllm_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

from oracle import mla_oracle as ora  # noqa: E402
from qmla.synth import Case, compact_requests, lognormal_lens, make_case, uniform_lens  # noqa: E402,F401

# Parity bound on a decode output against the float32 oracle: plain max-abs TOL for the cache format,
# or, where the reference kernel's own roundings (fp8 keys to bf16, P to bf16 before P.V, the output
# cast) already exceed it on the same inputs, C_REF times their error (the oracle's emulation of
# those roundings, mla_decode_reference_rounding). The natural-log LSE likewise: LSE_TOL, or C_REF
# times the emulated reference's LSE error.
TOL = {"bf16": 1e-2, "fp8": 3e-2}
C_REF = 1.25
LSE_TOL = 1e-2

ORACLE_RMS = {"bf16": ora.RMS_BF16, "log8": ora.RMS_LOG8, "bf16_bytes": ora.RMS_BF16_BYTES,
              "e4m3": ora.RMS_E4M3, "none": ora.RMS_NONE}


def cache_bytes(case: Case) -> torch.Tensor:
    """The cache as CPU bytes [pages, P, row_bytes]."""
    c = case.cache.detach().cpu().contiguous()
    pages, P = c.shape[0], c.shape[1]
    return c.view(torch.uint8).reshape(pages, P, -1)


def run_oracle(case: Case, rows=None, logit_cap: float = 0.0, reference_rounding: bool = False,
               num_splits: int = 1, align: int = 16):
    """Oracle (o [rows, H, d_c/G], lse [rows, H]) in float32 on the CPU. With reference_rounding,
    the oracle's emulation of the reference kernel's roundings (num_splits / align: its splits)."""
    cb = cache_bytes(case)
    bt = case.block_table.cpu()
    sl = case.seq_lens.cpu()
    qn = case.q_nope.cpu().float()
    qp = case.q_pe.cpu().float()
    if rows is not None:
        bt, sl, qn, qp = bt[rows], sl[rows], qn[rows], qp[rows]
    ks = float(case.k_scale.cpu()) if case.k_scale is not None else 1.0
    kw = dict(page_size=case.page_size, d_c=case.d_c, rope_w=case.rope_w, rms_offset=case.rms_offset, kv=case.kv,
              rms_mode=ORACLE_RMS[case.rms_mode], k_scale=ks, sm_scale=case.sm_scale, rms_heads=case.heads,
              groups=case.groups, logit_cap=logit_cap)
    if reference_rounding:
        return ora.mla_decode_reference_rounding(qn, qp, cb, bt, sl, num_splits=num_splits, align=align, **kw)
    return ora.mla_decode(qn, qp, cb, bt, sl, **kw)


def run_oracle_requests(case: Case, reqs, logit_cap: float = 0.0, reference_rounding: bool = False,
                        num_splits: int = 1, align: int = 16):
    """Oracle on the requests `reqs` only: (o, lse, rows). With reference_rounding, the oracle's
    emulation of the reference kernel's roundings (its own error against the float32 oracle)."""
    cache, bt, sl, qn, qp, rows = compact_requests(case, reqs)
    ks = float(case.k_scale.cpu()) if case.k_scale is not None else 1.0
    kw = dict(page_size=case.page_size, d_c=case.d_c, rope_w=case.rope_w, rms_offset=case.rms_offset, kv=case.kv,
              rms_mode=ORACLE_RMS[case.rms_mode], k_scale=ks, sm_scale=case.sm_scale, rms_heads=case.heads,
              groups=case.groups, logit_cap=logit_cap)
    if reference_rounding:
        o, lse = ora.mla_decode_reference_rounding(qn, qp, cache, bt, sl, num_splits=num_splits, align=align, **kw)
    else:
        o, lse = ora.mla_decode(qn, qp, cache, bt, sl, **kw)
    return o, lse, rows


def check_decode(name: str, case: Case, o, lse, *, logit_cap: float = 0.0, num_splits: int = 1, align: int = 16,
                 tol: float | None = None, ro=None, rl=None):
    """Assert the parity bound for a decode output o [rows, H, dv] (any float dtype) and its lse
    against the oracle on the same case; prints the plain max-abs, the reference roundings' error
    and the bound. Returns (err, ref_err, lse_err)."""
    if ro is None:
        ro, rl = run_oracle(case, logit_cap=logit_cap)
    eo, el = run_oracle(case, logit_cap=logit_cap, reference_rounding=True, num_splits=num_splits, align=align)
    of = o.float().cpu()
    err = (of - ro).abs().max().item()
    ref_err = (eo.to(o.dtype).float() - ro).abs().max().item()
    tol = TOL[case.kv] if tol is None else tol
    bound = max(tol, C_REF * ref_err)
    lerr, ref_lerr = 0.0, 0.0
    if lse is not None:
        lg = lse.float().cpu()
        empty = torch.isneginf(rl)
        assert torch.equal(torch.isneginf(lg), empty), f"[{name}] rows without tokens differ"
        if (~empty).any():
            lerr = (lg[~empty] - rl[~empty]).abs().max().item()
            ref_lerr = (el[~empty] - rl[~empty]).abs().max().item()
    lbound = max(LSE_TOL, C_REF * ref_lerr)
    # which clause decides: the plain tolerance, or C_REF x the reference roundings' own error
    clause = "plain" if err < tol else f"reference x{C_REF}"
    lclause = "plain" if lerr < LSE_TOL else f"reference x{C_REF}"
    print(f"[{name}] max-abs {err:.3e} (tol {tol}, reference roundings {ref_err:.3e}, bound {bound:.3e}: {clause}) "
          f"lse {lerr:.3e} (reference {ref_lerr:.3e}, bound {lbound:.3e}: {lclause})", flush=True)
    assert err < bound, f"[{name}] max-abs {err:.3e} >= bound {bound:.3e}"
    assert lerr < lbound, f"[{name}] lse error {lerr:.3e} >= bound {lbound:.3e}"
    return err, ref_err, lerr


def check_partials(name: str, case: Case, got, *, num_splits: int, align: int, tol: float | None = None):
    """The attn_logits partials [rows, H, S, dv + 1] against the oracle's: written exactly where the
    reference's split bounds put a non-empty split, and within the parity bound (the emulated
    reference partials' own error, C_REF times, where it exceeds the plain bound)."""
    cb = cache_bytes(case)
    ks = float(case.k_scale.cpu()) if case.k_scale is not None else 1.0
    kw = dict(page_size=case.page_size, d_c=case.d_c, rope_w=case.rope_w, rms_offset=case.rms_offset, kv=case.kv,
              rms_mode=ORACLE_RMS[case.rms_mode], k_scale=ks, sm_scale=case.sm_scale)
    args = (case.q_nope.cpu().float(), case.q_pe.cpu().float(), cb, case.block_table.cpu(), case.seq_lens.cpu())
    att = ora.mla_decode_partials(*args, num_splits=num_splits, align=align, **kw)
    emu = ora.mla_decode_reference_rounding(*args, num_splits=num_splits, align=align, rms_heads=case.heads,
                                            partials=True, **kw)
    got = got.float().cpu()
    written = ~torch.isnan(att[..., 0])
    assert torch.equal(written, ~torch.isnan(got[..., 0])), f"[{name}] split bounds differ from the reference"
    err = (got[written] - att[written]).abs().max().item() if written.any() else 0.0
    ref_err = (emu[written] - att[written]).abs().max().item() if written.any() else 0.0
    tol = TOL[case.kv] if tol is None else tol
    bound = max(tol, C_REF * ref_err)
    print(f"  [{name}] partials max-abs {err:.3e} (reference roundings {ref_err:.3e}, bound {bound:.3e})", flush=True)
    assert err < bound
