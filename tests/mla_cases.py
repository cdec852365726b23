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
from qmla.synth import Case, lognormal_lens, make_case, uniform_lens  # noqa: E402,F401

ORACLE_RMS = {"bf16": ora.RMS_BF16, "log8": ora.RMS_LOG8, "bf16_bytes": ora.RMS_BF16_BYTES,
              "e4m3": ora.RMS_E4M3, "none": ora.RMS_NONE}


def cache_bytes(case: Case) -> torch.Tensor:
    """The cache as CPU bytes [pages, P, row_bytes]."""
    c = case.cache.detach().cpu().contiguous()
    pages, P = c.shape[0], c.shape[1]
    return c.view(torch.uint8).reshape(pages, P, -1)


def run_oracle(case: Case, rows=None, logit_cap: float = 0.0):
    """Oracle (o [rows, H, d_c/G], lse [rows, H]) in float32 on the CPU."""
    cb = cache_bytes(case)
    bt = case.block_table.cpu()
    sl = case.seq_lens.cpu()
    qn = case.q_nope.cpu().float()
    qp = case.q_pe.cpu().float()
    if rows is not None:
        bt, sl, qn, qp = bt[rows], sl[rows], qn[rows], qp[rows]
    ks = float(case.k_scale.cpu()) if case.k_scale is not None else 1.0
    return ora.mla_decode(qn, qp, cb, bt, sl, page_size=case.page_size, d_c=case.d_c, rope_w=case.rope_w,
                          rms_offset=case.rms_offset, kv=case.kv, rms_mode=ORACLE_RMS[case.rms_mode],
                          k_scale=ks, sm_scale=case.sm_scale, rms_heads=case.heads, groups=case.groups,
                          logit_cap=logit_cap)
