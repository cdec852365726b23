"""The reference-rounding mode of the oracle (`mla_decode_reference_rounding`), pinned on the CPU
against a literal restatement of the reference kernel's loop: per split, tiles of 16 tokens, the
running max, `re_scale = exp(e_max - n_e_max)`, `acc = acc * re_scale + bf16(p) @ v`,
`e_sum = e_sum * re_scale + sum(p)`, keys dequantized to bf16 (ops/mla_decode_attention.py:383-586),
then the stage-2 merge (:1097-1132) -- token by token, in float64 except where the reference rounds.
"""
import math

import pytest
import torch

from tests.mla_cases import ORACLE_RMS, cache_bytes, make_case, ora


def _bf(x):
    return x.to(torch.bfloat16).double()


def _literal(case, num_splits, align, block_n=16, logit_cap=0.0):
    cb = cache_bytes(case)
    ks = float(case.k_scale) if case.k_scale is not None else 1.0
    R, H, dcg = case.q_nope.shape
    G = case.groups
    hpg = H // G
    o = torch.zeros(R, H, dcg, dtype=torch.float64)
    lse = torch.full((R, H), -math.inf, dtype=torch.float64)
    for i in range(R):
        L = int(case.seq_lens[i])
        if L == 0:
            continue
        rows = ora.gather_rows(cb, case.block_table, i, L, case.page_size)
        c, r = ora.dequant_rows(rows, d_c=case.d_c, rope_w=case.rope_w, kv=case.kv, k_scale=ks)
        c, r = c.double(), r.double()
        if case.kv == "fp8":
            c, r = _bf(c.float()), _bf(r.float())
        rms = ora.decode_rms(rows, rms_offset=case.rms_offset, n_heads=H, kv=case.kv,
                             mode=ORACLE_RMS[case.rms_mode], k_scale=ks).double()
        for h in range(H):
            g = h // hpg
            cg = c[:, g * dcg:(g + 1) * dcg]
            q = _bf(case.q_nope[i, h].float())
            qp = _bf(case.q_pe[i, h].float())
            mid = []
            for a, e in ora.split_bounds(L, num_splits, align):
                if e <= a:
                    continue
                e_max, e_sum, acc = -math.inf, 0.0, torch.zeros(dcg, dtype=torch.float64)
                for t0 in range(a, e, block_n):
                    t1 = min(t0 + block_n, e)
                    qk = (cg[t0:t1] @ q + r[t0:t1] @ qp) / rms[t0:t1, h] * case.sm_scale
                    if logit_cap > 0:
                        qk = logit_cap * torch.tanh(qk / logit_cap)
                    n_e_max = max(float(qk.max()), e_max)
                    re_scale = math.exp(e_max - n_e_max)
                    p = torch.exp(qk - n_e_max)
                    acc = acc * re_scale + _bf(p.float()) @ cg[t0:t1]
                    e_sum = e_sum * re_scale + float(p.sum())
                    e_max = n_e_max
                mid.append((acc / e_sum, e_max + math.log(e_sum)))
            e_max, e_sum, acc = -math.inf, 0.0, torch.zeros(dcg, dtype=torch.float64)
            for tv, tl in mid:
                n_e_max = max(tl, e_max)
                old = math.exp(e_max - n_e_max)
                w = math.exp(tl - n_e_max)
                acc = acc * old + w * tv
                e_sum = e_sum * old + w
                e_max = n_e_max
            o[i, h] = acc / e_sum
            lse[i, h] = e_max + math.log(e_sum)
    return o, lse


def _emulated(case, num_splits, align, logit_cap=0.0):
    ks = float(case.k_scale) if case.k_scale is not None else 1.0
    return ora.mla_decode_reference_rounding(
        case.q_nope.float(), case.q_pe.float(), cache_bytes(case), case.block_table, case.seq_lens,
        page_size=case.page_size, d_c=case.d_c, rope_w=case.rope_w, rms_offset=case.rms_offset, kv=case.kv,
        rms_mode=ORACLE_RMS[case.rms_mode], k_scale=ks, sm_scale=case.sm_scale, rms_heads=case.heads,
        groups=case.groups, num_splits=num_splits, align=align, logit_cap=logit_cap)


@pytest.mark.parametrize("kv,rms,splits,align,groups,cap", [
    ("bf16", "bf16", 1, 16, 1, 0.0),
    ("fp8", "log8", 1, 16, 1, 0.0),
    ("fp8", "e4m3", 3, 16, 1, 0.0),
    ("fp8", "bf16_bytes", 2, 0, 1, 0.0),
    ("bf16", "bf16", 4, 16, 1, 5.0),
    ("fp8", "log8", 2, 16, 2, 0.0),
])
def test_emulation_matches_literal_loop(kv, rms, splits, align, groups, cap):
    c = make_case(batch=3, heads=4, d_c=32, rope_w=16, page_size=16, lens=[1, 37, 70], kv=kv, rms_mode=rms, seed=3,
                  amp=3.0, rms="spread", groups=groups)
    eo, el = _emulated(c, splits, align, cap)
    lo, ll = _literal(c, splits, align, logit_cap=cap)
    assert (eo.double() - lo).abs().max().item() < 2e-5 * max(1.0, lo.abs().max().item())
    assert (el.double() - ll).abs().max().item() < 1e-5


def test_emulation_rounds_what_the_reference_rounds():
    """The mode is not the plain oracle: dropping the bf16 roundings of P and of the fp8 keys (a
    plausible mistake) changes the result by the size of a bf16 step, and the emulated error against
    the float32 oracle shrinks as the context grows (the rounding errors average out)."""
    c = make_case(batch=2, heads=4, d_c=64, rope_w=16, page_size=16, lens=[8, 3000], kv="fp8", rms_mode="log8",
                  seed=9, amp=4.0)
    eo, _ = _emulated(c, 1, 16)
    ks = float(c.k_scale)
    po, _ = ora.mla_decode(c.q_nope.float(), c.q_pe.float(), cache_bytes(c), c.block_table, c.seq_lens,
                           page_size=16, d_c=64, rope_w=16, rms_offset=c.rms_offset, kv="fp8", rms_mode=ora.RMS_LOG8,
                           k_scale=ks, sm_scale=c.sm_scale, rms_heads=4)
    d = (eo - po).abs()
    assert d.max().item() > 1e-5                     # it does round
    short, long_ = d[0].max().item() / po[0].abs().max().item(), d[1].max().item() / po[1].abs().max().item()
    assert short < 2.0 ** -6 and long_ < 2.0 ** -6
