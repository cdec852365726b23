"""Pins the oracle's decode arithmetic on the CPU.

* brute force: plain float64 Python loops over tiny paged caches, reading the cache through torch's
  own bfloat16 / float8_e4m3fn views (not the oracle's decoders), for every cache/rms format;
* closed forms: zero queries give the mean of the latent rows and lse = ln L; identical rows give
  that row; rms <= 0 divides by 1 (ops/mla_decode_attention.py:505);
* LSE algebra: every split count and alignment recombines to the unsplit result, with the
  reference's split bounds (ops/mla_decode_attention.py:389-396, :1097-1109);
* verify rows: the flattened per-row lengths (mla_impl.py:628-662) against explicit limits;
* GLA-g2: group-g output equals the full-width decode with the query zero outside group g
  (mla_impl.py:182-194, qwen3_5_mla.py:379-389);
* invariance under page renumbering.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import mla_oracle as ora
from tests.mla_cases import ORACLE_RMS, cache_bytes, make_case, run_oracle

F8 = getattr(torch, "float8_e4m3fn", None)


def _brute(case, rows=None, logit_cap: float = 0.0):
    """float64 loops: o [R, H, dv], lse [R, H] straight from the spec, no vectorized oracle code."""
    cb = cache_bytes(case)
    bt = case.block_table.cpu().tolist()
    sl = case.seq_lens.cpu().tolist()
    qn = case.q_nope.cpu().double().tolist()
    qp = case.q_pe.cpu().double().tolist()
    d_c, W, H, P, G = case.d_c, case.rope_w, case.heads, case.page_size, case.groups
    dv = d_c // G
    hpg = H // G
    ks = float(case.k_scale) if case.k_scale is not None else 1.0
    R = len(sl)
    o = np.zeros((R, H, dv))
    lse = np.full((R, H), -math.inf)
    for i in range(R if rows is None else rows):
        L = sl[i]
        toks = []
        for n in range(L):
            raw = cb[bt[i][n // P], n % P]
            if case.kv == "bf16":
                el = raw.contiguous().view(torch.bfloat16).double().tolist()
                lat, rope = el[:d_c], el[d_c:d_c + W]
                rms = [1.0] * H if case.rms_mode == "none" else el[d_c + W:d_c + W + H]
            else:
                vals = (raw[:d_c + W].contiguous().view(F8).double() * ks).tolist()
                lat, rope = vals[:d_c], vals[d_c:d_c + W]
                off = d_c + W
                codes = raw.tolist()
                if case.rms_mode == "log8":
                    rms = [2.0 ** (-3 + codes[off + h] * 6 / 255) for h in range(H)]
                elif case.rms_mode == "bf16_bytes":
                    rms = raw[off:off + 2 * H].contiguous().view(torch.bfloat16).double().tolist()
                elif case.rms_mode == "e4m3":
                    rms = (raw[off:off + H].contiguous().view(F8).double() * ks).tolist()
                else:
                    rms = [1.0] * H
            toks.append((lat, rope, rms))
        if L == 0:
            continue
        for h in range(H):
            g = h // hpg
            cols = range(g * dv, (g + 1) * dv)
            s = []
            for lat, rope, rms in toks:
                dot = math.fsum(qn[i][h][j] * lat[c] for j, c in enumerate(cols))
                dot += math.fsum(qp[i][h][j] * rope[j] for j in range(W))
                div = rms[h] if rms[h] > 0 else 1.0
                v = dot / div * case.sm_scale
                if logit_cap > 0:
                    v = logit_cap * math.tanh(v / logit_cap)
                s.append(v)
            m = max(s)
            e = [math.exp(x - m) for x in s]
            tot = math.fsum(e)
            for j, c in enumerate(cols):
                o[i, h, j] = math.fsum(e[n] * toks[n][0][c] for n in range(L)) / tot
            lse[i, h] = m + math.log(tot)
    return torch.from_numpy(o).float(), torch.from_numpy(lse).float()


def _oracle(case, logit_cap=0.0):
    cb = cache_bytes(case)
    ks = float(case.k_scale) if case.k_scale is not None else 1.0
    return ora.mla_decode(case.q_nope.float(), case.q_pe.float(), cb, case.block_table, case.seq_lens,
                          page_size=case.page_size, d_c=case.d_c, rope_w=case.rope_w, rms_offset=case.rms_offset,
                          kv=case.kv, rms_mode=ORACLE_RMS[case.rms_mode], k_scale=ks, sm_scale=case.sm_scale,
                          logit_cap=logit_cap, rms_heads=case.heads, groups=case.groups)


def _close(a, b, tol=2e-5):
    fin = torch.isfinite(b)
    assert torch.equal(torch.isfinite(a), fin)
    assert (a[fin] - b[fin]).abs().max().item() < tol


FORMATS = [("bf16", "bf16"), ("bf16", "none"), ("fp8", "log8"), ("fp8", "bf16_bytes"), ("fp8", "e4m3")]


@pytest.mark.parametrize("kv,rms", FORMATS)
def test_bruteforce_formats(kv, rms):
    case = make_case(batch=4, heads=3, d_c=16, rope_w=8, page_size=4, lens=[0, 1, 7, 13], kv=kv, rms_mode=rms,
                     seed=5, rms="spread", amp=2.0)
    o, lse = _oracle(case)
    bo, blse = _brute(case)
    _close(o, bo)
    _close(lse, blse)
    assert torch.all(o[0] == 0) and torch.all(torch.isneginf(lse[0]))   # empty row


def test_bruteforce_logit_cap():
    case = make_case(batch=2, heads=2, d_c=16, rope_w=8, page_size=4, lens=[6, 9], kv="fp8", seed=6, q_amp=8.0)
    o, lse = _oracle(case, logit_cap=5.0)
    bo, blse = _brute(case, logit_cap=5.0)
    _close(o, bo)
    _close(lse, blse)


def test_nonpositive_rms_divides_by_one():
    case = make_case(batch=1, heads=2, d_c=16, rope_w=8, page_size=4, lens=[8], kv="bf16", seed=7)
    flat = case.cache.view(-1, case.row)
    off = case.rms_offset
    flat[:, off] = 0.0
    flat[:, off + 1] = -3.0
    o, lse = _oracle(case)
    none = make_case(batch=1, heads=2, d_c=16, rope_w=8, page_size=4, lens=[8], kv="bf16", seed=7, rms_mode="none")
    none.cache.view(-1, none.row)[:, :off] = flat[:, :off]
    o1, lse1 = _oracle(none)
    _close(o, o1, 1e-6)
    _close(lse, lse1, 1e-6)


def test_closed_forms():
    case = make_case(batch=2, heads=3, d_c=16, rope_w=8, page_size=4, lens=[5, 11], kv="bf16", seed=8)
    case.q_nope.zero_()
    case.q_pe.zero_()
    o, lse = _oracle(case)
    cb = cache_bytes(case)
    for i, L in enumerate([5, 11]):
        rows = ora.gather_rows(cb, case.block_table, i, L, case.page_size).contiguous().view(torch.bfloat16).float()
        mean = rows[:, :16].mean(0)
        assert (o[i] - mean).abs().max() < 1e-6
        assert (lse[i] - math.log(L)).abs().max() < 1e-6
    # every token the same row: the output is that row, whatever the query
    case2 = make_case(batch=1, heads=2, d_c=16, rope_w=8, page_size=4, lens=[9], kv="bf16", seed=9)
    flat = case2.cache.view(-1, case2.row)
    flat[:] = flat[0]
    o2, _ = _oracle(case2)
    assert (o2[0] - flat[0, :16].float()).abs().max() < 1e-6


def test_split_bounds_known_answers():
    assert ora.split_bounds(100, 3, 16) == [(0, 48), (48, 96), (96, 100)]
    assert ora.split_bounds(100, 3, 0) == [(0, 34), (34, 68), (68, 100)]
    b = ora.split_bounds(10, 4, 16)
    assert b[0] == (0, 10) and all(e <= a for a, e in b[1:])
    assert ora.split_bounds(0, 2, 16) == [(0, 0), (0, 0)]


@pytest.mark.parametrize("align", [0, 16])
def test_split_combine_invariance(align):
    case = make_case(batch=3, heads=2, d_c=32, rope_w=8, page_size=16, lens=[1, 40, 97], kv="fp8", seed=10)
    o, lse = _oracle(case)
    cb = cache_bytes(case)
    ks = float(case.k_scale)
    for S in (1, 2, 3, 5, 8):
        att = ora.mla_decode_partials(case.q_nope.float(), case.q_pe.float(), cb, case.block_table, case.seq_lens,
                                      num_splits=S, align=align, page_size=16, d_c=32, rope_w=8,
                                      rms_offset=case.rms_offset, kv="fp8", rms_mode=ora.RMS_LOG8, k_scale=ks,
                                      sm_scale=case.sm_scale)
        for i, L in enumerate([1, 40, 97]):
            for s, (a, e) in enumerate(ora.split_bounds(L, S, align)):
                assert bool(torch.isnan(att[i, :, s]).all()) == (e <= a)
        co, clse = ora.combine_partials(att, case.seq_lens, num_splits=S, align=align)
        _close(co, o, 2e-6)
        _close(clse, lse, 2e-6)


def test_verify_flattening():
    bt = np.arange(6, dtype=np.int32).reshape(2, 3)
    fbt, fsl = ora.flatten_verify(bt, np.array([5, 2], np.int32), 3)
    assert fsl.tolist() == [3, 4, 5, 0, 1, 2]
    assert fbt.tolist() == [[0, 1, 2]] * 3 + [[3, 4, 5]] * 3
    # the flattened rows attend exactly to the causal prefix of each draft token
    case = make_case(batch=2, heads=2, d_c=16, rope_w=8, page_size=4, lens=[6, 10], kv="bf16", seed=12, qrows=4)
    assert case.seq_lens.tolist() == [3, 4, 5, 6, 7, 8, 9, 10]
    o, lse = _oracle(case)
    bo, blse = _brute(case)
    _close(o, bo)
    _close(lse, blse)


def test_gla_equals_zero_embedded_full_width():
    case = make_case(batch=2, heads=4, d_c=32, rope_w=8, page_size=4, lens=[7, 12], kv="fp8", seed=13, groups=2)
    o, lse = _oracle(case)
    qfull = torch.zeros(2, 4, 32)
    qfull[:, :2, :16] = case.q_nope[:, :2].float()
    qfull[:, 2:, 16:] = case.q_nope[:, 2:].float()
    cb = cache_bytes(case)
    of, lf = ora.mla_decode(qfull, case.q_pe.float(), cb, case.block_table, case.seq_lens, page_size=4, d_c=32,
                            rope_w=8, rms_offset=case.rms_offset, kv="fp8", rms_mode=ora.RMS_LOG8,
                            k_scale=float(case.k_scale), sm_scale=case.sm_scale)
    _close(o[:, :2], of[:, :2, :16], 1e-5)
    _close(o[:, 2:], of[:, 2:, 16:], 1e-5)
    _close(lse, lf, 1e-5)
    bo, blse = _brute(case)
    _close(o, bo)


def test_page_renumbering_invariance():
    case = make_case(batch=2, heads=2, d_c=16, rope_w=8, page_size=4, lens=[9, 14], kv="fp8", seed=14)
    o, lse = _oracle(case)
    pages = case.cache.shape[0]
    perm = torch.randperm(pages, generator=torch.Generator().manual_seed(3))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(pages)
    case.cache = case.cache[perm].contiguous()              # new page p holds old page perm[p]
    case.block_table = inv[case.block_table.long()].to(torch.int32)
    o2, lse2 = _oracle(case)
    assert torch.equal(o, o2) and torch.equal(lse, lse2)


def test_run_oracle_matches_direct_call():
    case = make_case(batch=2, heads=3, d_c=16, rope_w=8, page_size=4, lens=[3, 8], kv="fp8", seed=15)
    a = run_oracle(case)
    b = _oracle(case)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
