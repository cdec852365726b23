"""CPU oracle for absorbed-MLA latent-KV decode attention.

TEST INFRASTRUCTURE ONLY. This module is the oracle the tests compare against, never the product:
only the test suite (`tests/`), `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`
may import it. The product path (`qmla`) never calls it and fails loudly when its HIP library is
missing.

It restates, on the CPU, the arithmetic of the reference plugin's decode path:

* paged cache rows `[latent d_c | rope W | rms tail | pad]` addressed through a block table
  (ops/mla_decode_attention.py:412-440, mla_impl.py:148-165);
* the per-(token, head) score divisor in its four storage modes
  (ops/mla_decode_attention.py:466-505, mla_impl.py:125-145);
* FP8 e4m3fn latent/rope with one per-layer scale (ops/mla_decode_attention.py:451-463,
  mla_impl.py:309-342);
* scores `(q_lat.c + q_pe.r) / rms * sm_scale`, optional tanh cap, softmax, `o = P.c`, natural-log
  LSE (ops/mla_decode_attention.py:453-586, :1125-1137; tests/test_decode_numerics.py:25-44);
* split-KV partials and their LSE combine with the reference's tile-aligned split bounds
  (ops/mla_decode_attention.py:383-396, :1097-1137);
* spec-verify row flattening (mla_impl.py:628-662) and the grouped-latent (GLA) head/column mapping
  (mla_impl.py:182-194, qwen3_5_mla.py:58-73);
* the FP8 cache-row writer (mla_impl.py:309-342) and the prefill context gather
  (ops/mla_gather.py:28-76);
* the decode q / k_pe prep of the attention module (qwen3_5_mla.py:232-301, :341-354) and the
  partial-rope cos/sin table (partial_rope.py:66-76).

Floating-point work runs in float32 torch on the CPU; byte work (e4m3fn and log8 codes) is numpy
bit arithmetic. Every function is pinned by tests against closed forms, brute force on tiny
inputs, torch's own float8_e4m3fn conversion, and the known answers quoted in the reference's
docstrings and tests (tests/test_oracle_*.py).
"""
from __future__ import annotations

import math

import numpy as np
import torch

# rms log8 code range: rms = 2 ** (LO + code * (HI - LO) / 255)  (mla_impl.py:132)
RMS_LOG2_LO, RMS_LOG2_HI = -3.0, 3.0
E4M3_MAX = 448.0

KV_BF16, KV_FP8 = "bf16", "fp8"
# rms tail formats: one bf16 element per head in a bf16 cache; for an FP8 cache a uint8 log2 code,
# two raw bf16 bytes, or one e4m3 byte scaled like the row (mla_impl.py:125-145).
RMS_NONE, RMS_BF16, RMS_LOG8, RMS_BF16_BYTES, RMS_E4M3 = "none", "bf16", "log8", "bf16_bytes", "e4m3"


# ------------------------------------------------------------------------------------------------
# e4m3fn (OCP FP8: 1 sign, 4 exponent bits with bias 7, 3 mantissa bits, no inf, NaN = S.1111.111)
# ------------------------------------------------------------------------------------------------
def _e4m3_table() -> np.ndarray:
    t = np.zeros(256, dtype=np.float32)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 7
        if e == 15 and m == 7:
            t[b] = np.nan
        elif e == 0:
            t[b] = s * (m / 8.0) * 2.0 ** -6
        else:
            t[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


E4M3_TABLE = _e4m3_table()


def e4m3_decode(b: np.ndarray) -> np.ndarray:
    """uint8 e4m3fn codes -> float32 values (exact)."""
    return E4M3_TABLE[np.asarray(b, dtype=np.uint8)]


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 values already clamped to [-448, 448] -> e4m3fn codes, round to nearest even.

    Restates `.to(torch.float8_e4m3fn)` after the writer's clamp (mla_impl.py:331-332). Works in
    float64 so every step is exact; NaN inputs map to 0x7F.
    """
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    out = np.zeros(x.shape, dtype=np.uint8)
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.uint8)
    a = np.abs(x)
    nan = np.isnan(a)
    a = np.where(nan, 0.0, np.minimum(a, E4M3_MAX))
    # subnormal grid: multiples of 2^-9 below 2^-6
    sub = a < 2.0 ** -6
    q_sub = np.rint(a / 2.0 ** -9)                      # 0..8; 8 rounds up to the first normal
    code_sub = q_sub.astype(np.int64)                   # exponent field 0 (or 1 when q_sub == 8)
    # normal: a = 2^e * (1 + m/8), e in [-6, 8]
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(sub, 1.0, a)))
    e = np.clip(e, -6, 8)
    frac = np.where(sub, 0.0, a / 2.0 ** e)             # in [1, 2)
    q = np.rint((frac - 1.0) * 8.0)                     # 0..8
    carry = q >= 8
    e = np.where(carry, e + 1, e)
    q = np.where(carry, 0, q)
    code_norm = ((e + 7).astype(np.int64) << 3) | q.astype(np.int64)
    code_norm = np.minimum(code_norm, 0x7E)             # 448 is the largest finite value
    code = np.where(sub, code_sub, code_norm)
    out = (code.astype(np.uint8) | sign)
    out = np.where(nan, np.uint8(0x7F), out).astype(np.uint8)
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even (NaN kept quiet)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    rounded = np.where(nan, (u >> 16) | 0x40, rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------------------------------------------
# rms divisor codes
# ------------------------------------------------------------------------------------------------
def log8_encode(rms: np.ndarray) -> np.ndarray:
    """rms (float32) -> uint8 code, as the FP8 row writer stores it (mla_impl.py:333-336).

    `(log2(max(rms, 1e-30)) - LO) * (255 / (HI - LO))`, rounded half-to-even, clamped to [0, 255].
    The products and the subtraction are float32 operations as in the writer; log2 is evaluated
    correctly rounded to float32 (through float64).
    """
    r = np.maximum(np.asarray(rms, dtype=np.float32), np.float32(1e-30))
    lg = np.log2(r.astype(np.float64)).astype(np.float32)
    code = (lg - np.float32(RMS_LOG2_LO)) * np.float32(255.0 / (RMS_LOG2_HI - RMS_LOG2_LO))
    return np.clip(np.rint(code.astype(np.float32)), 0, 255).astype(np.uint8)


def log8_decode(code: np.ndarray) -> np.ndarray:
    """uint8 code -> rms = 2^(-3 + code * 6/255) (ops/mla_decode_attention.py:470-479)."""
    c = np.asarray(code, dtype=np.float64)
    return np.exp2(RMS_LOG2_LO + c * ((RMS_LOG2_HI - RMS_LOG2_LO) / 255.0)).astype(np.float32)


# ------------------------------------------------------------------------------------------------
# paged rows
# ------------------------------------------------------------------------------------------------
def gather_rows(cache_u8: torch.Tensor, block_table: torch.Tensor, b: int, length: int,
                page_size: int) -> torch.Tensor:
    """Rows [length, row_bytes] of sequence b: token n lives at page block_table[b, n // P],
    slot n % P (ops/mla_decode_attention.py:412-440)."""
    if length == 0:
        return cache_u8.new_zeros((0, cache_u8.shape[-1]))
    n = torch.arange(length)
    pages = block_table[b, n // page_size].long()
    return cache_u8[pages, n % page_size]


def dequant_rows(rows: torch.Tensor, *, d_c: int, rope_w: int, kv: str, k_scale: float):
    """Latent and rope of each row as float32. fp8 rows decode e4m3fn and multiply by the one
    per-layer scale shared by latent and rope (ops/mla_decode_attention.py:451-463)."""
    if kv == KV_BF16:
        el = rows.contiguous().view(torch.bfloat16).float()
        return el[:, :d_c], el[:, d_c:d_c + rope_w]
    vals = torch.from_numpy(e4m3_decode(rows[:, :d_c + rope_w].numpy())) * np.float32(k_scale)
    return vals[:, :d_c], vals[:, d_c:d_c + rope_w]


def decode_rms(rows: torch.Tensor, *, rms_offset: int, n_heads: int, kv: str, mode: str,
               k_scale: float) -> torch.Tensor:
    """Per-(token, head) divisor [L, n_heads] in float32; rms <= 0 reads as 1
    (ops/mla_decode_attention.py:466-505). rms_offset is in cache elements."""
    L = rows.shape[0]
    if mode == RMS_NONE:
        return torch.ones(L, n_heads)
    if kv == KV_BF16:
        assert mode == RMS_BF16
        el = rows.contiguous().view(torch.bfloat16).float()
        r = el[:, rms_offset:rms_offset + n_heads]
    elif mode == RMS_LOG8:
        r = torch.from_numpy(log8_decode(rows[:, rms_offset:rms_offset + n_heads].numpy()))
    elif mode == RMS_BF16_BYTES:
        raw = rows[:, rms_offset:rms_offset + 2 * n_heads].contiguous()
        r = raw.view(torch.bfloat16).float()
    elif mode == RMS_E4M3:
        r = torch.from_numpy(e4m3_decode(rows[:, rms_offset:rms_offset + n_heads].numpy())) * np.float32(k_scale)
    else:
        raise ValueError(mode)
    return torch.where(r > 0, r, torch.ones_like(r))


# ------------------------------------------------------------------------------------------------
# decode
# ------------------------------------------------------------------------------------------------
def _scores(q_lat, q_pe, c, r, rms, sm_scale, logit_cap):
    """[H, L] scores: divide by rms, then scale, then optional tanh cap
    (ops/mla_decode_attention.py:453-514)."""
    s = q_lat @ c.T
    if q_pe is not None and q_pe.shape[-1]:
        s = s + q_pe @ r.T
    s = s / rms.T
    s = s * sm_scale
    if logit_cap > 0:
        s = logit_cap * torch.tanh(s / logit_cap)
    return s


def mla_decode(q_lat: torch.Tensor, q_pe: torch.Tensor | None, cache_u8: torch.Tensor,
               block_table: torch.Tensor, seq_lens: torch.Tensor, *, page_size: int, d_c: int,
               rope_w: int, rms_offset: int, kv: str, rms_mode: str, k_scale: float = 1.0,
               sm_scale: float, logit_cap: float = 0.0, rms_heads: int | None = None,
               groups: int = 1, rms_head_of_row=None):
    """Full (unsplit) decode for every query row.

    q_lat [R, H, d_c/groups] absorbed latent queries, q_pe [R, H, W] rope queries. Row i attends to
    the first seq_lens[i] tokens of block_table[i]. With `groups` > 1 (GLA) head h belongs to group
    g = h // (H/groups) and reads latent columns [g*d_c/G, (g+1)*d_c/G) for both scores and values
    (mla_impl.py:182-194). `rms_head_of_row(h)` maps a query head to its rms slot (default h).
    Returns o [R, H, d_c/groups] and natural-log lse [R, H], float32.
    """
    R, H, dcg = q_lat.shape
    assert dcg * groups == d_c
    n_rms = rms_heads if rms_heads is not None else H
    hpg = H // groups
    o = torch.zeros(R, H, dcg)
    lse = torch.full((R, H), -math.inf)
    for i in range(R):
        L = int(seq_lens[i])
        if L <= 0:
            continue
        rows = gather_rows(cache_u8, block_table, i, L, page_size)
        c, r = dequant_rows(rows, d_c=d_c, rope_w=rope_w, kv=kv, k_scale=k_scale)
        rms = decode_rms(rows, rms_offset=rms_offset, n_heads=n_rms, kv=kv, mode=rms_mode,
                         k_scale=k_scale)
        heads = torch.arange(H)
        rh = heads if rms_head_of_row is None else torch.tensor([rms_head_of_row(int(h)) for h in heads])
        rms_h = rms[:, rh]
        for g in range(groups):
            hs = slice(g * hpg, (g + 1) * hpg)
            cg = c[:, g * dcg:(g + 1) * dcg]
            s = _scores(q_lat[i, hs].float(), None if q_pe is None else q_pe[i, hs].float(), cg, r,
                        rms_h[:, hs], sm_scale, logit_cap)
            m = s.max(dim=-1, keepdim=True).values
            p = torch.exp(s - m)
            l = p.sum(-1, keepdim=True)
            o[i, hs] = (p @ cg) / l
            lse[i, hs] = (m + torch.log(l)).squeeze(-1)
    return o, lse


def _bf16_t(x: torch.Tensor) -> torch.Tensor:
    """float32 tensor -> nearest-even bf16 values, as float32."""
    return x.to(torch.bfloat16).float()


def mla_decode_reference_rounding(q_lat: torch.Tensor, q_pe: torch.Tensor | None, cache_u8: torch.Tensor,
                                  block_table: torch.Tensor, seq_lens: torch.Tensor, *, page_size: int,
                                  d_c: int, rope_w: int, rms_offset: int, kv: str, rms_mode: str,
                                  k_scale: float = 1.0, sm_scale: float, logit_cap: float = 0.0,
                                  rms_heads: int | None = None, groups: int = 1, num_splits: int = 1,
                                  align: int = 16, block_n: int = 16, partials: bool = False):
    """The decode with the roundings the reference Triton kernel applies, so that its own error
    against the float32 oracle can be measured (ops/mla_decode_attention.py:297-586, :1064-1137):

    * fp8 keys are dequantized to bf16, `(k.float() * k_scale).to(bf16)` (:451-452, :463); the
      latent is both key and value (`v = tl.trans(k)`, :547-551), so values carry the same rounding;
    * scores `q.k` accumulate in fp32 from bf16 operands (:453-464), then `/ rms`, `* sm_scale`,
      optional cap, mask (:466-514);
    * per split (bounds of `split_bounds`, :383-396), an online softmax over tiles of `block_n`
      tokens from the split start with natural `exp` against the running max (:553-560), P rounded
      to bf16 before `P.V` while the sum uses the unrounded P (:557-559);
    * the stage-2 LSE merge in fp32 (:1097-1132).

    The running-max rescale `acc * exp(m_old - m_new)` is applied here in closed form: tile t's
    `P.V` is weighted by `exp(m_t - m_last)`, which is the product of the rescale factors after it.
    Returns (o float32 before the output cast, lse), like `mla_decode`; with `partials`, the split
    partials in the workspace format of `mla_decode_partials` instead.
    """
    R, H, dcg = q_lat.shape
    assert dcg * groups == d_c
    n_rms = rms_heads if rms_heads is not None else H
    hpg = H // groups
    o = torch.zeros(R, H, dcg)
    lse = torch.full((R, H), -math.inf)
    att = torch.full((R, H, num_splits, dcg + 1), math.nan) if partials else None
    for i in range(R):
        L = int(seq_lens[i])
        if L <= 0:
            continue
        rows = gather_rows(cache_u8, block_table, i, L, page_size)
        c, r = dequant_rows(rows, d_c=d_c, rope_w=rope_w, kv=kv, k_scale=k_scale)
        if kv == KV_FP8:
            c, r = _bf16_t(c), _bf16_t(r)
        rms = decode_rms(rows, rms_offset=rms_offset, n_heads=n_rms, kv=kv, mode=rms_mode, k_scale=k_scale)
        live = [(si, a, e) for si, (a, e) in enumerate(split_bounds(L, num_splits, align)) if e > a]
        for g in range(groups):
            hs = slice(g * hpg, (g + 1) * hpg)
            cg = c[:, g * dcg:(g + 1) * dcg]
            s = _scores(_bf16_t(q_lat[i, hs].float()), None if q_pe is None else _bf16_t(q_pe[i, hs].float()), cg, r,
                        rms[:, hs], sm_scale, logit_cap)                        # [hpg, L]
            parts_o, parts_l = [], []
            for si, a, e in live:
                ss = s[:, a:e]
                n = e - a
                nt = -(-n // block_n)
                pad = torch.full((ss.shape[0], nt * block_n), -math.inf)
                pad[:, :n] = ss
                tmax = pad.view(ss.shape[0], nt, block_n).max(-1).values        # [hpg, nt]
                mrun = torch.cummax(tmax, dim=-1).values
                mtok = mrun.repeat_interleave(block_n, dim=-1)[:, :n]
                p = torch.exp(ss - mtok)
                w = torch.exp(mtok - mrun[:, -1:])
                acc = (w * _bf16_t(p)) @ cg[a:e]
                esum = (w * p).sum(-1, keepdim=True)
                parts_o.append(acc / esum)
                parts_l.append(mrun[:, -1] + torch.log(esum.squeeze(-1)))
                if partials:
                    att[i, hs, si, :dcg] = parts_o[-1]
                    att[i, hs, si, dcg] = parts_l[-1]
            ls = torch.stack(parts_l, -1)                                       # [hpg, S']
            m = ls.max(-1, keepdim=True).values
            wt = torch.exp(ls - m)
            o[i, hs] = (wt[..., None] * torch.stack(parts_o, 1)).sum(1) / wt.sum(-1, keepdim=True)
            lse[i, hs] = (m + torch.log(wt.sum(-1, keepdim=True))).squeeze(-1)
    return att if partials else (o, lse)


def split_bounds(L: int, num_splits: int, align: int) -> list[tuple[int, int]]:
    """[start, end) of each split: per = ceil(ceil(L/S)/align)*align when align > 0, else
    ceil(L/S); empty splits have end <= start (ops/mla_decode_attention.py:389-396, :1101-1108)."""
    per = -(-L // num_splits)
    if align > 0:
        per = -(-per // align) * align
    out = []
    for s in range(num_splits):
        a = per * s
        out.append((a, min(a + per, L)))
    return out


def mla_decode_partials(q_lat, q_pe, cache_u8, block_table, seq_lens, *, num_splits: int, align: int,
                        page_size, d_c, rope_w, rms_offset, kv, rms_mode, k_scale=1.0, sm_scale,
                        logit_cap=0.0):
    """Split-KV partials in the reference workspace format [R, H, S, d_c + 1]: normalized partial
    output in [..., :d_c] and the split's natural-log LSE in [..., d_c]
    (ops/mla_decode_attention.py:562-586). Empty splits stay NaN (never written)."""
    R, H, _ = q_lat.shape
    att = torch.full((R, H, num_splits, d_c + 1), math.nan)
    for i in range(R):
        L = int(seq_lens[i])
        rows_all = gather_rows(cache_u8, block_table, i, L, page_size)
        c_all, r_all = dequant_rows(rows_all, d_c=d_c, rope_w=rope_w, kv=kv, k_scale=k_scale)
        rms_all = decode_rms(rows_all, rms_offset=rms_offset, n_heads=H, kv=kv, mode=rms_mode, k_scale=k_scale)
        for s_idx, (a, e) in enumerate(split_bounds(L, num_splits, align)):
            if e <= a:
                continue
            s = _scores(q_lat[i].float(), None if q_pe is None else q_pe[i].float(), c_all[a:e],
                        r_all[a:e], rms_all[a:e], sm_scale, logit_cap)
            m = s.max(-1, keepdim=True).values
            p = torch.exp(s - m)
            l = p.sum(-1, keepdim=True)
            att[i, :, s_idx, :d_c] = (p @ c_all[a:e]) / l
            att[i, :, s_idx, d_c] = (m + torch.log(l)).squeeze(-1)
    return att


def combine_partials(att: torch.Tensor, seq_lens: torch.Tensor, *, num_splits: int, align: int):
    """LSE-weighted merge of split partials, skipping empty splits with the same bounds as the
    partial pass (ops/mla_decode_attention.py:1097-1137). Returns o [R, H, Dv], lse [R, H]."""
    R, H, S, D1 = att.shape
    dv = D1 - 1
    o = torch.zeros(R, H, dv)
    lse = torch.full((R, H), -math.inf)
    for i in range(R):
        L = int(seq_lens[i])
        live = [s for s, (a, e) in enumerate(split_bounds(L, num_splits, align)) if e > a]
        if not live:
            continue
        ls = att[i, :, live, dv]                        # [H, n]
        m = ls.max(-1, keepdim=True).values
        w = torch.exp(ls - m)
        o[i] = (w[..., None] * att[i, :, live, :dv]).sum(1) / w.sum(-1, keepdim=True)
        lse[i] = (m + torch.log(w.sum(-1, keepdim=True))).squeeze(-1)
    return o, lse


# ------------------------------------------------------------------------------------------------
# spec-verify flattening
# ------------------------------------------------------------------------------------------------
def flatten_verify(block_table: np.ndarray, seq_lens: np.ndarray, q: int):
    """One decode row per query token: row j of a request with q tokens and total length L
    attends to the first max(L - (q-1-j), 0) tokens and shares the request's block-table row
    (mla_impl.py:628-662)."""
    n, width = block_table.shape
    bt = np.repeat(block_table[:, None, :], q, axis=1).reshape(n * q, width)
    offs = np.arange(1 - q, 1, dtype=np.int64)
    sl = np.maximum(seq_lens.astype(np.int64)[:, None] + offs[None, :], 0).reshape(-1)
    return bt.astype(block_table.dtype), sl.astype(seq_lens.dtype)


# ------------------------------------------------------------------------------------------------
# FP8 cache-row writer and prefill gather
# ------------------------------------------------------------------------------------------------
def fp8_row_bytes(kv_c: np.ndarray, k_pe: np.ndarray, *, packed_rope: int, n_heads: int,
                  k_scale: float, rms_mode: str) -> np.ndarray:
    """FP8 cache row bytes [n, d_c + packed_rope + n_heads*(1|2)] (mla_impl.py:328-339).

    Latent and rope: `(x.float() * (1/k_scale)).clamp(-448, 448)` then e4m3fn, all float32.
    rms (k_pe[:, packed_rope : packed_rope + n_heads]): a log8 code, or its bf16 bytes.
    """
    inv = np.float32(1.0) / np.float32(k_scale)
    lat = e4m3_encode(np.clip(np.asarray(kv_c, np.float32) * inv, -E4M3_MAX, E4M3_MAX))
    rope = e4m3_encode(np.clip(np.asarray(k_pe[:, :packed_rope], np.float32) * inv, -E4M3_MAX, E4M3_MAX))
    rms = np.asarray(k_pe[:, packed_rope:packed_rope + n_heads], np.float32)
    if rms_mode == RMS_LOG8:
        rb = log8_encode(rms)
    elif rms_mode == RMS_BF16_BYTES:
        rb = f32_to_bf16_bits(rms).view(np.uint8).reshape(rms.shape[0], -1)
    else:
        raise ValueError(rms_mode)
    return np.concatenate([lat, rope, rb], axis=1)


def fp8_cache_write(cache_flat: np.ndarray, slots: np.ndarray, rows: np.ndarray) -> None:
    """Write rows into a flat [num_slots, row] uint8 cache view; slot -1 (padding) is redirected
    to slot 0, the never-read null block (mla_impl.py:340-342)."""
    s = np.maximum(np.asarray(slots, np.int64), 0)
    cache_flat[s, :rows.shape[1]] = rows


def gather_context(cache_u8: np.ndarray, block_table: np.ndarray, cu_seq_lens: np.ndarray,
                   token_to_seq: np.ndarray, num_tokens: int, seq_starts: np.ndarray | None, *,
                   kv: str, scale: float = 1.0, rms_offset: int = 0, n_heads: int = 0,
                   rms_mode: str = RMS_NONE) -> np.ndarray:
    """Prefill context gather into bf16 rows (returned as uint16 bit patterns)
    (ops/mla_gather.py:28-76).

    Row j: s = token_to_seq[j]; tok = j - cu_seq_lens[s] (+ seq_starts[s]); the page is
    block_table[s, tok // P]. bf16 caches copy the row; FP8 rows decode latent+rope as
    bf16(e4m3 * scale) and the rms tail per mode into one bf16 element per head at rms_offset.
    """
    P = cache_u8.shape[1]
    j = np.arange(num_tokens)
    s = token_to_seq[:num_tokens].astype(np.int64)
    tok = j - cu_seq_lens.astype(np.int64)[s]
    if seq_starts is not None:
        tok = tok + seq_starts.astype(np.int64)[s]
    blk = block_table[s, tok // P].astype(np.int64)
    rows = cache_u8[blk, tok % P].reshape(num_tokens, -1)
    if kv == KV_BF16:
        return rows.view(np.uint16)
    width = rows.shape[1]
    out = np.zeros((num_tokens, width), dtype=np.uint16)
    sc = np.float32(scale)
    if rms_mode == RMS_E4M3:
        out[:, :rms_offset + n_heads] = f32_to_bf16_bits(e4m3_decode(rows[:, :rms_offset + n_heads]) * sc)
        return out
    out[:, :rms_offset] = f32_to_bf16_bits(e4m3_decode(rows[:, :rms_offset]) * sc)
    code = rows[:, rms_offset:rms_offset + n_heads]
    if rms_mode == RMS_LOG8:
        out[:, rms_offset:rms_offset + n_heads] = f32_to_bf16_bits(log8_decode(code))
    else:
        raw = rows[:, rms_offset:rms_offset + 2 * n_heads].copy().view(np.uint16)
        out[:, rms_offset:rms_offset + n_heads] = raw
    return out


# ------------------------------------------------------------------------------------------------
# decode q / k_pe prep (the attention module's per-token work before the attention call)
# ------------------------------------------------------------------------------------------------
def partial_rope_table(keep, model_rope_dim: int, theta: float, max_pos: int) -> np.ndarray:
    """cos/sin table of the kept rope subspaces (partial_rope.py:66-76): subspace keep[i] rotates
    at its ORIGINAL frequency theta^(-2*keep[i]/model_rope_dim); the angles t*inv are float32
    products; row t = [cos(angles) | sin(angles)] as float32 [max_pos, 2*len(keep)]. cos and sin
    are evaluated on the float32 angle in float64 and rounded once."""
    k = np.asarray(keep, dtype=np.float32)
    expo = (np.float32(2.0) * k / np.float32(model_rope_dim)).astype(np.float32)
    inv = (1.0 / np.power(np.float64(np.float32(theta)), expo.astype(np.float64))).astype(np.float32)
    ang = (np.arange(max_pos, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    a64 = ang.astype(np.float64)
    return np.concatenate([np.cos(a64), np.sin(a64)], axis=1).astype(np.float32)


def _bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bf16 value, as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, np.float32)))


def neox_rotate_bf16(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Neox rotation in bf16 arithmetic (qwen3_5_mla.py:346-353, the rotation vLLM's rotary applies
    with is_neox_style): x [..., rd] holds bf16 values, cos/sin [..., rd/2] are rounded to bf16
    first (the table is cast to the query dtype, :346); each product and each sum is rounded to
    bf16: [x1*cos - x2*sin | x2*cos + x1*sin]. Returns float32 values that are bf16."""
    half = x.shape[-1] // 2
    x = np.asarray(x, np.float32)
    c, s = _bf16(cos), _bf16(sin)
    x1, x2 = x[..., :half], x[..., half:]
    o1 = _bf16(_bf16(x1 * c) - _bf16(x2 * s))
    o2 = _bf16(_bf16(x2 * c) + _bf16(x1 * s))
    return np.concatenate([o1, o2], axis=-1)


def rope_rows(table: np.ndarray, positions: np.ndarray, rope_sec=None) -> tuple[np.ndarray, np.ndarray]:
    """(cos, sin) [n, rd/2] for each token. positions [n], or [3, n] with rope_sec[i] in 0..2
    naming the position row of frequency i (M-RoPE, qwen3_5_mla.py:346-348)."""
    half = table.shape[1] // 2
    pos = np.asarray(positions, np.int64)
    if pos.ndim == 1:
        rows = table[pos]
        return rows[:, :half], rows[:, half:]
    sec = np.asarray(rope_sec, np.int64)
    f = np.arange(half)
    p = pos[sec[f]]                                     # [half, n]
    return table[p.T, f[None, :]], table[p.T, half + f[None, :]]


def mla_decode_prep(q: np.ndarray, latent: np.ndarray, k_rope: np.ndarray, k_up: np.ndarray,
                    k_norm_weight: np.ndarray, table: np.ndarray, positions: np.ndarray, *,
                    head_offset: int, rope_group: int, rope_first: int, rope_span: int,
                    declared_rope: int, eps: float, rope_sec=None):
    """The decode prep of qwen3_5_mla.py:232-301 on bf16 inputs (float32 arrays holding bf16
    values): q [n, H, hd] (normed, rope dims first), latent [n, d_c], k_rope [n, kv_heads, rd] (raw),
    k_up [H*nope, d_c] (raw), k_norm_weight [hd], table [max_pos, rd] cos|sin.

      g(h)   = (head_offset + h) // rope_group                                      (:239-240)
      k_nope = bf16(latent @ k_up^T)   (the bf16 GEMM output; accumulated here in float64)  (:262)
      rms    = sqrt((sum bf16(k_nope)^2 + sum k_rope[:, g]^2) / hd + eps)   float32  (:263-265)
      q_rot  = rot(q[..., :rd]);  k_rot = rot(bf16(k_rope * (1 + w[:rd])))          (:274-283)
      q_out  = [q[..., rd:] | q_pe],  q_pe zero but slot (g - rope_first)*rd          (:289-292, :303)
      k_pe   = [k_rot[:, rope_first:rope_first+rope_span] | bf16(rms) | 0]          (:293-301)

    Returns (q_out [n, H, nope + declared_rope], k_pe [n, declared_rope], rms float32 [n, H]);
    the first two as bf16-valued float32.
    """
    n, H, hd = q.shape
    rd = table.shape[1]
    nope = hd - rd
    kv_heads = k_rope.shape[1]
    g = (head_offset + np.arange(H)) // rope_group
    k_nope = _bf16((latent.astype(np.float64) @ k_up.astype(np.float64).T).astype(np.float32))
    k_nope = k_nope.reshape(n, H, nope).astype(np.float64)
    kr = k_rope.astype(np.float64)
    sumsq = (k_nope ** 2).sum(-1) + (kr ** 2).sum(-1)[:, g]
    rms = np.sqrt((sumsq / hd).astype(np.float32) + np.float32(eps)).astype(np.float32)
    cos, sin = rope_rows(table, positions, rope_sec)
    q_rot = neox_rotate_bf16(q[..., :rd], cos[:, None, :], sin[:, None, :])
    gain = (np.float32(1.0) + np.asarray(k_norm_weight, np.float32))[:rd]
    k_in = _bf16(k_rope.astype(np.float32) * gain)
    k_rot = neox_rotate_bf16(k_in, cos[:, None, :], sin[:, None, :])
    q_out = np.zeros((n, H, nope + declared_rope), np.float32)
    q_out[..., :nope] = q[..., rd:]
    for h in range(H):
        s0 = nope + (g[h] - rope_first) * rd
        q_out[:, h, s0:s0 + rd] = q_rot[:, h]
    packed = rope_span * rd
    assert rope_first + rope_span <= kv_heads and declared_rope >= packed + H
    k_pe = np.zeros((n, declared_rope), np.float32)
    k_pe[:, :packed] = k_rot[:, rope_first:rope_first + rope_span].reshape(n, packed)
    k_pe[:, packed:packed + H] = _bf16(rms)
    return q_out, k_pe, rms
