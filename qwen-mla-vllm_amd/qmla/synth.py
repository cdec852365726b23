"""Synthetic decode workloads in the cache-row layout (for benchmarks, tests and the smoke check).

A case holds absorbed queries, a paged cache [num_pages, page_size, 1, row] filled with random
latent/rope rows and their rms tail, a random-permutation block table and per-request lengths.
FP8 rows are written with the reference writer's arithmetic (qwen_mla/mla_impl.py:309-342):
`(x * (1/k_scale)).clamp(-448, 448)` to e4m3fn, the rms as a log8 code, two bf16 bytes or one e4m3
byte. The per-layer scale is the absmax of the unscaled N(0,1) draw over 448, so an `amp` > 1
drives values into e4m3 saturation.
"""
from __future__ import annotations

import dataclasses
import math

import torch

F8 = getattr(torch, "float8_e4m3fn", None)


@dataclasses.dataclass
class Case:
    q_nope: torch.Tensor        # [rows, H, d_c / groups] bf16
    q_pe: torch.Tensor          # [rows, H, rope_w] bf16
    cache: torch.Tensor         # [pages, P, 1, row] bf16 or uint8
    block_table: torch.Tensor   # [rows, max_pages] int32
    seq_lens: torch.Tensor      # [rows] int32
    page_size: int
    d_c: int
    rope_w: int
    heads: int
    kv: str                     # "bf16" | "fp8"
    rms_mode: str               # "bf16" | "log8" | "bf16_bytes" | "e4m3" | "none"
    k_scale: torch.Tensor | None
    sm_scale: float
    qrows: int = 1
    groups: int = 1

    @property
    def rms_offset(self) -> int:
        return -1 if self.rms_mode == "none" else self.d_c + self.rope_w

    @property
    def row(self) -> int:
        return self.cache.shape[-1]

    def tokens(self) -> int:
        return int(self.seq_lens.to(torch.int64).sum())


def row_width(d_c: int, rope_w: int, heads: int, kv: str, rms_mode: str, pad: bool = True) -> int:
    """Cache row elements: [latent | rope | rms], padded to 16 elements as the plugin pads its rows
    (mla_impl.py:261-271), or unpadded as the reference's numerics test builds them."""
    per = 2 if (kv == "fp8" and rms_mode == "bf16_bytes") else 1
    raw = d_c + rope_w + (0 if rms_mode == "none" else heads * per)
    return ((raw + 15) // 16) * 16 if pad else raw


def _log8(rms: torch.Tensor) -> torch.Tensor:
    """rms -> uint8 code (mla_impl.py:333-336); log2 in float64 then float32 arithmetic."""
    lg = rms.float().clamp_min(1e-30).double().log2().float()
    code = (lg - (-3.0)) * (255.0 / 6.0)
    return code.round().clamp(0, 255).to(torch.uint8)


def _e4m3_bytes(x: torch.Tensor, inv: torch.Tensor) -> torch.Tensor:
    return (x.float() * inv).clamp(-448.0, 448.0).to(F8).view(torch.uint8)


def make_case(*, batch: int, heads: int, d_c: int, rope_w: int, page_size: int, lens, kv: str = "bf16",
              rms_mode: str | None = None, seed: int = 0, device="cpu", qrows: int = 1, groups: int = 1,
              amp: float = 1.0, rms: str = "row", q_amp: float = 1.0, shuffle: bool = True,
              extra_pages: int = 3, chunk_tokens: int = 1 << 20, pad: bool = True) -> Case:
    """Build a case. `lens` are per-request lengths (the last verify row's length when qrows > 1).

    rms = "row": every head's divisor is the RMS of the row's (amplified) latent; "spread": per-head
    exp(N(0, 0.6)) like the reference's FP8 test (tests/test_fp8_kv.py:23-31).
    """
    if rms_mode is None:
        rms_mode = "bf16" if kv == "bf16" else "log8"
    g = torch.Generator(device="cpu").manual_seed(seed)
    lens = [int(x) for x in lens]
    n_req = len(lens)
    assert n_req == batch
    pages_per = [max(1, -(-L // page_size)) for L in lens]
    max_pages = max(pages_per)
    total_pages = sum(pages_per) + extra_pages
    perm = torch.randperm(total_pages, generator=g) if shuffle else torch.arange(total_pages)
    bt_req = torch.zeros(n_req, max_pages, dtype=torch.int32)
    k = 0
    for b in range(n_req):
        bt_req[b, :pages_per[b]] = perm[k:k + pages_per[b]].to(torch.int32)
        k += pages_per[b]
    row = row_width(d_c, rope_w, heads, kv, rms_mode, pad)
    dev = torch.device(device)
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    # per-layer fp8 scale from an unscaled calibration draw (absmax / 448)
    k_scale = None
    inv = None
    if kv == "fp8":
        calib = torch.randn(1 << 16, generator=g)
        absmax = max(float(calib.abs().max()), 1e-6)
        # the absmax of N(0,1) grows with the sample count: use the expected maximum of the
        # cache's own draw so the unamplified data fits and `amp` sets the saturation
        n_el = total_pages * page_size * (d_c + rope_w)
        absmax = max(absmax, math.sqrt(2.0 * math.log(max(n_el, 2))))
        k_scale = torch.tensor(absmax / 448.0, dtype=torch.float32, device=dev)
        inv = (1.0 / k_scale.float()).reshape(())
    if kv == "bf16":
        cache = torch.zeros(total_pages, page_size, 1, row, dtype=torch.bfloat16, device=dev)
    else:
        cache = torch.zeros(total_pages, page_size, 1, row, dtype=torch.uint8, device=dev)
    flat = cache.view(total_pages * page_size, row)
    nslots = total_pages * page_size
    for a in range(0, nslots, chunk_tokens):
        e = min(a + chunk_tokens, nslots)
        n = e - a
        c = torch.randn(n, d_c, generator=gd, device=dev) * amp
        r = torch.randn(n, rope_w, generator=gd, device=dev) * amp
        if rms == "row":
            rr = c.pow(2).mean(-1, keepdim=True).sqrt().expand(n, heads)
        else:
            rr = torch.exp(torch.randn(n, heads, generator=gd, device=dev) * 0.6)
        if kv == "bf16":
            flat[a:e, :d_c] = c.to(torch.bfloat16)
            flat[a:e, d_c:d_c + rope_w] = r.to(torch.bfloat16)
            if rms_mode != "none":
                flat[a:e, d_c + rope_w:d_c + rope_w + heads] = rr.to(torch.bfloat16)
        else:
            flat[a:e, :d_c] = _e4m3_bytes(c, inv)
            flat[a:e, d_c:d_c + rope_w] = _e4m3_bytes(r, inv)
            o = d_c + rope_w
            if rms_mode == "log8":
                flat[a:e, o:o + heads] = _log8(rr)
            elif rms_mode == "bf16_bytes":
                flat[a:e, o:o + 2 * heads] = rr.to(torch.bfloat16).contiguous().view(torch.uint8).view(n, 2 * heads)
            elif rms_mode == "e4m3":
                flat[a:e, o:o + heads] = _e4m3_bytes(rr, inv)
    rows = n_req * qrows
    # spec-verify flattening: row j of a request of length L sees L - (qrows-1-j) tokens
    bt = bt_req.repeat_interleave(qrows, dim=0)
    sl = torch.tensor(lens, dtype=torch.int64).repeat_interleave(qrows)
    sl = (sl + torch.arange(1 - qrows, 1).repeat(n_req)).clamp_min(0).to(torch.int32)
    dcg = d_c // groups
    q_nope = (torch.randn(rows, heads, dcg, generator=gd, device=dev) * q_amp).to(torch.bfloat16)
    q_pe = (torch.randn(rows, heads, rope_w, generator=gd, device=dev) * q_amp).to(torch.bfloat16)
    sm_scale = 1.0 / math.sqrt(d_c + rope_w)
    return Case(q_nope=q_nope, q_pe=q_pe, cache=cache, block_table=bt.to(dev), seq_lens=sl.to(dev),
                page_size=page_size, d_c=d_c, rope_w=rope_w, heads=heads, kv=kv, rms_mode=rms_mode,
                k_scale=k_scale, sm_scale=sm_scale, qrows=qrows, groups=groups)


def lognormal_lens(batch: int, median: int, sigma: float, lo: int, hi: int, seed: int) -> list[int]:
    g = torch.Generator().manual_seed(seed)
    x = torch.exp(torch.randn(batch, generator=g, dtype=torch.float64) * sigma) * median
    return [int(v) for v in x.round().clamp(lo, hi).tolist()]


def uniform_lens(batch: int, lo: int, hi: int, seed: int) -> list[int]:
    g = torch.Generator().manual_seed(seed)
    return [int(v) for v in torch.randint(lo, hi + 1, (batch,), generator=g).tolist()]


def algorithmic_bytes(case: Case) -> int:
    """Bytes the decode must move at minimum (row padding and split-K scratch excluded):
    sum_b L_b (d_c*e + W*e + H*r) + q + o + lse + block table + seq_lens."""
    e = 1 if case.kv == "fp8" else 2
    r = 0 if case.rms_mode == "none" else (2 if case.rms_mode in ("bf16", "bf16_bytes") else 1)
    n_req = case.seq_lens.shape[0] // case.qrows
    req_len = case.seq_lens.view(n_req, case.qrows)[:, -1].to(torch.int64)
    toks = int(req_len.sum())
    per_tok = case.d_c * e + case.rope_w * e + case.heads * r
    rows, H = case.q_nope.shape[0], case.heads
    dv = case.d_c // case.groups
    q = rows * H * (dv + case.rope_w) * 2
    o = rows * H * dv * 2
    lse = rows * H * 4
    pages = int(((req_len + case.page_size - 1) // case.page_size).sum())
    return toks * per_tok + q + o + lse + pages * 4 + rows * 4


def compact_requests(case: Case, reqs):
    """The rows of the requests `reqs` (all qrows rows of each) with only their pages, as CPU tensors:
    (cache bytes [pages, P, row_bytes], block table remapped onto those pages, seq_lens, q_nope,
    q_pe, row indices). The pages are gathered on the case's device first, so a multi-GB cache is
    never copied whole."""
    P, qr = case.page_size, case.qrows
    bt = case.block_table.cpu()
    sl = case.seq_lens.cpu()
    rows = [b * qr + j for b in reqs for j in range(qr)]
    page_ids, new_bt = [], torch.zeros(len(rows), bt.shape[1], dtype=torch.int32)
    first = 0
    for i, r in enumerate(rows):
        if i % qr == 0:
            last = (int(reqs[i // qr]) + 1) * qr - 1          # the request's last row owns its pages
            n = max(1, -(-int(sl[last]) // P))
            first = len(page_ids)
            page_ids.extend(int(x) for x in bt[last, :n])
        n_r = max(1, -(-int(sl[r]) // P))
        new_bt[i, :n_r] = torch.arange(first, first + n_r, dtype=torch.int32)
    idx = torch.tensor(page_ids, dtype=torch.long, device=case.cache.device)
    cache = case.cache.index_select(0, idx).cpu().contiguous()
    cache = cache.view(torch.uint8).reshape(cache.shape[0], P, -1)
    return cache, new_bt, sl[rows], case.q_nope.cpu().float()[rows], case.q_pe.cpu().float()[rows], rows
