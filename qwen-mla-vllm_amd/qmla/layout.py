"""Cache-row layout of the absorbed-MLA latent cache: [latent | packed rope | rms tail | pad].

Integer helpers that size and place the row, restated from the reference plugin so a cache
allocated by the plugin is read identically here:

* rms tail formats and the log8 code range (qwen_mla/mla_impl.py:125-145)
* live tail width, rope span, GLA latent split, per-rank latent widths
  (qwen_mla/mla_impl.py:148-200)
* padded row width chosen between the pow2 and base-multiple schemes
  (qwen_mla/mla_impl.py:203-275) and its inverse (qwen_mla/mla_impl.py:278-285)
* rope window of a rank and the 16-byte alignment rule of paged rows
  (qwen_mla/fi_decode.py:103-127)
* partial-RoPE widths (qwen_mla/partial_rope.py:20-49)

`hf` is any object with the Hugging Face config attributes the reference reads:
num_attention_heads, num_key_value_heads, head_dim, optional partial_rotary_factor /
rope_parameters, mla_ranks {layer: rank}, optional mla_rope_keep and mla_latent_groups.
"""
from __future__ import annotations

import dataclasses

RMS_LOG2_LO, RMS_LOG2_HI = -3.0, 3.0
FP8_RMS_MODES = ("log8", "bf16", "e4m3")


def mla_fp8_rms_mode() -> str:
    """The FP8 rows' rms tail format from QWEN_MLA_FP8_RMS (qwen_mla/mla_impl.py:136-141): log8
    (default), bf16 (two raw bytes per head) or e4m3."""
    import os
    m = os.environ.get("QWEN_MLA_FP8_RMS", "log8")
    if m not in FP8_RMS_MODES:
        raise ValueError(f"QWEN_MLA_FP8_RMS={m!r}: expected one of {FP8_RMS_MODES}")
    return m


def rope_keep_from_config(hf):
    """Kept rope subspace indices, or None for full rope (qwen_mla/partial_rope.py:20-27)."""
    keep = getattr(hf, "mla_rope_keep", None)
    if keep is None:
        return None
    keep = [int(x) for x in keep]
    if not keep:
        raise ValueError("mla_rope_keep is empty")
    return keep


def model_rope_dim(hf) -> int:
    """The base model's rotary width (qwen_mla/partial_rope.py:30-34)."""
    rp = getattr(hf, "rope_parameters", None) or {}
    prf = rp.get("partial_rotary_factor", getattr(hf, "partial_rotary_factor", 0.25))
    return int(hf.head_dim * prf)


def effective_rope_dim(hf) -> int:
    """Per-group rope width actually cached: 2*len(keep) under partial rope
    (qwen_mla/partial_rope.py:37-40)."""
    keep = rope_keep_from_config(hf)
    return model_rope_dim(hf) if keep is None else 2 * len(keep)


def mla_rope_span(hf, tp_size: int = 1) -> int:
    """Rope groups a rank's query heads span, the same on every rank (qwen_mla/mla_impl.py:168-179)."""
    group = hf.num_attention_heads // hf.num_key_value_heads
    n_local = hf.num_attention_heads // tp_size
    return max((r * n_local + n_local - 1) // group - (r * n_local) // group + 1 for r in range(tp_size))


def mla_base_tail(hf, tp_size: int = 1, fp8: bool = False, fp8_rms: str = "log8") -> int:
    """Live tail beyond the latent: packed rope plus one rms per local head, two bytes per head for
    the FP8 bf16-rms row (qwen_mla/mla_impl.py:148-165)."""
    rope = effective_rope_dim(hf)
    per_head = 2 if (fp8 and fp8_rms == "bf16") else 1
    return mla_rope_span(hf, tp_size) * rope + (hf.num_attention_heads // tp_size) * per_head


def mla_gla_split(hf, tp_size: int, gla_shard: bool = True) -> int:
    """Latent groups a rank's latent is divided by: G when GLA groups align with TP
    (qwen_mla/mla_impl.py:182-194)."""
    g = int(getattr(hf, "mla_latent_groups", 1) or 1)
    if g > 1 and tp_size % g == 0 and gla_shard:
        return g
    return 1


def mla_local_ranks(hf, tp_size: int = 1) -> dict[int, int]:
    """Per-layer latent width cached on one rank (qwen_mla/mla_impl.py:197-200)."""
    g = mla_gla_split(hf, tp_size)
    return {int(k): int(v) // g for k, v in hf.mla_ranks.items()}


def _next_pow2(x: int) -> int:
    """Smallest power of two >= x (1 for x <= 1)."""
    x = int(x)
    return 1 if x <= 1 else 1 << (x - 1).bit_length()


def _row_schemes(raw: dict[int, int]):
    """The two row-width schemes whose pages vLLM can unify by block size, for raw widths
    {rank: rank + tail}: each width rounded up to a power of two, or to a power-of-two multiple of
    the smallest raw width rounded up to 16 elements (qwen_mla/mla_impl.py:230-266)."""
    unit = -(-min(raw.values()) // 16) * 16
    yield {r: _next_pow2(w) for r, w in raw.items()}
    yield {r: unit * _next_pow2(-(-w // unit)) for r, w in raw.items()}


def mla_padded_head_size(hf, kv_lora_rank: int, tp_size: int = 1, fp8: bool = False,
                         fp8_rms: str = "log8") -> int:
    """Cache row width of a layer of rank `kv_lora_rank` (qwen_mla/mla_impl.py:203-275).

    Of the two schemes of _row_schemes, the ones where every layer's row divides the largest and is
    a multiple of 16 elements qualify; the one with the smaller total row width over the model's
    layers wins (the pow2 scheme on a tie). A rank that no layer has gets its raw width rounded up
    to a power of two."""
    tail = mla_base_tail(hf, tp_size, fp8, fp8_rms)
    layer_ranks = [int(v) for v in mla_local_ranks(hf, tp_size).values()]
    best_total, best = None, None
    for rows in _row_schemes({r: r + tail for r in set(layer_ranks)}):
        top = max(rows.values())
        if any(top % w or w % 16 for w in rows.values()):
            continue
        total = sum(rows[r] for r in layer_ranks)
        if best_total is None or total < best_total:
            best_total, best = total, rows
    if best is not None and kv_lora_rank in best:
        return best[kv_lora_rank]
    return _next_pow2(kv_lora_rank + tail)


def mla_rank_by_head_size(hf, tp_size: int = 1, fp8: bool = False, fp8_rms: str = "log8") -> dict[int, int]:
    """padded head_size -> kv_lora_rank, max on collision (qwen_mla/mla_impl.py:278-285)."""
    out: dict[int, int] = {}
    for v in mla_local_ranks(hf, tp_size).values():
        r = int(v)
        hs = mla_padded_head_size(hf, r, tp_size, fp8, fp8_rms)
        out[hs] = max(out.get(hs, 0), r)
    return out


def rope_window(head_offset: int, n_local: int, rope_group: int, rope_dim: int) -> tuple[int, int]:
    """(offset, width) of the rope slice a rank's heads span; the cache stores only that window, so
    the offset is 0 (qwen_mla/fi_decode.py:103-114)."""
    first = head_offset // rope_group
    last = (head_offset + n_local - 1) // rope_group
    return 0, (last - first + 1) * rope_dim


def row_dma_safe(head_size: int, page_size: int, rank: int, off: int, itemsize: int) -> bool:
    """Every paged row and page start is 16-byte aligned, which the 16-byte LDS-DMA loads need
    (the same rule as cp_async_safe, qwen_mla/fi_decode.py:117-127)."""
    a = 16 // itemsize
    return head_size % a == 0 and (page_size * head_size) % a == 0 and rank % a == 0 and off % a == 0


def splitk_cap(batch: int, heads: int, lse_dim: int, splits: int, budget_mb: float = 512.0) -> int:
    """Largest split count <= splits whose fp32 split-K scratch fits the budget
    (qwen_mla/mla_impl.py:89-103)."""
    budget = int(budget_mb * (1 << 20))
    while splits > 1 and batch * heads * splits * lse_dim * 4 > budget:
        splits //= 2
    return max(1, splits)


def splitk_reserve_bytes(batch: int, heads: int, lse_dim: int, splits: int, budget_mb: float = 512.0) -> int:
    """Bytes covering every splitk_cap-ed request with batch <= `batch` (qwen_mla/mla_impl.py:106-111)."""
    budget = int(budget_mb * (1 << 20))
    full = batch * heads * splits * lse_dim * 4
    return min(full, max(budget, batch * heads * lse_dim * 4))


@dataclasses.dataclass(frozen=True)
class RowLayout:
    """Where things sit in one cache row (all offsets in cache elements).

    d_c         latent width (kv_lora_rank); scores read [0, d_c + rope_w)
    rope_w      packed rope window width
    heads       query heads of the rank; rms_heads rms slots per token
    row         padded row width (the cache's last dimension)
    kv          "bf16" or "fp8"; fp8_rms "log8" | "bf16" | "e4m3" (FP8 rows only)
    groups      GLA latent groups computed in one call (1 = plain MLA)
    """

    d_c: int
    rope_w: int
    heads: int
    row: int
    kv: str = "bf16"
    fp8_rms: str = "log8"
    rms_heads: int | None = None
    groups: int = 1
    has_rms: bool = True

    @property
    def rms_offset(self) -> int:
        return self.d_c + self.rope_w if self.has_rms else -1

    @property
    def n_rms(self) -> int:
        return self.rms_heads if self.rms_heads is not None else self.heads

    @property
    def tail_bytes(self) -> int:
        eb = 1 if self.kv == "fp8" else 2
        per = 2 if (self.kv == "fp8" and self.fp8_rms == "bf16") else eb
        return self.rope_w * eb + (self.n_rms * per if self.has_rms else 0)


def rank_layout(d_c: int = 512, rope_w: int = 64, heads: int = 24, fp8: bool = False,
                    fp8_rms: str = "log8", groups: int = 1) -> RowLayout:
    """Row layout of a single-layer config: the padded width for one rank d_c, tail = rope + rms."""
    per = 2 if (fp8 and fp8_rms == "bf16") else 1
    raw = d_c + rope_w + heads * per
    row = ((raw + 15) // 16) * 16
    return RowLayout(d_c=d_c, rope_w=rope_w, heads=heads, row=row, kv="fp8" if fp8 else "bf16",
                     fp8_rms=fp8_rms, groups=groups)
