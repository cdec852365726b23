"""The decode side of the plugin's vLLM attention backend, on libqmla.

Mirrors the registered surface of the reference (qwen_mla/mla_impl.py:431-465, :628-662,
:678-689; qwen_mla/fi_decode.py:338-384) without importing vLLM:

* `forward_mqa(impl, q, kv_c_and_k_pe_cache, attn_metadata, layer) -> (o, lse | None)` reads
  exactly what the reference's decode reads: from `attn_metadata` `.causal`, `.num_decode_tokens`,
  `.decode.seq_lens`, `.decode.block_table` and `.decode._mla_q`; from `impl` `rms_offset`,
  `kv_lora_rank`, `scale`, `mla_head_offset`, `mla_rope_group`, `mla_rope_dim`, `mla_local_heads`,
  `mla_packed_rope`, `mla_kv_fp8`, `need_to_return_lse_for_decode`; from `layer` the per-layer
  FP8 scale `_k_scale`. `q` is the absorbed query `[B, H, kv_lora_rank + declared_rope]` or the
  tuple `(q_nope, q_pe)`; only the latent and the `rms_offset - kv_lora_rank` rope columns are
  read, so neither form is copied.
* `DecodeMetadataBuilder.build_decode(...)` flattens a uniform multi-token (spec-verify) decode into
  one row per query token in persistent buffers (device ops only, static shapes: safe inside
  CUDA/HIP-graph capture), as `MLATritonMetadataBuilder._build_decode` does.
* `QwenMLAHipBackend` carries the backend triple `get_name / get_impl_cls / get_builder_cls`.

Where vLLM is installed, the maintainer subclasses vLLM's `TritonMLAImpl` / builder with these
bodies (INTEGRATION.md shows the change); the split-K partials of the reference's Triton path are
replaced by the balanced split mode, which has no split count to cap (the reference's
`splitk_cap` is `qmla.layout.splitk_cap` for callers of the fixed-split `decode_attention_fwd`).
"""
from __future__ import annotations

import os
from types import SimpleNamespace

import torch

from . import _lib
from .decode import Workspace, build_params, fold_rows, workspace_bytes
from .layout import mla_fp8_rms_mode


class QwenMLAHipImpl:
    """The decode attributes the model sets on the reference's impl before the first forward
    (qwen_mla/mla_impl.py:291-300, qwen3_5_mla.py:203-214), and its decode entry."""

    rms_offset: int = -1
    mla_local_heads: int = 0
    mla_rope_dim: int = 0
    mla_rope_group: int = 0
    mla_head_offset: int = 0
    mla_rope_first: int = 0
    mla_packed_rope: int = 0
    mla_kv_fp8: bool = False

    def __init__(self, kv_lora_rank: int, scale: float, need_to_return_lse_for_decode: bool = False):
        self.kv_lora_rank = kv_lora_rank
        self.scale = scale
        self.need_to_return_lse_for_decode = need_to_return_lse_for_decode
        self._workspace = Workspace()

    def reserve_decode_workspace(self, max_rows: int, device, qrows: int = 1) -> int:
        """Allocate the balanced-mode workspace for up to `max_rows` decode rows whose requests carry
        up to `qrows` query tokens each (1 + the speculative tokens of a verify step). Call it once
        before graph capture: every captured decode of at most that many rows and tokens per request
        then allocates nothing. Returns the size in bytes."""
        if max_rows % qrows:
            raise ValueError(f"max_rows {max_rows} is not a multiple of qrows {qrows}")
        n = max(reserve_bytes(self, max_rows, q) for q in range(1, qrows + 1) if max_rows % q == 0)
        self._workspace.reserve(n, device)
        return n

    def forward_mqa(self, q, kv_c_and_k_pe_cache, attn_metadata, layer):
        return forward_mqa(self, q, kv_c_and_k_pe_cache, attn_metadata, layer)


def _verify_rows(attn_metadata) -> int:
    """Query tokens per request folded back into one kernel request: `_mla_q` of a causal decode
    (qwen_mla/mla_impl.py:455-459; QWEN_MLA_GROUPED_VERIFY=0 keeps one kernel row per token)."""
    grouped = bool(attn_metadata.causal) and os.environ.get("QWEN_MLA_GROUPED_VERIFY", "1") != "0"
    return int(getattr(attn_metadata.decode, "_mla_q", 1) or 1) if grouped else 1


def _impl_rms_mode(impl) -> tuple[int, int]:
    """(kv dtype code, rms mode code) of the impl's cache rows, as decode_params sets them."""
    if impl.mla_kv_fp8:
        return _lib.KV_FP8, {"log8": _lib.RMS_LOG8, "bf16": _lib.RMS_BF16_BYTES,
                             "e4m3": _lib.RMS_E4M3}[mla_fp8_rms_mode()]
    return _lib.KV_BF16, _lib.RMS_BF16


def reserve_bytes(impl, rows: int, qtok: int) -> int:
    """Workspace bytes of a decode of `rows` flattened rows in requests of `qtok` query tokens, with
    the parameters decode_params builds (rms format, verify folding). The kernel family, and with
    it the balanced layout, can depend on the cache's row stride, which is not known before the
    cache exists: the size is the larger of the tightest row of this layout and a wide padded row."""
    heads = max(impl.mla_local_heads, 1)
    rank, rope_w = impl.kv_lora_rank, max(impl.rms_offset - impl.kv_lora_rank, 0)
    kv, mode = _impl_rms_mode(impl)
    eb = 1 if kv == _lib.KV_FP8 else 2
    rb = 2 if mode in (_lib.RMS_BF16, _lib.RMS_BF16_BYTES) else 1
    tight = -(-((rank + rope_w) * eb + heads * rb) // 16) * 16 // eb
    need = 0
    for row in (tight, 1 << 14):
        p = _lib.DecodeParams()
        p.rows, p.heads, p.rms_heads, p.qrows, p.groups = rows, heads, heads, 1, 1
        p.d_c, p.rope_w, p.rms_offset = rank, rope_w, impl.rms_offset
        p.kv_dtype, p.rms_mode = kv, mode
        p.token_stride, p.page_stride, p.page_size = row, row * 64, 64
        p.num_splits, p.num_workgroups = 0, 0
        p.qrows = fold_rows(p, qtok) if qtok > 1 else 1
        need = max(need, int(_lib.lib().qmla_workspace_bytes(p)))
    return need


def decode_params(impl, q, kv_c_and_k_pe_cache, attn_metadata, layer, out, lse):
    """The C parameter block of one decode call (pure host work): latent and rope views of q, the
    rope window [kv_lora_rank, rms_offset) of the cache rows, the rms tail format of the impl."""
    rank = impl.kv_lora_rank
    if impl.rms_offset < 0:
        raise ValueError("the decode needs impl.rms_offset (set by the model before the first forward)")
    rope_w = impl.rms_offset - rank
    if isinstance(q, tuple):
        q_nope, q_pe = q
    else:
        q_nope, q_pe = q[..., :rank], q[..., rank:]
    if q_nope.shape[-1] != rank or q_pe.shape[-1] < rope_w:
        raise ValueError(f"query widths {q_nope.shape[-1]} / {q_pe.shape[-1]} do not cover rank {rank} "
                         f"and the rope window {rope_w}")
    if impl.mla_local_heads and q_nope.shape[1] != impl.mla_local_heads:
        raise ValueError(f"{q_nope.shape[1]} query heads, the cache rows hold rms for {impl.mla_local_heads}")
    # vLLM's MLA cache is [num_blocks, block_size, head_size]; the paged-row view adds the kv-head
    # dim, as the reference does for its Triton call
    cache = kv_c_and_k_pe_cache.unsqueeze(2) if kv_c_and_k_pe_cache.dim() == 3 else kv_c_and_k_pe_cache
    kv, rms_mode = _impl_rms_mode(impl)
    k_scale = getattr(layer, "_k_scale", None) if kv == _lib.KV_FP8 else None
    if k_scale is not None and k_scale.dtype != torch.float32:
        raise TypeError("layer._k_scale must be a float32 device scalar")
    md = attn_metadata.decode
    page_size = cache.shape[1]
    qrows = _verify_rows(attn_metadata)
    if qrows > 1 and q_nope.shape[0] % qrows:
        raise ValueError(f"{q_nope.shape[0]} decode rows are not whole requests of {qrows} query tokens")
    p = build_params(q_nope=q_nope, q_pe=q_pe, kv_cache=cache, block_table=md.block_table, seq_lens=md.seq_lens,
                     out=out, lse=lse, d_c=rank, rope_w=rope_w, rms_offset=impl.rms_offset, rms_mode=rms_mode,
                     kv=kv, page_size=page_size, sm_scale=impl.scale, k_scale=k_scale,
                     qrows=1, groups=1, rms_heads=q_nope.shape[1], num_splits=0)
    if qrows > 1:
        p.qrows = fold_rows(p, qrows)
    return p


def forward_mqa(impl, q, kv_c_and_k_pe_cache, attn_metadata, layer):
    """Decode attention of the step's decode rows; returns (o [B, H, kv_lora_rank] in the query's
    dtype, lse [B, H] fp32 natural log if impl.need_to_return_lse_for_decode else None), as the
    reference's decode returns them (qwen_mla/fi_decode.py:381-384). Rows of a multi-token decode
    arrive flattened by build_decode; `_mla_q` folds each request's rows back so its cache is read
    once. Runs on the current stream; allocates only the outputs (and the workspace, if
    reserve_decode_workspace was not called for this many rows)."""
    q0 = q[0] if isinstance(q, tuple) else q
    B, H = q0.shape[0], q0.shape[1]
    if attn_metadata.decode.seq_lens.shape[0] != B:
        raise ValueError(f"{B} query rows against {attn_metadata.decode.seq_lens.shape[0]} decode rows")
    out = torch.empty(B, H, impl.kv_lora_rank, dtype=q0.dtype, device=q0.device)
    want_lse = bool(getattr(impl, "need_to_return_lse_for_decode", False))
    lse = torch.empty(B, H, dtype=torch.float32, device=q0.device) if want_lse else None
    if B == 0:
        return out, lse
    p = decode_params(impl, q, kv_c_and_k_pe_cache, attn_metadata, layer, out, lse)
    ws = getattr(impl, "_workspace", None)
    if ws is None:
        ws = impl._workspace = Workspace()
    need = workspace_bytes(p)
    if ws.buf is None or ws.buf.numel() < need:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("decode workspace too small inside graph capture: call "
                               "impl.reserve_decode_workspace(max_rows, device) before capturing")
        ws.reserve(need, q0.device)
    p.workspace = ws.buf.data_ptr()
    p.workspace_bytes = ws.buf.numel()
    _lib.check("qmla_decode", _lib.lib().qmla_decode(p, torch.cuda.current_stream().cuda_stream))
    return out, lse


class DecodeMetadataBuilder:
    """The decode half of the reference's metadata builder (qwen_mla/mla_impl.py:628-662)."""

    def __init__(self, max_rows: int = 0):
        self.max_rows = max_rows
        self._flat_bt = self._flat_sl = self._flat_offs = None

    def build_decode(self, block_table_tensor: torch.Tensor, seq_lens_device: torch.Tensor,
                     num_decode_tokens: int):
        """Decode metadata for n requests and num_decode_tokens = n*q query tokens. With q > 1, row j of
        a request of length L (its last query token included) gets the first max(L - (q-1-j), 0) tokens
        and the request's block-table row; the rows are written in place into persistent buffers (a
        replayed graph reads the addresses it captured). Returns a namespace with block_table,
        seq_lens and _mla_q."""
        n = block_table_tensor.shape[0]
        q = num_decode_tokens // n if n else 1
        md = SimpleNamespace(block_table=block_table_tensor, seq_lens=seq_lens_device, _mla_q=q)
        if q <= 1:
            md._mla_q = 1
            return md
        if q * n != num_decode_tokens:
            raise ValueError(f"{num_decode_tokens} decode tokens are not a uniform {q} per request over {n}")
        rows, width = n * q, block_table_tensor.shape[1]
        bt, sl = self._flat_bt, self._flat_sl
        if bt is None or bt.shape[0] < rows or bt.shape[1] != width or bt.device != block_table_tensor.device:
            if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
                raise RuntimeError("flattened decode metadata buffers too small inside graph capture")
            cap = max(rows, self.max_rows)
            bt = torch.zeros(cap, width, dtype=block_table_tensor.dtype, device=block_table_tensor.device)
            sl = torch.zeros(cap, dtype=seq_lens_device.dtype, device=seq_lens_device.device)
            self._flat_bt, self._flat_sl = bt, sl
        offs = self._flat_offs
        if offs is None or offs.numel() != q or offs.device != sl.device:
            offs = self._flat_offs = torch.arange(1 - q, 1, device=sl.device, dtype=sl.dtype)
        bt[:rows].view(n, q, width).copy_(block_table_tensor[:, None, :])
        v = sl[:rows].view(n, q)
        torch.add(seq_lens_device[:, None], offs[None, :], out=v)
        v.clamp_(min=0)
        md.block_table, md.seq_lens = bt[:rows], sl[:rows]
        return md


class QwenMLAHipBackend:
    """The backend triple the plugin registers per layer (qwen_mla/mla_impl.py:678-689), under the
    reference's name so a configuration that selects it needs no change."""

    @staticmethod
    def get_name() -> str:
        return "QWEN_MLA_TRITON"

    @staticmethod
    def get_impl_cls() -> type[QwenMLAHipImpl]:
        return QwenMLAHipImpl

    @staticmethod
    def get_builder_cls() -> type[DecodeMetadataBuilder]:
        return DecodeMetadataBuilder
