"""Absorbed-MLA decode over a paged latent cache, on the gfx950 HIP kernels of libqmla.so.

Two surfaces:

* `decode_attention_fwd(...)` keeps the reference kernel entry's signature and in-place contract
  (qwen_mla/ops/mla_decode_attention.py:1264-1359): q [B, H, d_c + rope(+tail)], k_buffer the
  paged cache, v_buffer = k_buffer[..., :d_c], o / lse / attn_logits written in place, a fixed
  split count with the reference's split bounds and partial layout.
* `forward(q_nope, q_rope, kv_cache, block_table, seq_lens, ...)` is the backend-level surface
  (the FlashInfer run() shape, qwen_mla/fi_decode.py:338-384): separate latent and rope queries,
  returns (o, lse). It defaults to the balanced split mode, where every workgroup gets the same
  number of 64-token tiles across requests, so ragged batches keep every compute unit busy.

Neither path has a CPU fallback: without libqmla.so, or on a device the library does not support,
they raise.
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import DecodeParams

_FP8_DTYPES = tuple(getattr(torch, n) for n in ("float8_e4m3fn",) if hasattr(torch, n))


def _dt_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.DT_BF16
    if t.dtype == torch.float32:
        return _lib.DT_F32
    if t.dtype == torch.float16:
        return _lib.DT_F16
    raise TypeError(f"unsupported output dtype {t.dtype}")


def _kv_code(t: torch.Tensor, kv_fp8: bool | None) -> int:
    if kv_fp8 is not None:
        return _lib.KV_FP8 if kv_fp8 else _lib.KV_BF16
    if t.dtype == torch.bfloat16:
        return _lib.KV_BF16
    if t.dtype in _FP8_DTYPES or t.dtype == torch.uint8:
        return _lib.KV_FP8
    raise TypeError(f"unsupported cache dtype {t.dtype}")


def _cache_strides(cache: torch.Tensor, page_size: int) -> tuple[int, int]:
    """(page_stride, token_stride) in elements. 4-D caches [pages, P, 1, row] carry the page stride;
    3-D caches [pages*P, 1, row] pack pages along the token dim. The real strides are read, never
    assumed: a cross-layer view has gaps (mla_decode_attention.py:78-84)."""
    if cache.dim() == 4:
        return cache.stride(0), cache.stride(1)
    if cache.dim() == 3:
        return cache.stride(0) * page_size, cache.stride(0)
    raise ValueError(f"cache must be 3-D or 4-D, got {tuple(cache.shape)}")


def _rms_mode(kv: int, rms_offset: int, rms_bf16: bool, rms_log8: bool) -> int:
    """Reference flag mapping (mla_decode_attention.py:466-505, mla_impl.py:302-307)."""
    if rms_offset < 0:
        return _lib.RMS_NONE
    if kv == _lib.KV_BF16:
        return _lib.RMS_BF16
    if rms_log8:
        return _lib.RMS_LOG8
    if rms_bf16:
        return _lib.RMS_BF16_BYTES
    return _lib.RMS_E4M3


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _check_layout(*, q_nope, q_pe, kv_cache, block_table, seq_lens, out, lse) -> None:
    """The kernels read int32 metadata with unit strides along a row (block_table) and along the
    batch (seq_lens), and every tensor row with a unit element stride. Anything else raises here:
    converting would allocate, which a caller inside HIP-graph capture cannot do."""
    if block_table.dtype != torch.int32:
        raise TypeError(f"block_table must be int32, got {block_table.dtype}")
    if seq_lens.dtype != torch.int32:
        raise TypeError(f"seq_lens must be int32, got {seq_lens.dtype}")
    if seq_lens.dim() != 1 or (seq_lens.numel() > 1 and seq_lens.stride(0) != 1):
        raise ValueError("seq_lens must be a contiguous 1-D tensor")
    if block_table.dim() != 2 or block_table.stride(-1) != 1:
        raise ValueError("block_table must be 2-D with a unit column stride")
    for name, t in (("q_nope", q_nope), ("q_pe", q_pe), ("kv_cache", kv_cache), ("out", out), ("lse", lse)):
        if t is not None and t.numel() > 0 and t.stride(-1) != 1:
            raise ValueError(f"{name} must have a unit stride in its last dimension")
    if q_nope.dtype != torch.bfloat16 or (q_pe is not None and q_pe.dtype != torch.bfloat16):
        raise TypeError("queries must be bfloat16")


def build_params(*, q_nope, q_pe, kv_cache, block_table, seq_lens, out, lse, d_c, rope_w, rms_offset,
                 rms_mode, kv, page_size, sm_scale, k_scale=None, logit_cap=0.0, qrows=1, groups=1,
                 rms_heads=None, num_splits=0, split_align=0, workspace=None, ws_strides=(0, 0, 0),
                 num_workgroups=0, status=None) -> DecodeParams:
    """Fill the C parameter block. Pure host work (no device access), so it is testable anywhere.
    Raises TypeError / ValueError for metadata or strides the kernels cannot read as given.

    The cache's page count bounds every block-table entry the kernels read: an entry outside it
    reads page 0 instead of faulting, and QMLA_ERR_PAGE is stored into `status` (a device int32
    tensor the caller clears) when one is given."""
    _check_layout(q_nope=q_nope, q_pe=q_pe if (q_pe is not None and rope_w > 0) else None, kv_cache=kv_cache,
                  block_table=block_table, seq_lens=seq_lens, out=out, lse=lse)
    rows, heads = q_nope.shape[0], q_nope.shape[1]
    page_stride, token_stride = _cache_strides(kv_cache, page_size)
    p = DecodeParams()
    p.q_nope = _ptr(q_nope)
    p.q_nope_stride_row, p.q_nope_stride_head = q_nope.stride(0), q_nope.stride(1)
    if q_pe is not None and rope_w > 0:
        p.q_pe = _ptr(q_pe)
        p.q_pe_stride_row, p.q_pe_stride_head = q_pe.stride(0), q_pe.stride(1)
    p.kv_cache = _ptr(kv_cache)
    p.page_stride, p.token_stride = page_stride, token_stride
    p.kv_dtype = kv
    p.page_size = page_size
    p.d_c, p.rope_w = d_c, rope_w
    p.rms_offset = rms_offset
    p.rms_mode = rms_mode
    p.k_scale = _ptr(k_scale)
    p.sm_scale = float(sm_scale)
    p.logit_cap = float(logit_cap)
    p.block_table = _ptr(block_table)
    p.bt_stride = block_table.stride(0)
    p.seq_lens = _ptr(seq_lens)
    p.rows, p.heads = rows, heads
    p.rms_heads = rms_heads if rms_heads is not None else heads
    p.qrows, p.groups = qrows, groups
    p.out = _ptr(out)
    p.out_stride_row, p.out_stride_head = out.stride(0), out.stride(1)
    p.out_dtype = _dt_code(out)
    if lse is not None:
        p.lse = _ptr(lse)
        p.lse_stride_row = lse.stride(0)
        p.lse_dtype = _dt_code(lse)
    p.num_splits, p.split_align = num_splits, split_align
    if workspace is not None:
        p.workspace = _ptr(workspace)
        p.workspace_bytes = workspace.numel() * workspace.element_size()
    p.ws_stride_row, p.ws_stride_head, p.ws_stride_split = ws_strides
    p.num_workgroups = num_workgroups
    p.num_pages = kv_cache.shape[0] if kv_cache.dim() == 4 else kv_cache.shape[0] // page_size
    if status is not None:
        # the kernels store into it from the device: it must live where the cache lives
        if status.dtype != torch.int32 or status.numel() < 1 or status.device != kv_cache.device:
            raise TypeError("status must be an int32 tensor on the cache's device")
        p.status = _ptr(status)
    return p


def workspace_bytes(params: DecodeParams) -> int:
    return int(_lib.lib().qmla_workspace_bytes(params))


def _check_device(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("qmla runs on the GPU only; got a tensor on " + str(t.device))


def fold_rows(params: DecodeParams, qrows: int) -> int:
    """Spec-verify tokens folded into one kernel request: the largest divisor d of qrows for which a
    compiled kernel serves d tokens x the heads as one request (qmla_decode_supported), so the cache
    is read once per group of d tokens instead of once per token. The reference folds groups of up
    to QWEN_MLA_VERIFY_MAX_ROWS = 64 rows (mla_decode_attention.py:1291-1310); the kernels here take
    up to 32 rows per workgroup and split a request's rows over up to four workgroups that read its
    token range together (48 rows per latent group for GLA-g2). `params` is left as it was."""
    lib = _lib.lib()
    saved = params.qrows
    best = 1
    try:
        for d in range(qrows, 1, -1):
            if qrows % d or params.rows % d:
                continue
            params.qrows = d
            if lib.qmla_decode_supported(params) == 0:
                best = d
                break
    finally:
        params.qrows = saved
    return best


def decode_attention_fwd(q, k_buffer, v_buffer, o, lse, req_to_token, b_seq_len, attn_logits,
                         num_kv_splits, sm_scale, page_size=1, logit_cap=0.0, k_scale=None, v_scale=None,
                         is_mla=False, rms_offset=-1, rms_bf16=False, rms_log8=False, qrows=1):
    """Drop-in for the reference decode entry (qwen_mla/ops/mla_decode_attention.py:1264-1359).

    Writes o [B, H, Lv], lse [B, H] (natural log) and the split partials attn_logits
    [B, H, S, Lv + 1] in place. qrows > 1 folds each run of qrows consecutive rows (one spec-verify
    request, as _build_decode flattens it) so the cache is read once per request. v_scale is
    accepted for signature parity; the latent serves as both key and value, so k_scale applies to
    both, as in the reference (mla_decode_attention.py:451-463).
    """
    if k_scale is not None and (not torch.is_tensor(k_scale) or k_scale.dtype != torch.float32
                                or k_scale.device != q.device):
        # the kernels read the scale through a device pointer; converting here would allocate,
        # which a caller inside HIP-graph capture cannot do
        raise TypeError("k_scale must be a float32 tensor on the query's device (the layer's _k_scale)")
    _check_device(q, k_buffer, o, req_to_token, b_seq_len, attn_logits)
    if k_buffer.shape[-2] != 1:
        raise NotImplementedError("only MLA (one latent KV head) is implemented")
    assert num_kv_splits == attn_logits.shape[2]
    Lv = v_buffer.shape[-1]
    Lk = k_buffer.shape[-1] if rms_offset < 0 else rms_offset
    B, H = q.shape[0], q.shape[1]
    kv = _kv_code(k_buffer, None)
    mode = _rms_mode(kv, rms_offset, rms_bf16, rms_log8)
    cache = k_buffer if k_buffer.dim() == 4 else k_buffer
    split_align = 16 if page_size % 16 == 0 else 0
    p = build_params(q_nope=q, q_pe=q[..., Lv:] if Lk > Lv else None, kv_cache=cache,
                     block_table=req_to_token, seq_lens=b_seq_len, out=o, lse=lse, d_c=Lv, rope_w=Lk - Lv,
                     rms_offset=rms_offset, rms_mode=mode, kv=kv, page_size=page_size, sm_scale=sm_scale,
                     k_scale=k_scale, logit_cap=logit_cap, qrows=1, groups=1, rms_heads=H,
                     num_splits=num_kv_splits, split_align=split_align, workspace=attn_logits,
                     ws_strides=(attn_logits.stride(0), attn_logits.stride(1), attn_logits.stride(2)))
    if qrows > 1 and B % qrows == 0:
        p.qrows = fold_rows(p, qrows)
    lib = _lib.lib()
    st = _stream()
    _lib.check("qmla_decode_partial", lib.qmla_decode_partial(p, st))
    if num_kv_splits > 1:
        _lib.check("qmla_combine", lib.qmla_combine(p, st))


class Workspace:
    """Device scratch for the balanced split mode, grown on demand and reused; allocate it (or call
    `reserve`) before HIP-graph capture so the captured call allocates nothing."""

    def __init__(self, device=None):
        self.device = device
        self.buf = None

    def reserve(self, nbytes: int, device) -> torch.Tensor:
        if self.buf is None or self.buf.numel() < nbytes or self.buf.device != torch.device(device):
            self.buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        return self.buf


_default_ws: dict = {}


def forward(q_nope, q_rope, kv_cache, block_table, seq_lens, *, d_c=None, rope_w=None, rms_offset=None,
            page_size, sm_scale, kv_fp8=None, fp8_rms="log8", k_scale=None, qrows=1, groups=1,
            rms_heads=None, logit_cap=0.0, out=None, lse=None, num_splits=0, workspace=None,
            num_workgroups=0, return_lse=True, status=None):
    """Decode every query row against its paged latent rows; returns (o, lse).

    q_nope [rows, H, d_c/G] absorbed latent queries, q_rope [rows, H, rope_w]; kv_cache
    [num_pages, page_size, (1,) row] with rows [latent d_c | rope rope_w | rms | pad]; block_table
    [rows, max_pages] int32, seq_lens [rows] int32 (spec-verify requests flattened one row per
    token). groups = 2 computes GLA-g2 (head h reads latent group h // (H/2)) in one launch and
    returns [rows, H, d_c/2]. num_splits = 0 selects the balanced split mode. Block-table entries
    outside the cache's pages read page 0 and store QMLA_ERR_PAGE into `status` (device int32).
    """
    _check_device(q_nope, kv_cache, block_table, seq_lens, status)
    rows, H = q_nope.shape[0], q_nope.shape[1]
    if d_c is None:
        d_c = q_nope.shape[-1] * groups
    if rope_w is None:
        rope_w = 0 if q_rope is None else q_rope.shape[-1]
    if rms_offset is None:
        rms_offset = d_c + rope_w
    kv = _kv_code(kv_cache, kv_fp8)
    mode = _rms_mode(kv, rms_offset, fp8_rms == "bf16", fp8_rms == "log8")
    dv = d_c // groups
    if out is None:
        out = torch.empty(rows, H, dv, dtype=torch.bfloat16, device=q_nope.device)
    if lse is None and return_lse:
        lse = torch.empty(rows, H, dtype=torch.float32, device=q_nope.device)
    if k_scale is not None and not torch.is_tensor(k_scale):
        k_scale = torch.tensor(float(k_scale), dtype=torch.float32, device=q_nope.device)
    if qrows > 1 and rows % qrows:
        raise ValueError(f"rows {rows} not a multiple of qrows {qrows}")
    if qrows > 1:
        probe = build_params(q_nope=q_nope, q_pe=q_rope, kv_cache=kv_cache, block_table=block_table,
                             seq_lens=seq_lens, out=out, lse=lse, d_c=d_c, rope_w=rope_w, rms_offset=rms_offset,
                             rms_mode=mode, kv=kv, page_size=page_size, sm_scale=sm_scale, logit_cap=logit_cap,
                             groups=groups, rms_heads=rms_heads, num_splits=num_splits)
        qrows = fold_rows(probe, qrows)
    args = dict(q_nope=q_nope, q_pe=q_rope, kv_cache=kv_cache, block_table=block_table, seq_lens=seq_lens,
                out=out, lse=lse, d_c=d_c, rope_w=rope_w, rms_offset=rms_offset, rms_mode=mode, kv=kv,
                page_size=page_size, sm_scale=sm_scale, k_scale=k_scale, logit_cap=logit_cap, qrows=qrows,
                groups=groups, rms_heads=rms_heads, num_splits=num_splits,
                split_align=16 if page_size % 16 == 0 else 0, num_workgroups=num_workgroups, status=status)
    lib = _lib.lib()
    ws_t = None
    ws_strides = (0, 0, 0)
    if num_splits > 1:
        ws_t = torch.empty(rows, H, num_splits, dv + 1, dtype=torch.float32, device=q_nope.device) \
            if workspace is None else workspace
        ws_strides = (ws_t.stride(0), ws_t.stride(1), ws_t.stride(2))
    elif num_splits == 0:
        need = workspace_bytes(build_params(**args))
        if isinstance(workspace, Workspace):
            ws_t = workspace.reserve(need, q_nope.device)
        elif workspace is not None:
            ws_t = workspace
        else:
            w = _default_ws.setdefault(q_nope.device, Workspace())
            ws_t = w.reserve(need, q_nope.device)
    p = build_params(workspace=ws_t, ws_strides=ws_strides, **args)
    _lib.check("qmla_decode", lib.qmla_decode(p, _stream()))
    return out, lse
