"""Cache rows: the writer (the new token's latent, rope and rms tail into its paged slot) and the
prefill context gather (paged rows back into the dense bf16 workspace the prefill path reads).

Mirrors QwenMLATritonImpl.do_kv_cache_update (qwen_mla/mla_impl.py:309-342): FP8 caches get
`[latent e4m3 | rope e4m3 | rms tail]` with e4m3 = RNE of clamp(x * (1/k_scale), -448, 448) and the
tail a log8 code per head (mode "log8"), the rms as two bf16 bytes per head ("bf16"), or e4m3 like
the rope ("e4m3", the bytes vLLM's concat_and_cache_mla writes for the plugin in that mode); bf16
caches get the row copied. Padding slots (-1) go to slot 0, vLLM's never-read null block. Runs as one
HIP kernel on the current stream (libqmla.so, `qmla_cache_write`); there is no CPU path.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_RMS_WRITE = {"log8": _lib.RMS_LOG8, "bf16": _lib.RMS_BF16_BYTES, "e4m3": _lib.RMS_E4M3}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def cache_write(kv_c: torch.Tensor, k_pe: torch.Tensor, kv_cache: torch.Tensor, slot_mapping: torch.Tensor, *,
                d_c: int | None = None, rope_w: int, rms_heads: int, kv_fp8: bool | None = None,
                rms: str = "log8", k_scale: torch.Tensor | None = None) -> None:
    """Write len(slot_mapping) rows: kv_c [>= n, d_c] and k_pe [>= n, rope_w + rms tail] (bf16) into
    kv_cache [num_pages, page_size, (1,) row] at the flat slots (page * page_size + token).

    rms: "log8" | "bf16" | "e4m3" | "none" for FP8 caches, "bf16" | "none" for bf16 caches.
    """
    p, keep = cache_write_params(kv_c, k_pe, kv_cache, slot_mapping, d_c=d_c, rope_w=rope_w, rms_heads=rms_heads,
                                 kv_fp8=kv_fp8, rms=rms, k_scale=k_scale)
    _lib.check("qmla_cache_write", _lib.lib().qmla_cache_write(ctypes.byref(p), _stream()))
    cur = torch.cuda.current_stream()
    for t in keep:
        t.record_stream(cur)


def cache_write_params(kv_c: torch.Tensor, k_pe: torch.Tensor, kv_cache: torch.Tensor, slot_mapping: torch.Tensor,
                       *, d_c: int | None = None, rope_w: int, rms_heads: int, kv_fp8: bool | None = None,
                       rms: str = "log8", k_scale: torch.Tensor | None = None):
    """The `qmla_cache_write_params` of a `cache_write` call, and the tensors it points into that the
    caller must keep alive (converted copies). For callers that launch the same write repeatedly."""
    slots = slot_mapping.reshape(-1)
    n = slots.shape[0]
    if kv_fp8 is None:
        kv_fp8 = kv_cache.dtype in (torch.uint8, torch.float8_e4m3fn)
    if d_c is None:
        d_c = kv_c.shape[-1]
    for t in (kv_c, k_pe, kv_cache, slots):
        if not t.is_cuda:
            raise ValueError("cache_write: every tensor must live on the GPU")
    if kv_c.dtype != torch.bfloat16 or k_pe.dtype != torch.bfloat16:
        raise TypeError("cache_write: kv_c and k_pe must be bf16")
    kv_c2 = kv_c.reshape(kv_c.shape[0], -1)
    k_pe2 = k_pe.reshape(k_pe.shape[0], -1)
    if kv_c2.shape[0] < n or k_pe2.shape[0] < n:
        raise ValueError("cache_write: fewer input rows than slots")
    if kv_c2.stride(-1) != 1 or k_pe2.stride(-1) != 1:
        raise ValueError("cache_write: rows must be contiguous in their last dimension")
    slots = slots.to(torch.int64)
    p = _lib.CacheWriteParams()
    p.kv_c, p.kv_c_stride = kv_c2.data_ptr(), kv_c2.stride(0)
    p.k_pe, p.k_pe_stride = k_pe2.data_ptr(), k_pe2.stride(0)
    p.slots = slots.data_ptr()
    p.n, p.d_c, p.rope_w, p.rms_heads = n, d_c, rope_w, rms_heads
    if kv_fp8:
        p.kv_dtype = _lib.KV_FP8
        p.rms_mode = _lib.RMS_NONE if rms == "none" else _RMS_WRITE[rms]
        if k_scale is None:
            raise ValueError("cache_write: FP8 caches need k_scale")
        ks = k_scale.reshape(-1)[:1].to(device=kv_cache.device, dtype=torch.float32).contiguous()
        p.k_scale = ks.data_ptr()
    else:
        p.kv_dtype = _lib.KV_BF16
        p.rms_mode = {"bf16": _lib.RMS_BF16, "none": _lib.RMS_NONE}[rms]
    esz = kv_cache.element_size()
    p.cache = kv_cache.data_ptr()
    p.page_stride, p.token_stride = kv_cache.stride(0) * esz, kv_cache.stride(1) * esz
    p.page_size = kv_cache.shape[1]
    p.num_slots = kv_cache.shape[0] * kv_cache.shape[1]
    return p, ((slots, ks) if kv_fp8 else (slots,))


def do_kv_cache_update(kv_c_normed: torch.Tensor, k_pe: torch.Tensor, kv_cache: torch.Tensor,
                       slot_mapping: torch.Tensor, kv_cache_dtype: str, k_scale: torch.Tensor, *,
                       packed_rope: int, n_heads: int, rms_mode: str = "log8") -> None:
    """The reference method's signature (mla_impl.py:309) with the layer attributes it reads
    (`mla_packed_rope`, `mla_local_heads`, `mla_fp8_rms_mode()`) as keywords. kv_cache_dtype
    "fp8*" writes FP8 rows, anything else bf16 rows with the rms tail copied."""
    if kv_cache.numel() == 0:
        return
    fp8 = str(kv_cache_dtype).startswith("fp8")
    d_c = kv_c_normed.shape[-1]
    cache_write(kv_c_normed, k_pe, kv_cache, slot_mapping, d_c=d_c, rope_w=packed_rope, rms_heads=n_heads,
                kv_fp8=fp8, rms=(rms_mode if fp8 else "bf16"), k_scale=k_scale)


_RMS_GATHER = {"log8": _lib.RMS_LOG8, "bf16": _lib.RMS_BF16_BYTES, "e4m3": _lib.RMS_E4M3}


def gather_cache(*, src_cache: torch.Tensor, dst: torch.Tensor, block_table: torch.Tensor,
                 cu_seq_lens: torch.Tensor, token_to_seq: torch.Tensor, num_tokens: int,
                 kv_cache_dtype: str, scale: torch.Tensor, seq_starts: torch.Tensor | None = None,
                 mla_rms=None) -> None:
    """gather_cache_torch (qwen_mla/ops/mla_gather.py:28-76) on the device, same keywords.

    Destination row j: s = token_to_seq[j], tok = j - cu_seq_lens[s] (+ seq_starts[s]); the cached
    row at block_table[s, tok // P], slot tok % P. bf16 caches copy the row; FP8 caches (mla_rms =
    (rms_offset, heads[, "log8" | "bf16" | "e4m3"])) write bf16(e4m3 * scale) for the first rms_offset
    columns and one decoded rms element per head after them.
    """
    if num_tokens <= 0:
        if not str(kv_cache_dtype).startswith("fp8") and kv_cache_dtype not in ("auto", "bfloat16", "float16"):
            raise NotImplementedError(f"MLA gather has no dequant path for kv_cache_dtype={kv_cache_dtype}")
        return
    p, keep = gather_params(src_cache=src_cache, dst=dst, block_table=block_table, cu_seq_lens=cu_seq_lens,
                            token_to_seq=token_to_seq, num_tokens=num_tokens, kv_cache_dtype=kv_cache_dtype,
                            scale=scale, seq_starts=seq_starts, mla_rms=mla_rms)
    _lib.check("qmla_gather", _lib.lib().qmla_gather(ctypes.byref(p), _stream()))
    cur = torch.cuda.current_stream()
    for t in keep:
        t.record_stream(cur)


def gather_params(*, src_cache: torch.Tensor, dst: torch.Tensor, block_table: torch.Tensor,
                  cu_seq_lens: torch.Tensor, token_to_seq: torch.Tensor, num_tokens: int,
                  kv_cache_dtype: str, scale: torch.Tensor, seq_starts: torch.Tensor | None = None, mla_rms=None):
    """The `qmla_gather_params` of a `gather_cache` call (num_tokens > 0), and the converted tensors it
    points into that the caller must keep alive."""
    fp8 = str(kv_cache_dtype).startswith("fp8")
    if not fp8 and kv_cache_dtype not in ("auto", "bfloat16", "float16"):
        raise NotImplementedError(f"MLA gather has no dequant path for kv_cache_dtype={kv_cache_dtype}")
    if fp8 and mla_rms is None:
        raise NotImplementedError("FP8 MLA gather needs the row layout (rms offset, heads)")
    for t in (src_cache, dst, block_table, cu_seq_lens, token_to_seq):
        if not t.is_cuda:
            raise ValueError("gather_cache: every tensor must live on the GPU")
    if dst.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("gather_cache: dst must be bf16 or fp16")
    dst2 = dst.reshape(dst.shape[0], -1)
    if dst2.stride(-1) != 1 or dst2.shape[0] < num_tokens:
        raise ValueError("gather_cache: dst rows must be contiguous and cover num_tokens")
    i32 = lambda t: t.to(torch.int32).contiguous()
    bt, cu, t2s = i32(block_table), i32(cu_seq_lens), i32(token_to_seq)
    ss = i32(seq_starts) if seq_starts is not None else None
    p = _lib.GatherParams()
    esz = src_cache.element_size()
    p.cache = src_cache.data_ptr()
    p.page_stride, p.token_stride = src_cache.stride(0) * esz, src_cache.stride(1) * esz
    p.page_size, p.num_pages = src_cache.shape[1], src_cache.shape[0]
    if fp8:
        off, nh = mla_rms[:2]
        mode = mla_rms[2] if len(mla_rms) > 2 else "bf16"
        p.kv_dtype, p.rms_mode, p.rms_offset, p.rms_heads = _lib.KV_FP8, _RMS_GATHER[mode], off, nh
        sc = scale.reshape(-1)[:1].to(device=dst.device, dtype=torch.float32).contiguous()
        p.scale = sc.data_ptr()
    else:
        p.kv_dtype, p.row_elems = _lib.KV_BF16, src_cache.reshape(src_cache.shape[0], src_cache.shape[1], -1).shape[-1]
    p.block_table, p.bt_stride = bt.data_ptr(), bt.stride(0)
    p.num_seqs, p.bt_cols = bt.shape[0], bt.shape[1]
    p.cu_seq_lens, p.token_to_seq = cu.data_ptr(), t2s.data_ptr()
    p.seq_starts = ss.data_ptr() if ss is not None else None
    p.num_tokens = num_tokens
    p.dst, p.dst_stride = dst2.data_ptr(), dst2.stride(0)
    p.dst_dtype = _lib.DT_BF16 if dst.dtype == torch.bfloat16 else _lib.DT_F16
    return p, tuple(t for t in (bt, cu, t2s, ss, sc if fp8 else None) if t is not None)
