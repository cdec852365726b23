"""Decode q / k_pe prep: the attention module's per-token work between its projections and the
attention call, as one HIP launch (libqmla.so, `qmla_prep`).

Mirrors Qwen3_5MLAAttention.forward (qwen_mla/qwen3_5_mla.py:262-301) from the normed query, the
latent, the raw rope key and the raw up-projection to the two tensors the attention layer takes:

* rms[t, h] = sqrt((sum bf16(latent . k_up_h)^2 + sum k_rope[t, g]^2) / head_dim + eps), the
  per-(token, head) score divisor, g = (head_offset + h) // rope_group (:239-240, :262-265);
* one neox rotation of q[..., :rd] and of bf16(k_rope * (1 + k_norm.weight[:rd])) with the cos/sin
  row of each token's position, in bf16 arithmetic (:274-283, :341-354), M-RoPE positions [3, n]
  included;
* q_out = [q[..., rd:] | q_pe], q_pe zero except the head's group slot (:289-292, :303);
* k_pe = [rotated rope keys of the cached groups | bf16(rms) | zero padding] (:293-301).

There is no CPU path: a missing library raises.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_DT = {torch.bfloat16: _lib.DT_BF16, torch.float32: _lib.DT_F32, torch.float16: _lib.DT_F16}


def k_gain(k_norm_weight: torch.Tensor, rope_dim: int) -> torch.Tensor:
    """(1 + k_norm.weight)[:rope_dim] in fp32, the gain the rope key takes before its rotation
    (Qwen3.5's (1 + w) RMSNorm weight, qwen3_5_mla.py:236, :279). Computed once per layer."""
    return (1.0 + k_norm_weight.float())[:rope_dim].contiguous()


def partial_rope_table(keep, model_rope_dim: int, theta: float, max_pos: int, *,
                       device=None, dtype=torch.float32) -> torch.Tensor:
    """The cos/sin table [max_pos, 2*len(keep)] with each kept subspace at its original frequency
    theta^(-2*keep[i]/model_rope_dim), angles accumulated in float32 (partial_rope.py:66-76). Built
    once per model; keep=range(model_rope_dim // 2) is the full-width table."""
    inv = 1.0 / (theta ** (2.0 * torch.tensor(list(keep), dtype=torch.float32) / model_rope_dim))
    freqs = torch.outer(torch.arange(max_pos, dtype=torch.float32), inv)
    return torch.cat([freqs.cos(), freqs.sin()], dim=-1).to(dtype=dtype, device=device)


def mla_decode_prep(positions: torch.Tensor, q: torch.Tensor, latent: torch.Tensor, k_rope: torch.Tensor,
                    k_up_raw: torch.Tensor, k_gain: torch.Tensor, cos_sin_cache: torch.Tensor, *,
                    head_offset: int, rope_group: int, rope_first: int, rope_span: int, declared_rope: int,
                    eps: float, rope_sec: torch.Tensor | None = None, q_out: torch.Tensor | None = None,
                    k_pe: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """q [n, H, head_dim] (bf16, rope dims first, last dim contiguous), latent [n, d_c], k_rope
    [n, kv_heads * rd] or [n, kv_heads, rd], k_up_raw [H * nope, d_c], k_gain fp32 [rd] (see
    `k_gain`), cos_sin_cache [max_pos, rd] (bf16, fp32 or fp16; rounded to bf16 for the rotation),
    positions [n] or [3, n] with rope_sec [rd/2] (M-RoPE: the position row of each frequency).

    Returns (q_out [n, H, nope + declared_rope], k_pe [n, declared_rope]), both bf16, written into
    the given tensors when passed. Positions outside the table give NaN in the rotated elements.
    """
    p, keep, q_out, k_pe = prep_params(positions, q, latent, k_rope, k_up_raw, k_gain, cos_sin_cache,
                                       head_offset=head_offset, rope_group=rope_group, rope_first=rope_first,
                                       rope_span=rope_span, declared_rope=declared_rope, eps=eps, rope_sec=rope_sec,
                                       q_out=q_out, k_pe=k_pe)
    _lib.check("qmla_prep", _lib.lib().qmla_prep(ctypes.byref(p), torch.cuda.current_stream().cuda_stream))
    s = torch.cuda.current_stream()
    for t in keep:
        t.record_stream(s)
    return q_out, k_pe


def prep_params(positions, q, latent, k_rope, k_up_raw, k_gain, cos_sin_cache, *, head_offset, rope_group,
                rope_first, rope_span, declared_rope, eps, rope_sec=None, q_out=None, k_pe=None):
    """The `qmla_prep_params` of a `mla_decode_prep` call, the converted tensors it points into (keep
    them alive), and the two outputs."""
    if q.dim() != 3:
        raise ValueError("mla_decode_prep: q must be [n, heads, head_dim]")
    n, H, hd = q.shape
    rd = cos_sin_cache.shape[-1]
    nope = hd - rd
    d_c = latent.shape[-1]
    dev = q.device
    for name, t in (("q", q), ("latent", latent), ("k_rope", k_rope), ("k_up_raw", k_up_raw), ("k_gain", k_gain),
                    ("cos_sin_cache", cos_sin_cache), ("positions", positions)):
        if not t.is_cuda:
            raise ValueError(f"mla_decode_prep: {name} must live on the GPU")
    for name, t in (("q", q), ("latent", latent), ("k_rope", k_rope), ("k_up_raw", k_up_raw)):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"mla_decode_prep: {name} must be bf16")
    if cos_sin_cache.dtype not in _DT or cos_sin_cache.dim() != 2 or not cos_sin_cache.is_contiguous():
        raise TypeError("mla_decode_prep: cos_sin_cache must be a contiguous [max_pos, rd] bf16/fp32/fp16 table")
    if q.stride(-1) != 1:
        raise ValueError("mla_decode_prep: q's last dimension must be contiguous")
    lat = latent.reshape(-1, d_c)
    kr = k_rope.reshape(k_rope.shape[0], -1)
    if lat.shape[0] < n or kr.shape[0] < n or lat.stride(-1) != 1 or kr.stride(-1) != 1:
        raise ValueError("mla_decode_prep: latent / k_rope need n contiguous rows")
    if kr.shape[1] % rd:
        raise ValueError("mla_decode_prep: k_rope width is not a multiple of the rope dim")
    kv_heads = kr.shape[1] // rd
    ku = k_up_raw.contiguous()
    if tuple(ku.shape) != (H * nope, d_c):
        raise ValueError(f"mla_decode_prep: k_up_raw must be [{H * nope}, {d_c}], got {tuple(ku.shape)}")
    gain = k_gain.to(torch.float32).contiguous()
    if gain.numel() < rd:
        raise ValueError("mla_decode_prep: k_gain needs rope_dim entries")
    pos = positions.to(torch.int64)
    if pos.dim() == 1:
        pos = pos.contiguous()
        rows, prs, sec = 1, 0, None
    elif pos.dim() == 2 and pos.shape[0] == 3:
        pos = pos.contiguous()
        if rope_sec is None:
            raise ValueError("mla_decode_prep: M-RoPE positions need rope_sec")
        sec = rope_sec.to(device=dev, dtype=torch.int32).contiguous()
        if sec.numel() < rd // 2:
            raise ValueError("mla_decode_prep: rope_sec needs rd/2 entries")
        rows, prs = 3, pos.stride(0)
    else:
        raise ValueError("mla_decode_prep: positions must be [n] or [3, n]")
    if pos.shape[-1] < n:
        raise ValueError("mla_decode_prep: fewer positions than tokens")
    if q_out is None:
        q_out = torch.empty(n, H, nope + declared_rope, dtype=torch.bfloat16, device=dev)
    if k_pe is None:
        k_pe = torch.empty(n, declared_rope, dtype=torch.bfloat16, device=dev)
    if q_out.dtype != torch.bfloat16 or k_pe.dtype != torch.bfloat16 or q_out.stride(-1) != 1 or k_pe.stride(-1) != 1:
        raise ValueError("mla_decode_prep: outputs must be bf16 with a contiguous last dimension")
    kp = k_pe.reshape(k_pe.shape[0], -1)

    p = _lib.PrepParams()
    p.q, p.q_token_stride, p.q_head_stride = q.data_ptr(), q.stride(0), q.stride(1)
    p.latent, p.latent_stride = lat.data_ptr(), lat.stride(0)
    p.k_rope, p.k_rope_stride = kr.data_ptr(), kr.stride(0)
    p.k_up = ku.data_ptr()
    p.k_gain = gain.data_ptr()
    p.cos_sin, p.cos_sin_dtype, p.max_pos = cos_sin_cache.data_ptr(), _DT[cos_sin_cache.dtype], cos_sin_cache.shape[0]
    p.positions, p.pos_row_stride, p.pos_rows = pos.data_ptr(), prs, rows
    p.rope_sec = sec.data_ptr() if sec is not None else None
    p.n, p.heads, p.head_dim, p.rope_dim, p.kv_heads, p.d_c = n, H, hd, rd, kv_heads, d_c
    p.head_offset, p.rope_group, p.rope_first, p.rope_span = head_offset, rope_group, rope_first, rope_span
    p.declared_rope, p.eps = declared_rope, eps
    p.q_out, p.q_out_token_stride, p.q_out_head_stride = q_out.data_ptr(), q_out.stride(0), q_out.stride(1)
    p.k_pe, p.k_pe_stride = kp.data_ptr(), kp.stride(0)
    return p, (ku, gain, pos) + ((sec,) if sec is not None else ()), q_out, k_pe
