"""Row-layout helpers, the FP8 row writer and the prefill context gather of the oracle.

Known answers for the row width are the ones the reference quotes in its docstrings
(qwen_mla/mla_impl.py:238-251, qwen_mla/partial_rope.py:10-13). The FP8 writer is checked against
torch's own float8_e4m3fn conversion of the writer's expression (qwen_mla/mla_impl.py:328-339),
and the gather against explicit index loops and its sliced/unsliced identity
(tests/test_fp8_kv.py:111-122).
"""
from __future__ import annotations

import types

import numpy as np
import pytest
import torch

from oracle import mla_oracle as ora
from qmla import layout

F8 = getattr(torch, "float8_e4m3fn", None)


def _hf(keep=None, ranks=(256, 768, 1792), groups=1):
    return types.SimpleNamespace(num_attention_heads=24, num_key_value_heads=4, head_dim=256,
                                 partial_rotary_factor=0.25, rope_parameters=None,
                                 mla_ranks={i: r for i, r in enumerate(ranks)}, mla_rope_keep=keep,
                                 mla_latent_groups=groups)


def test_row_width_known_answers():
    hf = _hf()
    assert layout.mla_base_tail(hf, 1) == 280
    assert [layout.mla_padded_head_size(hf, r, 1) for r in (256, 768, 1792)] == [544, 1088, 2176]
    assert layout.mla_base_tail(hf, 2) == 140
    assert [layout.mla_padded_head_size(hf, r, 2) for r in (256, 768, 1792)] == [512, 1024, 2048]
    hk = _hf(keep=list(range(29)))
    assert layout.effective_rope_dim(hk) == 58
    assert layout.mla_base_tail(hk, 1) == 256
    assert [layout.mla_padded_head_size(hk, r, 1) for r in (256, 768, 1792)] == [512, 1024, 2048]
    assert layout.rank_layout(512, 64, 24).row == 608
    assert layout.rank_layout(1792, 64, 24).row == 1888
    assert layout.rank_layout(512, 64, 24, fp8=True).row == 608
    # every width divides the largest one (pages of all layers unify)
    ws = [layout.mla_padded_head_size(hf, r, 1) for r in (256, 768, 1792)]
    assert all(max(ws) % w == 0 for w in ws)
    assert layout.mla_rank_by_head_size(hf, 1) == {544: 256, 1088: 768, 2176: 1792}


def test_gla_and_window_helpers():
    hf = _hf(groups=2)
    assert layout.mla_gla_split(hf, 2) == 2 and layout.mla_gla_split(hf, 1) == 1
    assert layout.mla_local_ranks(hf, 2) == {0: 128, 1: 384, 2: 896}
    assert layout.rope_window(12, 12, 6, 64) == (0, 128)
    assert layout.rope_window(0, 24, 6, 64) == (0, 256)
    assert layout.row_dma_safe(608, 64, 512, 0, 1) and not layout.row_dma_safe(600, 64, 512, 0, 1)
    assert layout.splitk_cap(128, 24, 513, 64, 512.0) == 64
    assert layout.splitk_cap(1024, 24, 513, 64, 512.0) == 8


@pytest.mark.skipif(F8 is None, reason="torch without float8_e4m3fn")
@pytest.mark.parametrize("mode", ["log8", "bf16_bytes"])
def test_fp8_writer_matches_torch_expression(mode):
    g = torch.Generator().manual_seed(3)
    n, d_c, pr, nh = 37, 64, 16, 6
    kv_c = (torch.randn(n, d_c, generator=g) * 40).bfloat16()
    k_pe = torch.cat([torch.randn(n, pr, generator=g) * 40,
                      torch.exp(torch.randn(n, nh, generator=g))], dim=1).bfloat16()
    k_scale = torch.tensor(0.0371)
    inv = (1.0 / k_scale.float()).reshape(())
    lat = (kv_c.float() * inv).clamp_(-448.0, 448.0).to(F8).view(torch.uint8)
    rope = (k_pe[:, :pr].float() * inv).clamp_(-448.0, 448.0).to(F8).view(torch.uint8)
    if mode == "log8":
        code = (k_pe[:, pr:pr + nh].float().clamp_min(1e-30).log2() + 3.0) * (255.0 / 6.0)
        rms = code.round_().clamp_(0, 255).to(torch.uint8)
    else:
        rms = k_pe[:, pr:pr + nh].to(torch.bfloat16).contiguous().view(torch.uint8)
    want = torch.cat([lat, rope, rms], dim=-1).numpy()
    got = ora.fp8_row_bytes(kv_c.float().numpy(), k_pe.float().numpy(), packed_rope=pr, n_heads=nh,
                            k_scale=float(k_scale), rms_mode=mode)
    assert np.array_equal(got, want)
    # some latent values saturate at +-448 (code 0x7E / 0xFE)
    assert np.isin(got[:, :d_c], [0x7E, 0xFE]).any()


def test_fp8_cache_write_redirects_padding_slot():
    cache = np.zeros((10, 32), np.uint8)
    rows = np.arange(3 * 20, dtype=np.uint8).reshape(3, 20) + 1
    ora.fp8_cache_write(cache, np.array([4, -1, 7]), rows)
    assert np.array_equal(cache[4, :20], rows[0]) and np.array_equal(cache[7, :20], rows[2])
    assert np.array_equal(cache[0, :20], rows[1])
    assert not cache[:, 20:].any()


def _gather_loops(cache, bt, cu, t2s, n, starts):
    P = cache.shape[1]
    out = []
    for j in range(n):
        s = int(t2s[j])
        tok = j - int(cu[s]) + (0 if starts is None else int(starts[s]))
        out.append(cache[int(bt[s, tok // P]), tok % P].reshape(-1))
    return np.stack(out)


@pytest.mark.skipif(F8 is None, reason="torch without float8_e4m3fn")
@pytest.mark.parametrize("mode", [ora.RMS_LOG8, ora.RMS_BF16_BYTES, ora.RMS_E4M3])
def test_gather_context_fp8(mode):
    rng = np.random.default_rng(4)
    P, pages, row, d, nh = 4, 12, 48, 32, 4
    off = d
    cache = rng.integers(0, 256, (pages, P, row), dtype=np.uint8)
    cache[..., :d + (2 * nh if mode == ora.RMS_BF16_BYTES else nh)] &= 0x77   # no NaN codes
    bt = rng.permutation(pages).astype(np.int32)[:9].reshape(3, 3)
    lens = np.array([5, 9, 3])
    cu = np.concatenate([[0], np.cumsum(lens)])
    t2s = np.repeat(np.arange(3), lens)
    n = int(cu[-1])
    got = ora.gather_context(cache, bt, cu, t2s, n, None, kv="fp8", scale=0.5, rms_offset=off, n_heads=nh,
                             rms_mode=mode)
    raw = _gather_loops(cache, bt, cu, t2s, n, None)
    tv = lambda b: torch.from_numpy(np.ascontiguousarray(b)).view(F8).float() * 0.5   # noqa: E731
    bits = lambda x: x.bfloat16().view(torch.int16).numpy().view(np.uint16)           # noqa: E731
    if mode == ora.RMS_E4M3:
        assert np.array_equal(got[:, :off + nh], bits(tv(raw[:, :off + nh])))
    else:
        assert np.array_equal(got[:, :off], bits(tv(raw[:, :off])))
        if mode == ora.RMS_LOG8:
            want = torch.exp2(-3 + torch.from_numpy(raw[:, off:off + nh].astype(np.float64)) * 6 / 255).float()
            assert np.array_equal(got[:, off:off + nh], bits(want))
        else:
            assert np.array_equal(got[:, off:off + nh], raw[:, off:off + 2 * nh].copy().view(np.uint16))
    # sliced == unsliced: a window starting at seq_starts reads the same rows as the full gather
    starts = np.array([2, 4, 0])
    lens2 = lens - starts
    cu2 = np.concatenate([[0], np.cumsum(lens2)])
    t2s2 = np.repeat(np.arange(3), lens2)
    part = ora.gather_context(cache, bt, cu2, t2s2, int(cu2[-1]), starts, kv="fp8", scale=0.5, rms_offset=off,
                              n_heads=nh, rms_mode=mode)
    full_idx = np.concatenate([cu[s] + np.arange(starts[s], lens[s]) for s in range(3)])
    assert np.array_equal(part, got[full_idx])


def test_gather_context_bf16_copies_rows():
    rng = np.random.default_rng(5)
    cache = rng.integers(0, 256, (6, 4, 64), dtype=np.uint8)
    bt = np.array([[3, 1], [5, 0]], np.int32)
    lens = np.array([6, 7])
    cu = np.concatenate([[0], np.cumsum(lens)])
    t2s = np.repeat(np.arange(2), lens)
    got = ora.gather_context(cache, bt, cu, t2s, 13, None, kv="bf16")
    assert np.array_equal(got.view(np.uint8), _gather_loops(cache, bt, cu, t2s, 13, None))
