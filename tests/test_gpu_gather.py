"""GPU parity of the prefill context gather (qmla_gather) against the oracle's restatement of
gather_cache_torch (ops/mla_gather.py:28-76): the index math (sequence, token, page, slot from the
chunk metadata) and the dequant are bit-exact, columns past the decoded row are left alone, and a
chunk that starts inside the sequences (seq_starts) equals the matching rows of the unsliced gather
(the reference's tests/test_fp8_kv.py:111-122 property).
"""
import numpy as np
import pytest
import torch

from tests.mla_cases import cache_bytes, make_case, ora

pytestmark = pytest.mark.gpu

SENT = 0x7E7E   # sentinel bit pattern in the destination


def _meta(chunk_lens, starts=None):
    chunk_lens = torch.tensor(chunk_lens, dtype=torch.int64)
    cu = torch.zeros(len(chunk_lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(chunk_lens, 0).to(torch.int32)
    t2s = torch.repeat_interleave(torch.arange(len(chunk_lens), dtype=torch.int32), chunk_lens)
    ss = None if starts is None else torch.tensor(starts, dtype=torch.int32)
    return cu, t2s, ss, int(chunk_lens.sum())


def _run(gpu, c, kv_cache_dtype, mla_rms, cu, t2s, ss, n, width, dtype=torch.bfloat16):
    import qmla
    dst = torch.full((n + 3, width), SENT, dtype=torch.int16, device=gpu).view(dtype)
    scale = c.k_scale if c.k_scale is not None else torch.ones((), device=gpu)
    qmla.gather_cache(src_cache=c.cache, dst=dst, block_table=c.block_table, cu_seq_lens=cu.to(gpu),
                      token_to_seq=t2s.to(gpu), num_tokens=n, kv_cache_dtype=kv_cache_dtype, scale=scale,
                      seq_starts=None if ss is None else ss.to(gpu), mla_rms=mla_rms)
    torch.cuda.synchronize()
    return dst.view(torch.int16).cpu().numpy().view(np.uint16)


def _oracle(c, cu, t2s, ss, n, kv, rms_mode):
    ks = float(c.k_scale.cpu()) if c.k_scale is not None else 1.0
    return ora.gather_context(cache_bytes(c).numpy(), c.block_table.cpu().numpy(), cu.numpy(), t2s.numpy(), n,
                              None if ss is None else ss.numpy(), kv=kv, scale=ks, rms_offset=c.rms_offset,
                              n_heads=c.heads, rms_mode=rms_mode)


@pytest.mark.parametrize("rms", ["log8", "bf16_bytes", "e4m3"])
def test_fp8_gather_bit_exact(gpu, rms):
    lens = [700, 64, 1500, 3]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv="fp8", rms_mode=rms,
                  seed=21, device=gpu, rms="spread", amp=4.0)
    u8 = c.cache.view(torch.uint8).view(c.cache.shape[0], 64, -1)
    u8[int(c.block_table[0, 0]), :2, :256] = torch.arange(256, dtype=torch.uint8, device=gpu).masked_fill(
        (torch.arange(256, device=gpu) & 0x7F) == 0x7F, 0)      # every finite e4m3 code, -0 included
    cu, t2s, ss, n = _meta(lens)
    mode = {"log8": "log8", "bf16_bytes": "bf16", "e4m3": "e4m3"}[rms]
    width = c.row
    got = _run(gpu, c, "fp8", (c.rms_offset, c.heads, mode), cu, t2s, ss, n, width)
    exp = _oracle(c, cu, t2s, ss, n, "fp8", {"log8": ora.RMS_LOG8, "bf16_bytes": ora.RMS_BF16_BYTES,
                                             "e4m3": ora.RMS_E4M3}[rms])
    k = c.rms_offset + c.heads
    assert np.array_equal(got[:n, :k], exp[:, :k]), np.argwhere(got[:n, :k] != exp[:, :k])[:5]
    assert np.all(got[:n, k:] == SENT) and np.all(got[n:] == SENT)


def test_log8_tail_every_code(gpu):
    """All 256 codes decode to the oracle's bf16 (2^(-3 + code*6/255))."""
    lens = [256]
    c = make_case(batch=1, heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv="fp8", rms_mode="log8",
                  seed=22, device=gpu)
    u8 = c.cache.view(torch.uint8).view(c.cache.shape[0], 64, -1)
    bt = c.block_table.cpu()
    for t in range(256):
        u8[int(bt[0, t // 64]), t % 64, c.rms_offset:c.rms_offset + c.heads] = (t + torch.arange(c.heads)) % 256
    cu, t2s, ss, n = _meta(lens)
    got = _run(gpu, c, "fp8", (c.rms_offset, c.heads, "log8"), cu, t2s, ss, n, c.row)
    exp = _oracle(c, cu, t2s, ss, n, "fp8", ora.RMS_LOG8)
    assert np.array_equal(got[:n, c.rms_offset:c.rms_offset + c.heads], exp[:, c.rms_offset:c.rms_offset + c.heads])


def test_bf16_gather_copies_rows(gpu):
    lens = [100, 900, 33]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=16, lens=lens, kv="bf16", seed=23,
                  device=gpu)
    cu, t2s, ss, n = _meta(lens)
    got = _run(gpu, c, "auto", None, cu, t2s, ss, n, c.row)
    exp = _oracle(c, cu, t2s, ss, n, "bf16", ora.RMS_NONE)
    assert np.array_equal(got[:n], exp) and np.all(got[n:] == SENT)


@pytest.mark.parametrize("kv", ["fp8", "bf16"])
def test_sliced_window_equals_unsliced(gpu, kv):
    """Chunks that start inside the sequences (seq_starts) give the same rows as the whole gather."""
    lens = [1200, 300, 777]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv=kv, seed=24,
                  device=gpu, rms="spread")
    dt = "fp8" if kv == "fp8" else "auto"
    rms = (c.rms_offset, c.heads, "log8") if kv == "fp8" else None
    cu, t2s, ss, n = _meta(lens)
    full = _run(gpu, c, dt, rms, cu, t2s, ss, n, c.row)
    starts, clen = [500, 0, 77], [400, 300, 700]
    cu2, t2s2, ss2, n2 = _meta(clen, starts)
    part = _run(gpu, c, dt, rms, cu2, t2s2, ss2, n2, c.row)
    rows = np.concatenate([np.arange(st, st + cl) + int(cu[s]) for s, (st, cl) in enumerate(zip(starts, clen))])
    assert np.array_equal(part[:n2], full[rows])
    exp = _oracle(c, cu2, t2s2, ss2, n2, kv, ora.RMS_LOG8 if kv == "fp8" else ora.RMS_NONE)
    k = c.rms_offset + c.heads if kv == "fp8" else c.row
    assert np.array_equal(part[:n2, :k], exp[:, :k])


def test_fp16_destination(gpu):
    """fp16 workspaces: e4m3 * scale rounded to fp16 (torch's conversion of the fp32 product)."""
    lens = [300]
    c = make_case(batch=1, heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv="fp8", rms_mode="log8",
                  seed=25, device=gpu, amp=4.0)
    # every e4m3 code (negative zero and subnormals included) in the first rows' latent
    u8 = c.cache.view(torch.uint8).view(c.cache.shape[0], 64, -1)
    first = int(c.block_table[0, 0])
    u8[first, :4, :256] = torch.arange(256, dtype=torch.uint8, device=gpu).masked_fill(
        (torch.arange(256, device=gpu) & 0x7F) == 0x7F, 0)      # no NaN codes
    cu, t2s, ss, n = _meta(lens)
    got = _run(gpu, c, "fp8", (c.rms_offset, c.heads, "log8"), cu, t2s, ss, n, c.row, dtype=torch.float16)
    rows = ora.gather_rows(cache_bytes(c), c.block_table.cpu(), 0, n, 64).numpy()
    lat = torch.from_numpy(ora.e4m3_decode(rows[:, :c.rms_offset])) * float(c.k_scale.cpu())
    exp = lat.to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    bad = np.argwhere(got[:n, :c.rms_offset] != exp)
    assert bad.size == 0, [(float(lat[r, k]), hex(got[r, k]), hex(exp[r, k])) for r, k in bad[:6]] + [len(bad)]
    rms = torch.from_numpy(ora.log8_decode(rows[:, c.rms_offset:c.rms_offset + c.heads])).to(torch.float16)
    assert np.array_equal(got[:n, c.rms_offset:c.rms_offset + c.heads], rms.view(torch.int16).numpy().view(np.uint16))


def test_wide_latent_gather(gpu):
    """d_c 1792 FP8 rows (rms offset 1856, the per-row kernel): bit-exact against the oracle."""
    lens = [300, 77]
    c = make_case(batch=2, heads=24, d_c=1792, rope_w=64, page_size=16, lens=lens, kv="fp8", rms_mode="log8",
                  seed=26, device=gpu, rms="spread")
    cu, t2s, ss, n = _meta(lens)
    got = _run(gpu, c, "fp8", (c.rms_offset, c.heads, "log8"), cu, t2s, ss, n, c.row)
    exp = _oracle(c, cu, t2s, ss, n, "fp8", ora.RMS_LOG8)
    k = c.rms_offset + c.heads
    assert np.array_equal(got[:n, :k], exp[:, :k]) and np.all(got[:n, k:] == SENT)
