"""The writer and the gather at prefill sizes (65536 rows and more), where they take several rows a
wave: bit-exact against the oracle on every cache format they serve, with the slot -1 redirect,
chunks that start inside the sequences, tokens outside every sequence, and, for the writer's log8
codes, rms values on and beside every rounding midpoint of the code grid (the fast log2 path hands
those to the double one)."""
import numpy as np
import pytest
import torch

from tests.mla_cases import cache_bytes, make_case, ora

pytestmark = pytest.mark.gpu

N = 70000


@pytest.mark.parametrize("rms,mode", [("log8", ora.RMS_LOG8), ("bf16", ora.RMS_BF16_BYTES), ("e4m3", ora.RMS_E4M3),
                                      ("none", ora.RMS_NONE)])
@pytest.mark.parametrize("d_c,rope,heads", [(512, 64, 24), (768, 232, 24), (256, 116, 12)])
def test_writer_large_bit_exact(gpu, d_c, rope, heads, rms, mode):
    import qmla
    g = torch.Generator().manual_seed(d_c + heads)
    kv_c = (torch.randn(N, d_c, generator=g) * 4).to(torch.bfloat16)
    rms_v = torch.exp(torch.randn(N, heads, generator=g) * 2.0)
    # rms on, and one bf16 step either side of, the midpoints between log8 codes
    c = np.arange(255, dtype=np.float64)
    mids = torch.from_numpy(np.exp2(-3 + (c + 0.5) * 6 / 255)).float().to(torch.bfloat16)
    mb = mids.view(torch.int16)
    edge = torch.cat([mids, (mb + 1).view(torch.bfloat16), (mb - 1).view(torch.bfloat16)]).float()
    flat = rms_v.view(-1)
    flat[:edge.numel()] = edge
    flat[edge.numel():edge.numel() + 4] = torch.tensor([0.0, 1e-35, float("inf"), 1e10])
    k_pe = torch.empty(N, rope + heads, dtype=torch.bfloat16)
    k_pe[:, :rope] = (torch.randn(N, rope, generator=g) * 4).to(torch.bfloat16)
    k_pe[:, rope:] = rms_v.to(torch.bfloat16)
    rb = 2 if rms == "bf16" else (0 if rms == "none" else 1)
    width = d_c + rope + rb * heads
    width += (-width) % 16
    P = 64
    pages = (2 * N) // P
    rng = np.random.default_rng(d_c)
    slots = 1 + rng.permutation(pages * P - 1)[:N]
    slots[7::1000] = -1                                   # padding rows -> slot 0
    ks = 0.0123456
    cache = torch.full((pages, P, 1, width), 0xAB, dtype=torch.uint8, device=gpu)
    qmla.cache_write(kv_c.to(gpu), k_pe.to(gpu), cache, torch.as_tensor(slots).to(gpu), rope_w=rope,
                     rms_heads=heads if rms != "none" else 0, kv_fp8=True, rms=rms,
                     k_scale=torch.tensor(ks, device=gpu))
    torch.cuda.synchronize()
    got = cache.cpu().view(pages * P, width).numpy()
    kc, kp = kv_c.float().numpy(), k_pe.float().numpy()
    inv = np.float32(1.0) / np.float32(ks)
    q = lambda x: ora.e4m3_encode(np.clip(x.astype(np.float32) * inv, -448.0, 448.0))
    if mode in (ora.RMS_LOG8, ora.RMS_BF16_BYTES):
        exp = ora.fp8_row_bytes(kc, kp, packed_rope=rope, n_heads=heads, k_scale=ks, rms_mode=mode)
    elif mode == ora.RMS_E4M3:
        exp = np.concatenate([q(kc), q(kp[:, :rope]), q(kp[:, rope:])], axis=1)
    else:
        exp = np.concatenate([q(kc), q(kp[:, :rope])], axis=1)
    nb = exp.shape[1]
    keep = slots >= 0
    bad = np.nonzero((got[slots[keep], :nb] != exp[keep]).any(axis=1))[0]
    assert bad.size == 0, (rms, bad[:5])
    assert np.all(got[slots[keep], nb:] == 0xAB), "bytes past the written row were touched"
    untouched = np.setdiff1d(np.arange(pages * P), np.maximum(slots, 0))
    assert np.all(got[untouched] == 0xAB)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rms", ["log8", "bf16_bytes", "e4m3"])
@pytest.mark.parametrize("d_c,rope,heads", [(512, 64, 24), (768, 232, 24)])
def test_gather_large_bit_exact(gpu, d_c, rope, heads, rms, dtype):
    import qmla
    lens = [40000, 25000, 7, 10000]
    c = make_case(batch=len(lens), heads=heads, d_c=d_c, rope_w=rope, page_size=64, lens=lens, kv="fp8",
                  rms_mode=rms, seed=d_c + len(rms), device=gpu, rms="spread", amp=4.0)
    u8 = c.cache.view(torch.uint8).view(c.cache.shape[0], 64, -1)
    u8[int(c.block_table[0, 0]), :2, :256] = torch.arange(256, dtype=torch.uint8, device=gpu).masked_fill(
        (torch.arange(256, device=gpu) & 0x7F) == 0x7F, 0)      # every finite e4m3 code, -0 included
    # a chunk that starts inside the sequences, and tokens of no sequence (token_to_seq -1)
    starts = [1000, 0, 0, 2500]
    chunk = [30000, 25000, 7, 7500]
    cl = torch.tensor(chunk, dtype=torch.int64)
    cu = torch.zeros(len(chunk) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(cl, 0).to(torch.int32)
    n = int(cl.sum()) + 64
    t2s = torch.cat([torch.repeat_interleave(torch.arange(len(chunk), dtype=torch.int32), cl),
                     torch.full((64,), -1, dtype=torch.int32)])
    ss = torch.tensor(starts, dtype=torch.int32)
    mode = {"log8": "log8", "bf16_bytes": "bf16", "e4m3": "e4m3"}[rms]
    dst = torch.full((n + 3, c.row), 0x7E7E, dtype=torch.int16, device=gpu).view(dtype)
    qmla.gather_cache(src_cache=c.cache, dst=dst, block_table=c.block_table, cu_seq_lens=cu.to(gpu),
                      token_to_seq=t2s.to(gpu), num_tokens=n, kv_cache_dtype="fp8", scale=c.k_scale,
                      seq_starts=ss.to(gpu), mla_rms=(c.rms_offset, c.heads, mode))
    torch.cuda.synchronize()
    got = dst.view(torch.int16).cpu().numpy().view(np.uint16)
    m = n - 64
    omode = {"log8": ora.RMS_LOG8, "bf16_bytes": ora.RMS_BF16_BYTES, "e4m3": ora.RMS_E4M3}[rms]
    cb = cache_bytes(c).numpy()
    exp = ora.gather_context(cb, c.block_table.cpu().numpy(), cu.numpy(), t2s[:m].numpy(), m, ss.numpy(), kv="fp8",
                             scale=float(c.k_scale.cpu()), rms_offset=c.rms_offset, n_heads=c.heads, rms_mode=omode)
    if dtype == torch.float16:
        # the same values rounded to fp16 instead of bf16: bf16 bit patterns -> exact fp32 is not
        # enough (the fp32 product is rounded once), so the fp32 values are rebuilt from the bytes
        sc = np.float32(float(c.k_scale.cpu()))
        s_ = t2s[:m].numpy().astype(np.int64)
        tok = np.arange(m) - cu.numpy().astype(np.int64)[s_] + ss.numpy().astype(np.int64)[s_]
        blk = c.block_table.cpu().numpy()[s_, tok // 64].astype(np.int64)
        rows = cb[blk, tok % 64].reshape(m, -1)
        ro = c.rms_offset
        f32 = np.zeros((m, ro + c.heads), np.float32)
        f32[:, :ro] = ora.e4m3_decode(rows[:, :ro]) * sc
        code = rows[:, ro:ro + c.heads]
        if omode == ora.RMS_LOG8:
            f32[:, ro:] = ora.log8_decode(code)
        elif omode == ora.RMS_E4M3:
            f32[:, ro:] = ora.e4m3_decode(code) * sc
        else:
            f32[:, ro:] = (rows[:, ro:ro + 2 * c.heads].copy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        exp = np.zeros_like(exp)
        exp[:, :ro + c.heads] = f32.astype(np.float16).view(np.uint16)
    k = c.rms_offset + c.heads
    assert np.array_equal(got[:m, :k], exp[:m, :k]), np.argwhere(got[:m, :k] != exp[:m, :k])[:5]
    assert np.all(got[:, k:] == 0x7E7E) and np.all(got[m:] == 0x7E7E)
