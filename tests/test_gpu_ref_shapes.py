"""The plugin's deployed FP8 layouts, built the way its own FP8 test builds them
(tests/test_fp8_kv.py:23-31, :79-100): latent x2 with four outlier channels x8, rope x1.5, rms
exp(N(0, 0.6)), query x0.05, per-layer scale = max|x| / 448, rows [latent | rope | rms | pad to 16],
784-token pages behind a permuted block table, ragged lengths ctx - (37 b) % 784, 32 fixed splits,
sm_scale 1/16, called through the reference's entry signature (decode_attention_fwd). Layouts: 24
heads with rope 232 (one GPU) and 12 heads with rope 116 (rank-local at TP 2); latent ranks 256, 768
and 1792 (:137); rms as log8 codes, raw bf16 bytes or e4m3.

The kernel is checked against the oracle on the same cache bytes (max-abs 3e-2, the FP8 bar, and
the reference test's own bar: max-rel < 2e-2 against the dequantized reference, :127).
"""
import math

import numpy as np
import pytest
import torch

from tests.mla_cases import C_REF, TOL, ora

pytestmark = pytest.mark.gpu

PAGE = 784
F8 = torch.float8_e4m3fn
ORA_MODE = {"log8": ora.RMS_LOG8, "bf16": ora.RMS_BF16_BYTES, "e4m3": ora.RMS_E4M3}


def _case(batch, heads, ctx, rank, rope, mode, seed):
    g = torch.Generator().manual_seed(seed)
    pps = (ctx + PAGE - 1) // PAGE
    lat = torch.randn(batch * pps, PAGE, rank, generator=g) * 2.0
    lat[..., :4] *= 8
    rp = torch.randn(batch * pps, PAGE, rope, generator=g) * 1.5
    rms = torch.exp(torch.randn(batch * pps, PAGE, heads, generator=g) * 0.6)
    q = (torch.randn(batch, heads, rank + rope, generator=g) * 0.05).to(torch.bfloat16)
    scale = float(max(lat.abs().max(), rp.abs().max())) / 448
    if mode == "bf16":
        rb = rms.to(torch.bfloat16).contiguous().view(torch.uint8)
    elif mode == "e4m3":
        rb = (rms / scale).clamp(-448, 448).to(F8).view(torch.uint8)
    else:
        rb = ((rms.log2() + 3.0) * (255.0 / 6.0)).round().clamp(0, 255).to(torch.uint8)
    row = torch.cat([(lat / scale).clamp(-448, 448).to(F8).view(torch.uint8),
                     (rp / scale).clamp(-448, 448).to(F8).view(torch.uint8), rb], -1)
    width = rank + rope + (2 if mode == "bf16" else 1) * heads
    width += (-width) % 16
    cache = torch.zeros(batch * pps, PAGE, 1, width, dtype=torch.uint8)
    cache[:, :, 0, :row.shape[-1]] = row
    bt = torch.randperm(batch * pps, generator=torch.Generator().manual_seed(1)).reshape(batch, pps).to(torch.int32)
    lens = torch.tensor([ctx - (37 * b) % PAGE for b in range(batch)], dtype=torch.int32)
    return q, cache, bt, lens, scale, width


@pytest.mark.parametrize("mode", ["log8", "bf16", "e4m3"])
@pytest.mark.parametrize("heads,rope", [(24, 232), (12, 116)])
@pytest.mark.parametrize("rank", [256, 768, 1792])
def test_deployed_fp8_layouts(gpu, mode, heads, rope, rank):
    import qmla
    batch, ctx = 4, 3000
    q, cache, bt, lens, scale, width = _case(batch, heads, ctx, rank, rope, mode, seed=rank + heads)
    cd = cache.to(gpu).view(F8)
    o = torch.zeros(batch, heads, rank, dtype=torch.bfloat16, device=gpu)
    lse = torch.zeros(batch, heads, dtype=torch.bfloat16, device=gpu)
    logits = torch.zeros(batch, heads, 32, rank + 1, dtype=torch.float32, device=gpu)
    ks = torch.tensor(scale, device=gpu)
    qmla.decode_attention_fwd(q.to(gpu), cd, cd[..., :rank], o, lse, bt.to(gpu), lens.to(gpu), logits, 32, 1 / 16.0,
                              PAGE, k_scale=ks, v_scale=ks, is_mla=True, rms_offset=rank + rope,
                              rms_bf16=mode == "bf16", rms_log8=mode == "log8")
    torch.cuda.synchronize()
    ro, rl = ora.mla_decode(q[..., :rank].float(), q[..., rank:].float(), cache.view(batch * bt.shape[1], PAGE, width),
                            bt, lens, page_size=PAGE, d_c=rank, rope_w=rope, rms_offset=rank + rope, kv="fp8",
                            rms_mode=ORA_MODE[mode], k_scale=scale, sm_scale=1 / 16.0, rms_heads=heads, groups=1)
    got = o.float().cpu()
    err = (got - ro).abs().max().item()
    rel = err / ro.abs().max().item()
    assert err < 3e-2 and rel < 2e-2, (err, rel)
    # lse is stored as bf16: its own rounding (2^-9 relative) is allowed
    assert ((lse.float().cpu() - rl).abs() - 2.0 ** -8 * rl.abs()).max().item() < 1e-2
    assert np.isfinite(got.numpy()).all()


def _bf16_case(batch, heads, ctx, rank, rope, page, seed):
    """tests/test_fi_partial_rope.py:27-46 with --shuffle --ragged --rms-spread: bf16 rows
    [latent | rope | one rms per head | pad to 16 bytes], rms exp(N(0,1)) per (key, head)."""
    g = torch.Generator().manual_seed(seed)
    entry = rank + rope + heads + (-(rope + heads)) % 8
    pps = (ctx + page - 1) // page
    cache = (torch.randn(batch * pps, page, 1, entry, generator=g) * 0.05).to(torch.bfloat16)
    cache[..., rank + rope:] = torch.exp(torch.randn(batch * pps, page, 1, entry - rank - rope, generator=g)).to(torch.bfloat16)
    q = (torch.randn(batch, heads, rank + rope, generator=g) * 0.05).to(torch.bfloat16)
    gb = torch.Generator().manual_seed(1)
    bt = torch.randperm(batch * pps, generator=gb).reshape(batch, pps).to(torch.int32)
    lens = torch.tensor([ctx - (int(torch.randint(0, page + 37, (1,), generator=gb)) if b else 0) for b in range(batch)],
                        dtype=torch.int32)
    return cache, q, bt, lens, entry


@pytest.mark.parametrize("rank,heads,rope", [(256, 24, 232), (256, 12, 116), (768, 24, 232), (768, 12, 116),
                                             (256, 24, 256), (256, 12, 256), (768, 24, 256), (768, 12, 256)])
def test_deployed_bf16_layouts(gpu, rank, heads, rope):
    """The layouts of tests/test_fi_partial_rope.py:105 (tp1, tp2, and the full-rope tp1full / tp2full)
    at its ranks 256 and 768 (:109)."""
    import qmla
    batch, ctx, page = 4, 2048, 400
    cache, q, bt, lens, entry = _bf16_case(batch, heads, ctx, rank, rope, page, seed=rank + heads)
    cd = cache.to(gpu)
    o = torch.zeros(batch, heads, rank, dtype=torch.bfloat16, device=gpu)
    lse = torch.zeros(batch, heads, dtype=torch.bfloat16, device=gpu)
    logits = torch.zeros(batch, heads, 64, rank + 1, dtype=torch.float32, device=gpu)
    qmla.decode_attention_fwd(q.to(gpu), cd, cd[..., :rank], o, lse, bt.to(gpu), lens.to(gpu), logits, 64,
                              1.0 / 256 ** 0.5, page, is_mla=True, rms_offset=rank + rope)
    torch.cuda.synchronize()
    cu8 = cache.view(torch.uint8).view(cache.shape[0], page, entry * 2)
    ro, rl = ora.mla_decode(q[..., :rank].float(), q[..., rank:].float(), cu8, bt, lens, page_size=page, d_c=rank,
                            rope_w=rope, rms_offset=rank + rope, kv="bf16", rms_mode=ora.RMS_BF16,
                            sm_scale=1.0 / 256 ** 0.5, rms_heads=heads, groups=1)
    eo, _ = ora.mla_decode_reference_rounding(q[..., :rank].float(), q[..., rank:].float(), cu8, bt, lens,
                                              page_size=page, d_c=rank, rope_w=rope, rms_offset=rank + rope, kv="bf16",
                                              rms_mode=ora.RMS_BF16, sm_scale=1.0 / 256 ** 0.5, rms_heads=heads,
                                              num_splits=64, align=16)
    got = o.float().cpu()
    err = (got - ro).abs().max().item()
    ref_err = (eo.to(torch.bfloat16).float() - ro).abs().max().item()
    print(f"[bf16 rank {rank} heads {heads} rope {rope}] max-abs {err:.3e} (reference roundings {ref_err:.3e})")
    assert err < max(TOL["bf16"], C_REF * ref_err), err
    # lse is stored as bf16: its own rounding (2^-9 relative) is allowed
    assert ((lse.float().cpu() - rl).abs() - 2.0 ** -8 * rl.abs()).max().item() < 1e-2


@pytest.mark.parametrize("ctx,batch", [(4096, 4), (16384, 6)])
@pytest.mark.parametrize("heads,rope", [(24, 232), (12, 116), (24, 256), (12, 256)])
def test_deployed_bf16_rank1792(gpu, heads, rope, ctx, batch):
    """tests/test_two_pass_1792.py:10-19: rank 1792 on the bf16 rows of test_fi_partial_rope.py
    (784-token pages, shuffled table, ragged lengths, rms exp(N(0,1)) per key and head), 24 heads with
    rope 232 (TP 1), 12 with 116 (TP 2), and full rope 256; through decode_attention_fwd with fixed
    splits and through forward in the balanced mode."""
    import qmla
    rank, page = 1792, 784
    cache, q, bt, lens, entry = _bf16_case(batch, heads, ctx, rank, rope, page, seed=7 + heads + ctx)
    cd = cache.to(gpu)
    splits = 8 if ctx == 4096 else 16
    o = torch.full((batch, heads, rank), float("nan"), dtype=torch.bfloat16, device=gpu)
    lse = torch.zeros(batch, heads, dtype=torch.float32, device=gpu)
    logits = torch.zeros(batch, heads, splits, rank + 1, dtype=torch.float32, device=gpu)
    qd = q.to(gpu)
    qmla.decode_attention_fwd(qd, cd, cd[..., :rank], o, lse, bt.to(gpu), lens.to(gpu), logits, splits,
                              1.0 / 256 ** 0.5, page, is_mla=True, rms_offset=rank + rope)
    ob, lb = qmla.forward(qd[..., :rank], qd[..., rank:], cd, bt.to(gpu), lens.to(gpu), d_c=rank, rope_w=rope,
                          rms_offset=rank + rope, page_size=page, sm_scale=1.0 / 256 ** 0.5, rms_heads=heads)
    torch.cuda.synchronize()
    cu8 = cache.view(torch.uint8).view(cache.shape[0], page, entry * 2)
    kw = dict(page_size=page, d_c=rank, rope_w=rope, rms_offset=rank + rope, kv="bf16", rms_mode=ora.RMS_BF16,
              sm_scale=1.0 / 256 ** 0.5, rms_heads=heads)
    ro, rl = ora.mla_decode(q[..., :rank].float(), q[..., rank:].float(), cu8, bt, lens, **kw)
    eo, _ = ora.mla_decode_reference_rounding(q[..., :rank].float(), q[..., rank:].float(), cu8, bt, lens,
                                              num_splits=splits, align=16, **kw)
    ref_err = (eo.to(torch.bfloat16).float() - ro).abs().max().item()
    bound = max(TOL["bf16"], C_REF * ref_err)
    for name, out, l in (("fixed", o, lse), ("balanced", ob, lb)):
        err = (out.float().cpu() - ro).abs().max().item()
        lerr = (l.float().cpu() - rl).abs().max().item()
        print(f"[bf16 rank 1792 heads {heads} rope {rope} ctx {ctx} {name}] max-abs {err:.3e} "
              f"(reference roundings {ref_err:.3e}, bound {bound:.3e}) lse {lerr:.3e}", flush=True)
        assert err < bound and lerr < 1e-2


def _numerics_case(batch, heads, rank, page, lens, seed, shuffle):
    """tests/test_decode_numerics.py:60-67: unpadded rows [latent | 256 packed rope | one bf16 rms per
    head] (rank + 256 + heads elements), entries N(0, 0.05), rms |x| + 0.3, query N(0, 0.05)."""
    g = torch.Generator().manual_seed(seed)
    entry = rank + 256 + heads
    pps = (max(lens) + page - 1) // page
    cache = (torch.randn(batch * pps + 4, page, 1, entry, generator=g) * 0.05).to(torch.bfloat16)
    cache[..., rank + 256:] = cache[..., rank + 256:].abs() + 0.3
    q = (torch.randn(batch, heads, rank + 256, generator=g) * 0.05).to(torch.bfloat16)
    order = torch.randperm(batch * pps, generator=g) if shuffle else torch.arange(batch * pps)
    bt = order.reshape(batch, pps).to(torch.int32)
    return cache, q, bt, torch.tensor(lens, dtype=torch.int32), entry


@pytest.mark.parametrize("page", [400, 401])
@pytest.mark.parametrize("heads", [12, 24])
@pytest.mark.parametrize("rank", [256, 768, 1792])
def test_numerics_test_rows(gpu, rank, heads, page):
    """The reference's standalone numerics test (tests/test_decode_numerics.py:60-91): B 2 x 900 tokens
    on 400-token pages, 8 fixed splits, sm_scale 1/16, through decode_attention_fwd. Its 12-head rows
    (1048 / 2072 / 4120 bytes) sit on 8-byte boundaries and take the narrow-row kernels; the 24-head
    rows are 16-byte aligned. Also a ragged, shuffled batch in the balanced mode (forward), and
    401-token pages, whose page starts are off 16-byte boundaries too and whose tiles straddle pages.
    Checked against the oracle at the bf16 bar and at the reference test's own bar (norm-relative
    error < 5e-2)."""
    import qmla
    kw = dict(page_size=page, d_c=rank, rope_w=256, rms_offset=rank + 256, kv="bf16", rms_mode=ora.RMS_BF16,
              sm_scale=1.0 / 16, rms_heads=heads)
    for name, lens, shuffle in (("fixed", [900, 900], False), ("balanced", [2500, 1, 900, 0, 1777], True)):
        batch = len(lens)
        cache, q, bt, sl, entry = _numerics_case(batch, heads, rank, page, lens, seed=rank + heads + page, shuffle=shuffle)
        cd, qd = cache.to(gpu), q.to(gpu)
        if name == "fixed":
            o = torch.zeros(batch, heads, rank, dtype=torch.bfloat16, device=gpu)
            lse = torch.zeros(batch, heads, dtype=torch.bfloat16, device=gpu)
            logits = torch.zeros(batch, heads, 8, rank + 1, dtype=torch.float32, device=gpu)
            qmla.decode_attention_fwd(qd, cd, cd[..., :rank], o, lse, bt.to(gpu), sl.to(gpu), logits, 8, 1.0 / 16,
                                      page, is_mla=True, rms_offset=rank + 256)
        else:
            o, lse = qmla.forward(qd[..., :rank], qd[..., rank:], cd, bt.to(gpu), sl.to(gpu), d_c=rank, rope_w=256,
                                  rms_offset=rank + 256, page_size=page, sm_scale=1.0 / 16, rms_heads=heads)
        torch.cuda.synchronize()
        cu8 = cache.view(torch.uint8).view(cache.shape[0], page, entry * 2)
        ro, rl = ora.mla_decode(q[..., :rank].float(), q[..., rank:].float(), cu8, bt, sl, **kw)
        got = o.float().cpu()
        err = (got - ro).abs().max().item()
        rel = ((got - ro).norm() / ro.norm().clamp(min=1e-9)).item()
        live = sl > 0
        lerr = (lse.float().cpu()[live] - rl[live]).abs().max().item()
        print(f"[numerics rows rank {rank} heads {heads} page {page} {name}] max-abs {err:.3e} rel {rel:.2e} "
              f"lse {lerr:.3e}", flush=True)
        assert err < TOL["bf16"] and rel < 5e-2, (err, rel)
        assert lerr < 2e-2


@pytest.mark.parametrize("qrows", [2, 4])
@pytest.mark.parametrize("rank", [256, 768, 1792])
def test_numerics_test_rows_verify(gpu, rank, qrows):
    """The same unpadded 12-head rows (rank + 256 + 12 bf16 elements, on 8-byte boundaries) with
    spec-verify rows folded into one request (2 or 4 tokens x 12 heads: 24 or 48 rows, split over the
    narrow-row instances' workgroups where they exceed one), 401-token pages, short and empty requests,
    through forward in the balanced mode and with 8 fixed splits."""
    import qmla
    from tests.mla_cases import check_decode, make_case
    c = make_case(batch=5, heads=12, d_c=rank, rope_w=256, page_size=401, lens=[2500, 3, 900, 0, 1777],
                  kv="bf16", rms_mode="bf16", seed=rank + qrows, device=gpu, qrows=qrows, rms="spread", pad=False)
    assert c.cache.shape[-1] == rank + 256 + 12
    for splits in (0, 8):
        kw = dict(num_splits=splits) if splits else {}
        o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, d_c=c.d_c, rope_w=c.rope_w,
                              rms_offset=c.d_c + c.rope_w, page_size=c.page_size, sm_scale=c.sm_scale, qrows=qrows,
                              **kw)
        torch.cuda.synchronize()
        check_decode(f"numerics rows rank {rank} q{qrows} splits {splits}", c, o, lse, num_splits=max(splits, 1))
