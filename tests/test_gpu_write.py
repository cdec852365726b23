"""GPU parity of the cache-row writer (qmla_cache_write) against the oracle's restatement of the
plugin's FP8 writer (mla_impl.py:309-342): bit-exact bytes for latent and rope (e4m3 of the scaled,
saturated values, round to nearest even), log8 codes, bf16 rms bytes, the slot -1 redirect, and the
bytes it must not touch. Then the round trip: rows written on the device decode like the oracle's.
"""
import math

import numpy as np
import pytest
import torch

from tests.mla_cases import ora

pytestmark = pytest.mark.gpu

D_C, ROPE, H = 512, 64, 24


def _e4m3_values():
    """Every finite e4m3 value, the midpoints between neighbours (ties) and the bf16 values just
    beside each midpoint, both signs: all exact in bf16."""
    v = np.sort(np.unique(np.abs(ora.e4m3_decode(np.arange(256, dtype=np.uint8)))))
    v = v[np.isfinite(v)]
    mid = (v[1:] + v[:-1]) / 2
    bf = lambda x: torch.tensor(x, dtype=torch.float32).to(torch.bfloat16)
    near = []
    for m in mid:
        b = bf(m).view(torch.int16).item()
        near += [torch.tensor([b - 1, b + 1], dtype=torch.int16).view(torch.bfloat16).float().numpy()]
    allv = np.concatenate([v, mid, np.concatenate(near), [500.0, 1e4, 448.0 + 16]])
    return np.concatenate([allv, -allv]).astype(np.float32)


def _inputs(n, seed, amp=4.0, rms=None):
    g = torch.Generator().manual_seed(seed)
    kv_c = (torch.randn(n, D_C, generator=g) * amp).to(torch.bfloat16)
    k_pe = torch.empty(n, ROPE + H, dtype=torch.bfloat16)
    k_pe[:, :ROPE] = (torch.randn(n, ROPE, generator=g) * amp).to(torch.bfloat16)
    if rms is None:
        rms = torch.exp(torch.randn(n, H, generator=g) * 2.0)
    k_pe[:, ROPE:] = rms.to(torch.bfloat16)
    return kv_c, k_pe


def _expected_rows(kv_c, k_pe, k_scale, mode):
    kc, kp = kv_c.float().numpy(), k_pe.float().numpy()
    if mode in (ora.RMS_LOG8, ora.RMS_BF16_BYTES):
        return ora.fp8_row_bytes(kc, kp, packed_rope=ROPE, n_heads=H, k_scale=k_scale, rms_mode=mode)
    inv = np.float32(1.0) / np.float32(k_scale)
    q = lambda x: ora.e4m3_encode(np.clip(x.astype(np.float32) * inv, -448.0, 448.0))
    if mode == ora.RMS_E4M3:
        return np.concatenate([q(kc), q(kp[:, :ROPE]), q(kp[:, ROPE:])], axis=1)
    return np.concatenate([q(kc), q(kp[:, :ROPE])], axis=1)


def _write(gpu, kv_c, k_pe, slots, k_scale, rms, pages=40, P=64, width=608):
    import qmla
    cache = torch.full((pages, P, 1, width), 0xAB, dtype=torch.uint8, device=gpu)
    ks = torch.tensor(k_scale, dtype=torch.float32, device=gpu)
    qmla.cache_write(kv_c.to(gpu), k_pe.to(gpu), cache, torch.as_tensor(slots, dtype=torch.int64).to(gpu),
                     rope_w=ROPE, rms_heads=H, kv_fp8=True, rms=rms, k_scale=ks)
    torch.cuda.synchronize()
    return cache.cpu().view(pages * P, width).numpy()


@pytest.mark.parametrize("rms,mode,width", [("log8", ora.RMS_LOG8, 608), ("bf16", ora.RMS_BF16_BYTES, 624),
                                            ("e4m3", ora.RMS_E4M3, 608), ("none", ora.RMS_NONE, 576)])
def test_fp8_rows_bit_exact(gpu, rms, mode, width):
    n = 300
    kv_c, k_pe = _inputs(n, seed=1)
    k_scale = 0.0123456
    rng = np.random.default_rng(2)
    slots = 1 + rng.permutation(40 * 64 - 1)[:n]   # distinct, slot 0 left to the padding row
    slots[5] = -1                                   # padding row -> slot 0
    got = _write(gpu, kv_c, k_pe, slots, k_scale, rms, width=width)
    exp = _expected_rows(kv_c, k_pe, k_scale, mode)
    nb = exp.shape[1]
    written = np.maximum(slots, 0)
    for i, s in enumerate(written):
        assert np.array_equal(got[s, :nb], exp[i]), (rms, i, s, np.nonzero(got[s, :nb] != exp[i])[0][:8])
    assert np.all(got[written, nb:] == 0xAB), "bytes past the written row were touched"
    untouched = np.setdiff1d(np.arange(got.shape[0]), written)
    assert np.all(got[untouched] == 0xAB)


def test_e4m3_grid_ties_and_saturation(gpu):
    """Every e4m3 value, every tie and its bf16 neighbours, beyond-range values, scale 1 and a
    generic scale: the device conversion rounds exactly as torch's (pinned by the oracle)."""
    vals = _e4m3_values()
    n = math.ceil(vals.size / D_C)
    flat = np.zeros(n * D_C, np.float32)
    flat[:vals.size] = vals
    kv_c = torch.from_numpy(flat.reshape(n, D_C)).to(torch.bfloat16)
    k_pe = torch.zeros(n, ROPE + H, dtype=torch.bfloat16)
    k_pe[:, :ROPE] = kv_c[:, :ROPE]
    k_pe[:, ROPE:] = 1.0
    for k_scale in (1.0, 0.37, 3.0):
        got = _write(gpu, kv_c, k_pe, np.arange(n), k_scale, "log8")
        exp = _expected_rows(kv_c, k_pe, k_scale, ora.RMS_LOG8)
        bad = np.nonzero(got[:n, :exp.shape[1]] != exp)
        assert bad[0].size == 0, (k_scale, [(float(kv_c.float()[r, c]) if c < D_C else None, got[r, c], exp[r, c])
                                            for r, c in zip(*bad)][:6])


def test_log8_codes_edges(gpu):
    """rms at and around the code grid (2^(-3 + c*6/255)), the clamp at 1e-30, zero, huge values."""
    c = np.arange(256, dtype=np.float64)
    grid = np.exp2(-3 + c * 6 / 255)
    mids = np.exp2(-3 + (c[:-1] + 0.5) * 6 / 255)
    vals = np.concatenate([grid, mids, mids * (1 + 2.0 ** -8), mids * (1 - 2.0 ** -8),
                           [0.0, 1e-35, 1e-30, 1e-20, 0.124, 8.01, 1e10, 1.0]])
    n = math.ceil(vals.size / H)
    flat = np.ones(n * H, np.float32)
    flat[:vals.size] = vals
    rms = torch.from_numpy(flat.reshape(n, H))
    kv_c, k_pe = _inputs(n, seed=3, rms=rms)
    got = _write(gpu, kv_c, k_pe, np.arange(n), 0.05, "log8")
    exp = _expected_rows(kv_c, k_pe, 0.05, ora.RMS_LOG8)
    assert np.array_equal(got[:n, D_C + ROPE:D_C + ROPE + H], exp[:, D_C + ROPE:])


def test_bf16_rows_copied(gpu):
    import qmla
    n, P, pages = 50, 16, 10
    kv_c, k_pe = _inputs(n, seed=4)
    cache = torch.zeros(pages, P, 1, 600, dtype=torch.bfloat16, device=gpu)
    slots = torch.randperm(pages * P)[:n]
    qmla.cache_write(kv_c.to(gpu), k_pe.to(gpu), cache, slots.to(gpu), rope_w=ROPE, rms_heads=H, kv_fp8=False,
                     rms="bf16")
    torch.cuda.synchronize()
    flat = cache.cpu().view(pages * P, 600)
    assert torch.equal(flat[slots, :D_C], kv_c)
    assert torch.equal(flat[slots, D_C:D_C + ROPE + H], k_pe)
    rest = torch.ones(pages * P, dtype=torch.bool)
    rest[slots] = False
    assert torch.count_nonzero(flat[rest]) == 0 and torch.count_nonzero(flat[slots, D_C + ROPE + H:]) == 0


def test_written_cache_decodes_like_the_oracle(gpu):
    """Write a whole context with the device writer, decode it with the library and with the oracle
    on the oracle's own rows: the same bytes, so the same result."""
    import qmla
    lens = [700, 129, 1000]
    P = 64
    pages_per = [math.ceil(L / P) for L in lens]
    total_pages = sum(pages_per) + 2
    perm = torch.randperm(total_pages, generator=torch.Generator().manual_seed(5))
    bt = torch.zeros(len(lens), max(pages_per), dtype=torch.int32)
    k = 0
    slot_list = []
    for b, L in enumerate(lens):
        bt[b, :pages_per[b]] = perm[k:k + pages_per[b]].to(torch.int32)
        k += pages_per[b]
        t = torch.arange(L)
        slot_list.append(bt[b, t // P].long() * P + t % P)
    slots = torch.cat(slot_list)
    n = slots.numel()
    kv_c, k_pe = _inputs(n, seed=6)
    k_scale = 0.0199
    cache = torch.zeros(total_pages, P, 1, 608, dtype=torch.uint8, device=gpu)
    ks = torch.tensor(k_scale, dtype=torch.float32, device=gpu)
    qmla.cache_write(kv_c.to(gpu), k_pe.to(gpu), cache, slots.to(gpu), rope_w=ROPE, rms_heads=H, kv_fp8=True,
                     rms="log8", k_scale=ks)
    ref = np.zeros((total_pages * P, 608), np.uint8)
    ora.fp8_cache_write(ref, slots.numpy(), _expected_rows(kv_c, k_pe, k_scale, ora.RMS_LOG8))
    torch.cuda.synchronize()
    assert np.array_equal(cache.cpu().view(-1, 608).numpy(), ref)
    g = torch.Generator().manual_seed(7)
    qn = torch.randn(len(lens), H, D_C, generator=g).to(torch.bfloat16)
    qp = torch.randn(len(lens), H, ROPE, generator=g).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32)
    sm = 1 / math.sqrt(D_C + ROPE)
    o, lse = qmla.forward(qn.to(gpu), qp.to(gpu), cache, bt.to(gpu), sl.to(gpu), page_size=P, sm_scale=sm,
                          kv_fp8=True, fp8_rms="log8", k_scale=ks, num_workgroups=4)
    torch.cuda.synchronize()
    ro, rl = ora.mla_decode(qn.float(), qp.float(), torch.from_numpy(ref).view(total_pages, P, 608), bt, sl,
                            page_size=P, d_c=D_C, rope_w=ROPE, rms_offset=D_C + ROPE, kv="fp8",
                            rms_mode=ora.RMS_LOG8, k_scale=k_scale, sm_scale=sm, rms_heads=H, groups=1)
    err = ((o.float().cpu() - ro).abs() - 2.0 ** -7 * ro.abs()).max().item()
    assert err < 3e-2 and (lse.cpu() - rl).abs().max().item() < 1e-2


def test_wide_latent_rows_bit_exact(gpu):
    """d_c 1792 (the per-row kernel rather than the multi-row one): the same bytes as the oracle."""
    import qmla
    n, d_c, width = 70, 1792, 1888
    g = torch.Generator().manual_seed(8)
    kv_c = (torch.randn(n, d_c, generator=g) * 4).to(torch.bfloat16)
    k_pe = torch.empty(n, ROPE + H, dtype=torch.bfloat16)
    k_pe[:, :ROPE] = (torch.randn(n, ROPE, generator=g) * 4).to(torch.bfloat16)
    k_pe[:, ROPE:] = torch.exp(torch.randn(n, H, generator=g)).to(torch.bfloat16)
    slots = torch.randperm(20 * 16, generator=g)[:n]
    cache = torch.full((20, 16, 1, width), 0xAB, dtype=torch.uint8, device=gpu)
    ks = torch.tensor(0.021, device=gpu)
    qmla.cache_write(kv_c.to(gpu), k_pe.to(gpu), cache, slots.to(gpu), rope_w=ROPE, rms_heads=H, kv_fp8=True,
                     rms="log8", k_scale=ks)
    torch.cuda.synchronize()
    got = cache.cpu().view(-1, width).numpy()
    exp = ora.fp8_row_bytes(kv_c.float().numpy(), k_pe.float().numpy(), packed_rope=ROPE, n_heads=H, k_scale=0.021,
                            rms_mode=ora.RMS_LOG8)
    nb = exp.shape[1]
    assert np.array_equal(got[slots.numpy(), :nb], exp) and np.all(got[slots.numpy(), nb:] == 0xAB)


@pytest.mark.parametrize("rms,mode", [("log8", ora.RMS_LOG8), ("bf16", ora.RMS_BF16_BYTES), ("e4m3", ora.RMS_E4M3)])
@pytest.mark.parametrize("d_c,rope,heads", [(256, 232, 24), (768, 116, 12), (1792, 116, 12), (1792, 232, 24)])
def test_fp8_rows_deployed_layouts(gpu, d_c, rope, heads, rms, mode):
    """The plugin's deployed rows (tests/test_fp8_kv.py:105-120: rope 232 with 24 heads, 116 with 12;
    rope 116 leaves the rms tail at 4 mod 8): the same bytes as the oracle, nothing past the row."""
    import qmla
    n, P, pages = 200, 16, 20
    g = torch.Generator().manual_seed(d_c + rope + heads)
    kv_c = (torch.randn(n, d_c, generator=g) * 4.0).to(torch.bfloat16)
    k_pe = torch.empty(n, rope + heads, dtype=torch.bfloat16)
    k_pe[:, :rope] = (torch.randn(n, rope, generator=g) * 4.0).to(torch.bfloat16)
    k_pe[:, rope:] = torch.exp(torch.randn(n, heads, generator=g)).to(torch.bfloat16)
    rb = 2 if rms == "bf16" else 1
    width = d_c + rope + rb * heads
    width += (-width) % 16
    k_scale = 0.0217
    slots = torch.randperm(pages * P, generator=g)[:n]
    cache = torch.full((pages, P, 1, width), 0xAB, dtype=torch.uint8, device=gpu)
    qmla.cache_write(kv_c.to(gpu), k_pe.to(gpu), cache, slots.to(gpu), rope_w=rope, rms_heads=heads, kv_fp8=True,
                     rms=rms, k_scale=torch.tensor(k_scale, device=gpu))
    torch.cuda.synchronize()
    got = cache.cpu().view(pages * P, width).numpy()
    kc, kp = kv_c.float().numpy(), k_pe.float().numpy()
    if mode == ora.RMS_E4M3:
        inv = np.float32(1.0) / np.float32(k_scale)
        q = lambda x: ora.e4m3_encode(np.clip(x.astype(np.float32) * inv, -448.0, 448.0))
        exp = np.concatenate([q(kc), q(kp[:, :rope]), q(kp[:, rope:])], axis=1)
    else:
        exp = ora.fp8_row_bytes(kc, kp, packed_rope=rope, n_heads=heads, k_scale=k_scale, rms_mode=mode)
    nb = exp.shape[1]
    s = slots.numpy()
    bad = [(i, np.nonzero(got[s[i], :nb] != exp[i])[0][:6]) for i in range(n) if not np.array_equal(got[s[i], :nb], exp[i])]
    assert not bad, bad[:3]
    assert np.all(got[s, nb:] == 0xAB)
    assert np.all(np.delete(got, s, axis=0) == 0xAB)
