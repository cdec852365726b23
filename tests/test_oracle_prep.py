"""Pins the oracle's restatement of the decode q / k_pe prep (qwen_mla/qwen3_5_mla.py:232-301,
:341-354; qwen_mla/partial_rope.py:52-76) with checks a plausible mistake would fail:

* the partial-rope table keeps each subspace's ORIGINAL frequency: its columns equal the matching
  columns of the full-width table (the property partial_rope.py:61-65 states), and its entries are
  cos/sin of t * theta^(-2k/64) in float64 up to the float32 angle;
* the bf16 rotation equals torch's bf16 arithmetic of the same expression bit for bit, is the
  identity at position 0, and is within bf16 rounding of the exact float64 rotation;
* M-RoPE with equal position rows equals the 1-D rotation bit for bit, and with distinct rows
  every frequency follows its own section's position (float64 brute force);
* the rms, by float64 brute-force loops, and its closed form when k_up selects latent columns;
* the group slot of each head under a second tensor-parallel rank (global head 12 belongs to group
  2, qwen3_5_mla.py:286-288), the k_pe window, rms position and zero padding.
"""
import math

import numpy as np
import torch

from tests.mla_cases import ora

THETA = 1e7


def _bf16(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).float().numpy()


def test_partial_table_keeps_original_frequencies():
    full = ora.partial_rope_table(list(range(32)), 64, THETA, 512)
    keep = [i for i in range(32) if i not in (29, 30, 31)]
    part = ora.partial_rope_table(keep, 64, THETA, 512)
    assert part.shape == (512, 58)
    assert np.array_equal(part[:, :29], full[:, keep]) and np.array_equal(part[:, 29:], full[:, [32 + k for k in keep]])
    t = np.arange(512, dtype=np.float64)[:, None]
    ang = t * THETA ** (-2.0 * np.asarray(keep, np.float64) / 64)
    # the float32 angle carries a relative error of 2^-23 at most (two roundings)
    tol = np.abs(ang) * 2.0 ** -22 + 1e-7
    assert np.all(np.abs(part[:, :29] - np.cos(ang)) <= tol) and np.all(np.abs(part[:, 29:] - np.sin(ang)) <= tol)
    assert np.array_equal(full[0], np.concatenate([np.ones(32), np.zeros(32)]).astype(np.float32))


def test_rotation_matches_torch_bf16_arithmetic():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(200, 5, 64, generator=g) * 3).to(torch.bfloat16)
    ang = torch.rand(200, 1, 32, generator=g, dtype=torch.float64) * 1000
    cos, sin = ang.cos().float(), ang.sin().float()
    got = ora.neox_rotate_bf16(x.float().numpy(), cos.numpy(), sin.numpy())
    cb, sb = cos.to(torch.bfloat16), sin.to(torch.bfloat16)
    x1, x2 = x[..., :32], x[..., 32:]
    ref = torch.cat([x1 * cb - x2 * sb, x2 * cb + x1 * sb], dim=-1).float().numpy()   # bf16 tensor ops
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_rotation_identity_at_zero_and_close_to_exact():
    g = np.random.default_rng(1)
    x = _bf16(g.standard_normal((64, 3, 58)) * 2)
    tab = ora.partial_rope_table([i for i in range(29)], 64, THETA, 4096)
    c0, s0 = ora.rope_rows(tab, np.zeros(64, np.int64))
    assert np.array_equal(ora.neox_rotate_bf16(x, c0[:, None], s0[:, None]), x)
    pos = g.integers(0, 4096, 64)
    c, s = ora.rope_rows(tab, pos)
    got = ora.neox_rotate_bf16(x, c[:, None], s[:, None]).astype(np.float64)
    ang = pos[:, None].astype(np.float64) * THETA ** (-2.0 * np.arange(29) / 64)
    C, S = np.cos(ang)[:, None], np.sin(ang)[:, None]
    x1, x2 = x[..., :29].astype(np.float64), x[..., 29:].astype(np.float64)
    exact = np.concatenate([x1 * C - x2 * S, x2 * C + x1 * S], axis=-1)
    scale = np.abs(x1) + np.abs(x2)
    scale = np.concatenate([scale, scale], axis=-1)
    assert np.all(np.abs(got - exact) <= scale * 2.0 ** -6 + 1e-30)   # three bf16 roundings + table
    assert np.allclose((got ** 2).sum(-1), (x.astype(np.float64) ** 2).sum(-1), rtol=2e-2)


def test_mrope_rows():
    g = np.random.default_rng(2)
    keep = [i for i in range(32) if i not in (29, 30, 31)]
    tab = ora.partial_rope_table(keep, 64, THETA, 4096)
    sec_of = lambda f: 1 if (f % 3 == 1 and f < 33) else (2 if (f % 3 == 2 and f < 30) else 0)
    sec = np.array([sec_of(f) for f in keep])
    p = g.integers(0, 4096, 37)
    c1, s1 = ora.rope_rows(tab, p)
    c3, s3 = ora.rope_rows(tab, np.stack([p, p, p]), sec)
    assert np.array_equal(c1, c3) and np.array_equal(s1, s3)
    p3 = g.integers(0, 4096, (3, 37))
    c, s = ora.rope_rows(tab, p3, sec)
    for t in range(37):
        for i, f in enumerate(keep):
            a = np.float64(np.float32(np.float32(p3[sec_of(f), t]) * np.float32(THETA ** (-2.0 * f / 64))))
            assert abs(c[t, i] - math.cos(a)) < 1e-6 and abs(s[t, i] - math.sin(a)) < 1e-6


def _case(n=5, H=4, hd=32, rd=8, kv=2, rope_group=2, d_c=16, seed=3):
    g = np.random.default_rng(seed)
    q = _bf16(g.standard_normal((n, H, hd)))
    lat = _bf16(g.standard_normal((n, d_c)))
    kr = _bf16(g.standard_normal((n, kv, rd)))
    ku = _bf16(g.standard_normal((H * (hd - rd), d_c)) * 0.3)
    w = _bf16(g.standard_normal(hd) * 0.1)
    tab = ora.partial_rope_table(list(range(rd // 2)), rd, THETA, 64)
    pos = g.integers(0, 64, n)
    return q, lat, kr, ku, w, tab, pos


def test_rms_brute_force():
    q, lat, kr, ku, w, tab, pos = _case()
    n, H, hd = q.shape
    rd, nope = 8, 24
    _, k_pe, rms = ora.mla_decode_prep(q, lat, kr, ku, w, tab, pos, head_offset=0, rope_group=2, rope_first=0,
                                       rope_span=2, declared_rope=2 * rd + H + 4, eps=1e-6)
    for t in range(n):
        for h in range(H):
            s = 0.0
            for j in range(nope):
                dot = sum(float(lat[t, k]) * float(ku[h * nope + j, k]) for k in range(lat.shape[1]))
                v = float(_bf16(np.float32(dot)))
                s += v * v
            s += sum(float(kr[t, h // 2, i]) ** 2 for i in range(rd))
            assert abs(rms[t, h] - math.sqrt(s / hd + 1e-6)) <= 1e-6 * math.sqrt(s / hd)
            assert k_pe[t, 2 * rd + h] == _bf16(rms[t, h])


def test_rms_selection_closed_form():
    """k_up rows that pick single latent columns: k_nope is the latent itself, exactly."""
    q, lat, kr, ku, w, tab, pos = _case(n=3, H=2, hd=20, rd=4, kv=1, rope_group=2, d_c=32)
    nope = 16
    ku = np.zeros((2 * nope, 32), np.float32)
    for h in range(2):
        for j in range(nope):
            ku[h * nope + j, (h * nope + j) % 32] = 1.0
    _, _, rms = ora.mla_decode_prep(q, lat, kr, ku, w, tab, pos, head_offset=0, rope_group=2, rope_first=0,
                                    rope_span=1, declared_rope=4 + 2, eps=0.0)
    for h in range(2):
        sel = lat[:, h * nope:(h + 1) * nope].astype(np.float64)
        exp = np.sqrt(((sel ** 2).sum(-1) + (kr[:, 0].astype(np.float64) ** 2).sum(-1)) / 20)
        assert np.allclose(rms[:, h], exp, rtol=1e-6)


def test_second_rank_slots_window_and_padding():
    """24 heads in 4 rope groups of 6, split over two ranks: rank 1 holds global heads 12..23, so its
    local head 0 reads group 2 (slot 0) and local head 6 group 3 (slot rd); k_pe caches groups 2, 3."""
    g = np.random.default_rng(4)
    n, H, hd, rd, d_c = 3, 12, 256, 58, 128
    q = _bf16(g.standard_normal((n, H, hd)))
    lat = _bf16(g.standard_normal((n, d_c)))
    kr = _bf16(g.standard_normal((n, 4, rd)))
    ku = _bf16(g.standard_normal((H * (hd - rd), d_c)) * 0.1)
    w = _bf16(g.standard_normal(hd) * 0.1)
    keep = [i for i in range(32) if i not in (29, 30, 31)]
    tab = ora.partial_rope_table(keep, 64, THETA, 1000)
    pos = g.integers(0, 1000, n)
    declared = 140                                         # 2*58 rope + 12 rms + 12 padding
    q_out, k_pe, rms = ora.mla_decode_prep(q, lat, kr, ku, w, tab, pos, head_offset=12, rope_group=6,
                                           rope_first=2, rope_span=2, declared_rope=declared, eps=1e-6)
    nope = hd - rd
    c, s = ora.rope_rows(tab, pos)
    for h, slot in ((0, 0), (5, 0), (6, rd), (11, rd)):
        rot = ora.neox_rotate_bf16(q[:, h, :rd], c, s)
        assert np.array_equal(q_out[:, h, nope + slot:nope + slot + rd], rot)
        other = np.ones(declared, bool)
        other[slot:slot + rd] = False
        assert np.all(q_out[:, h, nope:][:, other] == 0)
        assert np.array_equal(q_out[:, h, :nope], q[:, h, rd:])
    gain = (1 + w)[:rd]
    for gi, grp in enumerate((2, 3)):
        kin = _bf16(kr[:, grp] * gain)
        assert np.array_equal(k_pe[:, gi * rd:(gi + 1) * rd], ora.neox_rotate_bf16(kin, c, s))
    assert np.array_equal(k_pe[:, 2 * rd:2 * rd + H], _bf16(rms))
    assert np.all(k_pe[:, 2 * rd + H:] == 0)
