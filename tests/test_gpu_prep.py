"""GPU parity of the fused decode q / k_pe prep (qmla_prep) against the oracle's restatement of
qwen_mla/qwen3_5_mla.py:262-301: the copied and rotated query elements, the q_pe slot layout and the
k_pe rope window and padding are bit-exact (the rotation is bf16 arithmetic with every product and
sum rounded, as the reference's torch ops do); the rms is within one bf16 step of the oracle's
float64-accumulated value (the up-projection GEMM accumulates in fp32 here, as the reference's bf16
GEMM does on its tensor cores, so its bf16 outputs may differ from the float64 ones in the last
place), and almost always equal.
"""
import numpy as np
import pytest
import torch

from tests.mla_cases import ora

pytestmark = pytest.mark.gpu

THETA = 1e7


def _bits(x: torch.Tensor) -> np.ndarray:
    return x.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _obits(x: np.ndarray) -> np.ndarray:
    return ora.f32_to_bf16_bits(x)


def _run(gpu, *, n, H, hd, rd, kv, group, d_c, head_offset, rope_first, span, declared, keep=None,
         table_dtype=torch.bfloat16, mrope=False, max_pos=8192, seed=0, bad_pos=None, strided_q=True):
    import qmla
    g = torch.Generator().manual_seed(seed)
    nope = hd - rd
    qg = torch.randn(n, H, 2 * hd, generator=g).to(torch.bfloat16)
    q = qg[..., :hd] if strided_q else qg[..., :hd].contiguous()          # a chunk view, as the module has
    lat = torch.randn(n, d_c, generator=g).to(torch.bfloat16)
    kr = (torch.randn(n, kv * rd, generator=g) * 1.5).to(torch.bfloat16)
    ku = (torch.randn(H * nope, d_c, generator=g) * d_c ** -0.5).to(torch.bfloat16)
    w = (torch.randn(hd, generator=g) * 0.1).to(torch.bfloat16)
    keep = keep if keep is not None else list(range(rd // 2))
    tab32 = ora.partial_rope_table(keep, 2 * len(keep) if keep == list(range(rd // 2)) else 64, THETA, max_pos)
    tab = torch.from_numpy(tab32).to(table_dtype)
    sec = None
    if mrope:
        pos = torch.randint(0, max_pos, (3, n), generator=g)
        sec = torch.tensor([(1 if (f % 3 == 1 and f < 33) else (2 if (f % 3 == 2 and f < 30) else 0)) for f in keep],
                           dtype=torch.int32)
    else:
        pos = torch.randint(0, max_pos, (n,), generator=g)
    if bad_pos is not None:
        pos[..., bad_pos] = max_pos + 5
    q_out, k_pe = qmla.mla_decode_prep(
        pos.to(gpu), q.to(gpu), lat.to(gpu), kr.to(gpu), ku.to(gpu), qmla.k_gain(w.to(gpu), rd), tab.to(gpu),
        head_offset=head_offset, rope_group=group, rope_first=rope_first, rope_span=span, declared_rope=declared,
        eps=1e-6, rope_sec=None if sec is None else sec.to(gpu))
    torch.cuda.synchronize()
    ok = np.ones(n, bool)
    if bad_pos is not None:
        ok[bad_pos] = False
    posn = pos.numpy().copy()
    posn[..., ~ok] = 0
    eq, ek, erms = ora.mla_decode_prep(q.float().numpy()[ok], lat.float().numpy()[ok],
                                       kr.float().numpy().reshape(n, kv, rd)[ok], ku.float().numpy(),
                                       w.float().numpy(), tab.float().numpy(), posn[..., ok],
                                       head_offset=head_offset, rope_group=group, rope_first=rope_first,
                                       rope_span=span, declared_rope=declared, eps=1e-6,
                                       rope_sec=None if sec is None else sec.numpy())
    return _bits(q_out), _bits(k_pe), _obits(eq), _obits(ek), erms, ok, k_pe


def _check(gq, gk, eq, ek, erms, ok, H, span, rd):
    gq, gk = gq[ok], gk[ok]
    assert np.array_equal(gq, eq), np.argwhere(gq != eq)[:6]
    packed = span * rd
    assert np.array_equal(gk[:, :packed], ek[:, :packed]), np.argwhere(gk[:, :packed] != ek[:, :packed])[:6]
    assert np.array_equal(gk[:, packed + H:], ek[:, packed + H:])
    got = ora.bf16_bits_to_f32(gk[:, packed:packed + H]).astype(np.float64)
    ref = erms.astype(np.float64)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7), np.max(np.abs(got - ref) / ref)
    same = np.mean(gk[:, packed:packed + H] == ek[:, packed:packed + H])
    assert same > 0.97, same


@pytest.mark.parametrize("n", [128, 1, 37, 200])
def test_full_rope_single_rank(gpu, n):
    """24 heads of 256 (rope 64 first), 4 rope groups of 6 heads, d_c 512, bf16 table."""
    r = _run(gpu, n=n, H=24, hd=256, rd=64, kv=4, group=6, d_c=512, head_offset=0, rope_first=0, span=4,
             declared=296, seed=n)
    _check(*r[:6], H=24, span=4, rd=64)


def test_partial_rope_second_rank_fp32_table(gpu):
    """Rank 1 of 2: global heads 12..23, rope 58 (29 kept subspaces), groups 2-3 cached, tail 140."""
    keep = [i for i in range(32) if i not in (29, 30, 31)]
    r = _run(gpu, n=77, H=12, hd=256, rd=58, kv=4, group=6, d_c=768, head_offset=12, rope_first=2, span=2,
             declared=140, keep=keep, table_dtype=torch.float32, seed=11)
    _check(*r[:6], H=12, span=2, rd=58)


def test_mrope_positions_fp16_table(gpu):
    keep = [i for i in range(32) if i not in (29, 30, 31)]
    r = _run(gpu, n=45, H=24, hd=256, rd=58, kv=4, group=6, d_c=512, head_offset=0, rope_first=0, span=4,
             declared=256, keep=keep, table_dtype=torch.float16, mrope=True, seed=12)
    _check(*r[:6], H=24, span=4, rd=58)


@pytest.mark.parametrize("d_c", [256, 1792])
def test_latent_widths(gpu, d_c):
    r = _run(gpu, n=64, H=24, hd=256, rd=64, kv=4, group=6, d_c=d_c, head_offset=0, rope_first=0, span=4,
             declared=296, seed=d_c, strided_q=False)
    _check(*r[:6], H=24, span=4, rd=64)


def test_position_outside_the_table_gives_nan(gpu):
    r = _run(gpu, n=40, H=24, hd=256, rd=64, kv=4, group=6, d_c=512, head_offset=0, rope_first=0, span=4,
             declared=296, seed=13, bad_pos=7, max_pos=2048)
    gq, gk, eq, ek, erms, ok, k_pe = r
    _check(gq, gk, eq, ek, erms, ok, H=24, span=4, rd=64)
    assert torch.isnan(k_pe[7, :256].float()).all() and not torch.isnan(k_pe[7, 256:].float()).any()
