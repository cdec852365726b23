"""GLA-g2 (two latent groups of 256 columns, 12 heads per group, fp8 + log8) on the warp-specialized
decode, against the CPU oracle (tolerances of tests/test_gpu_ws.py): fixed splits, 1, 2 and 4 verify
tokens (12 / 24 / 48 rows per group), pages that change inside a tile, hundreds of short and empty
requests over two workgroups (several planning windows), and long requests split into many pieces.
The reference runs GLA as its TP = 2 rank-local decode (mla_impl.py:628-662 for the verify rows).
"""
import pytest
import torch

from tests.mla_cases import make_case
from tests.test_gpu_ws import _check

pytestmark = pytest.mark.gpu


def _case(gpu, lens, qrows=4, page_size=64, seed=50):
    return make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=page_size, lens=lens, kv="fp8",
                     rms_mode="log8", seed=seed, device=gpu, qrows=qrows, groups=2, rms="spread", amp=4.0)


def _forward(c, **kw):
    import qmla
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, d_c=c.d_c, page_size=c.page_size,
                          sm_scale=c.sm_scale, kv_fp8=True, fp8_rms="log8", k_scale=c.k_scale, qrows=c.qrows,
                          groups=2, **kw)
    torch.cuda.synchronize()
    return o, lse


def test_gla_fixed_splits(gpu):
    c = _case(gpu, [1, 900, 4097, 2500, 33], seed=51)
    o, lse = _forward(c, num_splits=8)
    _check("gla fixed 8 splits", c, o, lse)


@pytest.mark.parametrize("qrows", [1, 2])
def test_gla_verify_tokens(gpu, qrows):
    c = _case(gpu, [2, 777, 3001, 64, 1500], qrows=qrows, seed=52 + qrows)
    o, lse = _forward(c, num_workgroups=5)
    _check(f"gla q{qrows}", c, o, lse)


@pytest.mark.parametrize("page_size", [16, 1])
def test_gla_small_pages(gpu, page_size):
    c = _case(gpu, [5, 333, 1200], page_size=page_size, seed=55)
    o, lse = _forward(c, num_workgroups=4)
    _check(f"gla pages of {page_size}", c, o, lse)


def test_gla_many_short_requests(gpu):
    g = torch.Generator().manual_seed(56)
    lens = [int(x) for x in torch.randint(0, 90, (200,), generator=g)]
    lens[::13] = [0] * len(lens[::13])
    c = _case(gpu, lens, seed=56)
    o, lse = _forward(c, num_workgroups=2)
    _check("gla 200 short requests, 2 workgroups", c, o, lse)


def test_gla_long_requests(gpu):
    c = _case(gpu, [40000, 31001], seed=57)
    o, lse = _forward(c, num_workgroups=64)
    _check("gla 2 long requests over 64 workgroups", c, o, lse)


# GLA-g2 on the cache formats of the per-group kernel (fp8 rows with e4m3 or bf16-byte rms, bf16 rows
# with bf16 rms): 48 rows per group with 4 verify tokens, 12 with one
GLA_FORMATS = [("fp8", "e4m3"), ("fp8", "bf16_bytes"), ("bf16", "bf16")]


@pytest.mark.parametrize("kv,rms_mode", GLA_FORMATS)
@pytest.mark.parametrize("qrows,splits", [(4, 0), (4, 5), (1, 0)])
def test_gla_other_formats(gpu, kv, rms_mode, qrows, splits):
    import qmla
    lens = [1, 900, 4097, 2500, 33, 0] if splits == 0 else [1, 900, 4097, 2500, 33]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv=kv,
                  rms_mode=rms_mode, seed=60 + qrows + splits, device=gpu, qrows=qrows, groups=2, rms="spread",
                  amp=4.0 if kv == "fp8" else 1.0)
    fp8_rms = {"e4m3": "e4m3", "bf16_bytes": "bf16"}.get(rms_mode, "log8")
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, d_c=c.d_c, page_size=c.page_size,
                          sm_scale=c.sm_scale, kv_fp8=kv == "fp8", fp8_rms=fp8_rms, k_scale=c.k_scale,
                          qrows=qrows, groups=2, num_splits=splits, num_workgroups=0 if splits else 6)
    torch.cuda.synchronize()
    _check(f"gla {kv}/{rms_mode} q{qrows} splits {splits}", c, o, lse)


@pytest.mark.parametrize("sm_scale", [-0.05, 0.0])
def test_gla_sign_of_the_scale(gpu, sm_scale):
    """A negative or zero softmax scale (the reference takes any float): the row-owner kernel folds
    its sign into the query parts."""
    c = _case(gpu, [700, 33, 2049], seed=70)
    c.sm_scale = sm_scale
    o, lse = _forward(c, num_workgroups=4)
    _check(f"gla sm_scale {sm_scale}", c, o, lse)


@pytest.mark.parametrize("qrows", [4, 1])
@pytest.mark.parametrize("where", ["latent", "rope", "both"])
def test_gla_query_outlier_channels(gpu, where, qrows):
    """The row-owner kernel's query split (e4m3 hi + lo parts of q * 2^e per row, the row's 2^-e as
    the MFMA's B scale, the rope's hi and lo parts sharing one MFMA) on query rows whose elements span
    more than 2^10: a few outlier channels per row (x 1024 over the rest), as the reference's FP8 test
    draws outlier latent channels (tests/test_fp8_kv.py:23-31). 4 verify tokens take the quad-shared
    rms instance, 1 token the other one."""
    lens = [700, 3000, 64, 1500, 5]
    c = _case(gpu, lens, qrows=qrows, seed=81 + qrows)
    g = torch.Generator(device="cpu").manual_seed(82)
    rows = c.q_nope.shape[0]
    qn = torch.randn(rows, 24, 256, generator=g) * 0.02
    qp = torch.randn(rows, 24, 64, generator=g) * 0.02
    for r in range(rows):
        for h in range(24):
            # outliers of magnitude 24 against a median |q| of about 0.0135
            if where in ("latent", "both"):
                qn[r, h, torch.randperm(256, generator=g)[:3]] = 24.0 * torch.sign(torch.randn(3, generator=g))
            if where in ("rope", "both"):
                qp[r, h, torch.randperm(64, generator=g)[:2]] = 24.0 * torch.sign(torch.randn(2, generator=g))
    c.q_nope = qn.to(torch.bfloat16).to(gpu)
    c.q_pe = qp.to(torch.bfloat16).to(gpu)
    amax = torch.cat([qn, qp], -1).abs().amax(-1)
    amin = torch.cat([qn, qp], -1).abs().clamp_min(1e-30).median(-1).values
    assert (amax / amin).min() > 2 ** 10
    o, lse = _forward(c, num_workgroups=7)
    _check(f"gla q{qrows} query outliers in {where}", c, o, lse)
