"""GPU parity of the FP8 + log8 decode shapes served by the warp-specialized kernel (d_c 512, rope 64,
one latent group, at most 32 query rows per request) against the CPU oracle: verify rows read
per-row rms codes, pages that tiles straddle, and a context whose score maximum keeps climbing, so
that the softmax reference moves at many tiles (reference: ops/mla_decode_attention.py:297-586).

Bound: tests.mla_cases.check_decode (plain max-abs 3e-2 for an fp8 cache against the float32
oracle, or C_REF times the reference roundings' own error where that is larger), lse 1e-2.
"""
import pytest
import torch

from tests.mla_cases import check_decode, make_case

pytestmark = pytest.mark.gpu


def _check(name, c, o, lse):
    check_decode(name, c, o, lse)


def _forward(c, **kw):
    import qmla
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, page_size=c.page_size,
                          sm_scale=c.sm_scale, kv_fp8=True, fp8_rms="log8", k_scale=c.k_scale, qrows=c.qrows, **kw)
    torch.cuda.synchronize()
    return o, lse


@pytest.mark.parametrize("qrows,heads", [(4, 8), (2, 16)])
def test_ws_verify_rows(gpu, qrows, heads):
    """Causal verify rows (row j of a request sees L - (qrows-1-j) tokens), rms codes per row."""
    lens = [3, 700, 64, 2049, 130]
    c = make_case(batch=len(lens), heads=heads, d_c=512, rope_w=64, page_size=64, lens=lens, kv="fp8",
                  rms_mode="log8", seed=11, device=gpu, qrows=qrows, rms="spread")
    o, lse = _forward(c, num_workgroups=7)
    _check(f"verify q{qrows} h{heads}", c, o, lse)


@pytest.mark.parametrize("page_size", [40, 16, 1])
def test_ws_straddling_pages(gpu, page_size):
    """Page sizes that are not multiples of the 32-token tile: tiles gather rows from several pages."""
    lens = [1000, 77, 333] if page_size > 1 else [300, 45]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=page_size, lens=lens, kv="fp8",
                  rms_mode="log8", seed=12, device=gpu, rms="spread")
    o, lse = _forward(c, num_workgroups=4)
    _check(f"pages P={page_size}", c, o, lse)


def test_ws_climbing_max(gpu):
    """rms codes fall from 255 to 0 along each request, so the divisor shrinks 64x and the score
    maximum climbs through the whole context: the reference max moves at many tiles."""
    lens = [4096, 1500, 5000]
    P = 64
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=P, lens=lens, kv="fp8",
                  rms_mode="log8", seed=13, device=gpu, rms="spread", q_amp=3.0)
    cb = c.cache.view(torch.uint8).view(c.cache.shape[0], P, -1)
    bt = c.block_table.cpu()
    for b, L in enumerate(lens):
        t = torch.arange(L)
        code = (255 - torch.round(255.0 * t.float() / max(L - 1, 1))).to(torch.uint8)
        pages = bt[b, t // P].long()
        slots = t % P
        cb[pages.to(gpu), slots.to(gpu), c.rms_offset:c.rms_offset + 24] = code.to(gpu)[:, None]
    o, lse = _forward(c, num_workgroups=6)
    _check("climbing max", c, o, lse)
    # the same through fixed splits
    o2, lse2 = _forward(c, num_splits=5)
    _check("climbing max, 5 splits", c, o2, lse2)


@pytest.mark.parametrize("nwg", [1, 2, 3, 4, 5, 7])
@pytest.mark.parametrize("lens", [[0, 0, 64, 0, 0, 128, 0, 64, 0, 0], [0, 0, 0], [5, 0, 0, 0, 70, 0], [0, 200, 0, 1]])
def test_ws_empty_requests_at_range_edges(gpu, lens, nwg):
    """Requests of length 0 before, between and after the others, at the plan positions where the
    workgroups' ranges start and end, and a batch with no token at all: every row is written (zero
    output, lse -inf for the empty ones; outputs start as NaN), whichever workgroup owns it."""
    import qmla
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv="fp8", rms_mode="log8",
                  seed=17, device=gpu, rms="spread", amp=2.0)
    rows = c.q_nope.shape[0]
    o = torch.full((rows, 24, 512), float("nan"), dtype=torch.bfloat16, device=gpu)
    lse = torch.full((rows, 24), float("nan"), dtype=torch.float32, device=gpu)
    _forward(c, num_workgroups=nwg, out=o, lse=lse)
    assert not torch.isnan(o.float()).any() and not torch.isnan(lse).any(), "unwritten rows"
    _check(f"empty requests {lens} nwg {nwg}", c, o, lse)


@pytest.mark.parametrize("heads,qrows,nwg,splits", [(24, 4, 0, 0), (24, 4, 5, 0), (24, 4, 16, 0), (24, 4, 0, 3),
                                                    (24, 2, 0, 0), (16, 4, 0, 0), (24, 3, 0, 0)])
def test_ws_head_split_verify(gpu, heads, qrows, nwg, splits):
    """More verify rows than one workgroup holds (24 heads x 4 tokens = 96): the request's heads are
    split over workgroups that read the same token range (8 heads x 4 tokens each), in the balanced
    mode (default ranges on shared XCDs, a caller's range count, 16 ranges) and with fixed splits;
    2 tokens x 24 heads and 4 x 16 split in two; 3 tokens x 24 heads in three splits of 24 rows."""
    import qmla
    lens = [4, 1500, 3000, 64, 777]
    c = make_case(batch=len(lens), heads=heads, d_c=512, rope_w=64, page_size=64, lens=lens, kv="fp8",
                  rms_mode="log8", seed=41 + qrows + heads, device=gpu, qrows=qrows, rms="spread", amp=2.0)
    rows = c.q_nope.shape[0]
    o = torch.full((rows, heads, 512), float("nan"), dtype=torch.bfloat16, device=gpu)
    lse = torch.full((rows, heads), float("nan"), dtype=torch.float32, device=gpu)
    _forward(c, num_workgroups=nwg, num_splits=splits, out=o, lse=lse)
    assert not torch.isnan(o.float()).any() and not torch.isnan(lse).any(), "unwritten rows"
    _check(f"head split {heads}x{qrows} nwg {nwg} S={splits}", c, o, lse)


@pytest.mark.parametrize("where", ["latent", "rope", "both"])
def test_ws_query_outlier_channels(gpu, where):
    """Query rows whose elements span more than 2^10: a few outlier channels per row (x 1024 over the
    rest), as the reference's FP8 test draws outlier latent channels (tests/test_fp8_kv.py:23-31). The
    fp8 score path splits the bf16 query into two e4m3 parts scaled to the row maximum, so the small
    elements lose low bits to e4m3 subnormals; the output stays within the parity bound."""
    lens = [700, 3000, 64, 1500]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv="fp8",
                  rms_mode="log8", seed=77, device=gpu, rms="spread", amp=4.0)
    g = torch.Generator(device="cpu").manual_seed(78)
    rows = c.q_nope.shape[0]
    qn = torch.randn(rows, 24, 512, generator=g) * 0.02
    qp = torch.randn(rows, 24, 64, generator=g) * 0.02
    for r in range(rows):
        for h in range(24):
            # outliers of magnitude 24 against a median |q| of about 0.0135
            if where in ("latent", "both"):
                qn[r, h, torch.randperm(512, generator=g)[:4]] = 24.0 * torch.sign(torch.randn(4, generator=g))
            if where in ("rope", "both"):
                qp[r, h, torch.randperm(64, generator=g)[:2]] = 24.0 * torch.sign(torch.randn(2, generator=g))
    c.q_nope = qn.to(torch.bfloat16).to(gpu)
    c.q_pe = qp.to(torch.bfloat16).to(gpu)
    amax = torch.cat([qn, qp], -1).abs().amax(-1)
    amin = torch.cat([qn, qp], -1).abs().clamp_min(1e-30).median(-1).values
    assert (amax / amin).min() > 2 ** 10
    o, lse = _forward(c, num_workgroups=9)
    _check(f"query outliers in {where}", c, o, lse)
