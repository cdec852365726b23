"""GPU parity: the HIP decode against the CPU oracle on the same seeded inputs.

Bound (tests.mla_cases.check_decode): plain max-abs 1e-2 for a bf16 cache and 3e-2 for an fp8
cache against the float32 oracle, or, where the reference kernel's own roundings already exceed
that on the same inputs, C_REF times their error; LSE (natural log) within 1e-2.
"""
import pytest
import torch

from tests.mla_cases import check_decode, check_partials, make_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kv,rms_mode", [("bf16", "bf16"), ("fp8", "log8"), ("fp8", "bf16_bytes"), ("fp8", "e4m3")])
def test_forward_balanced(gpu, kv, rms_mode):
    import qmla
    lens = [1, 63, 64, 65, 700, 2047, 3000, 129]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv=kv,
                  rms_mode=rms_mode, seed=5, device=gpu, rms="spread", amp=2.0 if kv == "fp8" else 1.0)
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, page_size=c.page_size,
                          sm_scale=c.sm_scale, kv_fp8=kv == "fp8", fp8_rms={"log8": "log8", "bf16_bytes": "bf16",
                                                                          "e4m3": "e4m3", "bf16": "log8"}[rms_mode],
                          k_scale=c.k_scale, num_workgroups=5)
    torch.cuda.synchronize()
    check_decode(f"balanced {kv}/{rms_mode}", c, o, lse)


@pytest.mark.parametrize("splits", [1, 3, 8])
@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_reference_surface(gpu, kv, splits):
    """decode_attention_fwd: q = [latent | rope | tail], attn_logits partials, in-place outputs."""
    import qmla
    lens = [900, 77, 1600, 513]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv=kv, seed=7,
                  device=gpu, rms="spread")
    B, H = c.q_nope.shape[:2]
    q = torch.zeros(B, H, c.row - 0, dtype=torch.bfloat16, device=gpu)
    q[..., :512] = c.q_nope
    q[..., 512:576] = c.q_pe
    q[..., 576:] = 7.0          # tail columns must be ignored (Lk = rms_offset)
    o = torch.full((B, H, 512), float("nan"), dtype=torch.bfloat16, device=gpu)
    lse = torch.zeros(B, H, dtype=torch.float32, device=gpu)
    logits = torch.full((B, H, splits, 513), float("nan"), dtype=torch.float32, device=gpu)
    cache = c.cache if kv == "bf16" else c.cache.view(torch.float8_e4m3fn)
    qmla.decode_attention_fwd(q, cache, cache[..., :512], o, lse, c.block_table, c.seq_lens, logits, splits,
                              c.sm_scale, c.page_size, k_scale=c.k_scale, is_mla=True, rms_offset=576,
                              rms_log8=kv == "fp8")
    torch.cuda.synchronize()
    check_decode(f"ref-surface {kv} S={splits}", c, o, lse, num_splits=splits)
    if splits > 1:
        # the partials follow the reference bounds and layout exactly
        check_partials(f"ref-surface {kv} S={splits}", c, logits, num_splits=splits, align=16)


def test_small_pages_config1(gpu):
    """B=4, ctx 2048, 16-token pages with a random-permutation block table, bf16 (config 1 shape)."""
    import qmla
    c = make_case(batch=4, heads=24, d_c=512, rope_w=64, page_size=16, lens=[2048] * 4, kv="bf16", seed=0,
                  device=gpu)
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, page_size=16,
                          sm_scale=c.sm_scale, num_workgroups=7)
    torch.cuda.synchronize()
    check_decode("config1 P16", c, o, lse)


def test_gla_verify(gpu):
    """GLA-g2 (2 x 256 latent, 12 heads per group) with 4-token causal verify rows, fp8 + log8."""
    import qmla
    lens = [300, 1000, 64, 2100, 5]
    c = make_case(batch=len(lens), heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv="fp8",
                  rms_mode="log8", seed=4, device=gpu, qrows=4, groups=2, rms="spread")
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, d_c=512, page_size=64,
                          sm_scale=c.sm_scale, kv_fp8=True, fp8_rms="log8", k_scale=c.k_scale, qrows=4,
                          groups=2, num_workgroups=6)
    torch.cuda.synchronize()
    check_decode("gla-g2 verify", c, o, lse)


@pytest.mark.parametrize("kv,rms,d_c,qrows", [("fp8", "log8", 512, 1), ("fp8", "e4m3", 512, 1), ("bf16", "bf16", 512, 4),
                                              ("bf16", "bf16", 1792, 1)])
def test_single_split_empty_requests(gpu, kv, rms, d_c, qrows):
    """One split (final rows written by the decode kernel itself, no combine): requests of length 0
    still get a zero output and -inf lse, as every combine writes them. Outputs start as NaN."""
    import qmla
    lens = [0, 700, 0, 3, 1]
    c = make_case(batch=len(lens), heads=24, d_c=d_c, rope_w=64, page_size=64, lens=lens, kv=kv, rms_mode=rms,
                  seed=61, device=gpu, qrows=qrows, rms="spread")
    rows = c.q_nope.shape[0]
    o = torch.full((rows, 24, d_c), float("nan"), dtype=torch.bfloat16, device=gpu)
    lse = torch.full((rows, 24), float("nan"), dtype=torch.float32, device=gpu)
    kw = dict(kv_fp8=True, fp8_rms=rms, k_scale=c.k_scale) if kv == "fp8" else {}
    qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, page_size=64, sm_scale=c.sm_scale, qrows=qrows,
                 num_splits=1, out=o, lse=lse, **kw)
    torch.cuda.synchronize()
    assert not torch.isnan(o.float()).any() and not torch.isnan(lse).any(), "unwritten rows"
    check_decode(f"one split {kv} {rms} d_c {d_c} q{qrows}", c, o, lse)
