"""Spec-verify folding on every cache format and deployed layout: a request's query tokens x heads
decode as one kernel request (its cache rows read once, or once per pair of tokens on the rank-1792
instances), with the rows split over up to four workgroups that read the token range together. The
reference folds groups of up to 64 rows (ops/mla_decode_attention.py:1291-1310): 2 tokens at 24
heads. Each family is checked against the float32 oracle through both entry points, in the balanced
and the fixed-split mode, with requests shorter than the verify window (early rows see no token).
"""
import pytest
import torch

from tests.mla_cases import check_decode, make_case

pytestmark = pytest.mark.gpu

# (kv, rms, d_c, heads, rope, fold of 4 tokens)
FAMILIES = [
    ("bf16", "bf16", 512, 24, 64, 4),          # per-group kernel, 96 rows over 3 workgroups
    ("fp8", "e4m3", 512, 24, 64, 4),
    ("fp8", "bf16_bytes", 512, 24, 64, 4),
    ("fp8", "log8", 768, 24, 232, 4),          # the plugin's deployed rows: rope 232 (TP 1)
    ("fp8", "e4m3", 256, 24, 232, 4),
    ("fp8", "log8", 768, 12, 116, 4),          # ... rope 116, 12 heads (TP 2): 48 rows
    ("bf16", "bf16", 768, 24, 232, 4),         # column-split kernel, 32 rows per workgroup
    ("bf16", "bf16", 1792, 24, 64, 2),         # column-split kernel, 16 rows per workgroup
    ("fp8", "log8", 1792, 24, 232, 4),         # column-split kernel, 16-token tiles of 32 rows
    ("bf16", "bf16", 1792, 24, 232, 4),        # column-split kernel, 32 rows per workgroup
]
QTOK = 4
LENS = [3, 1, 900, 2500, 64, 1700]


def _case(gpu, fam, seed):
    kv, rms, d_c, heads, rope, _ = fam
    return make_case(batch=len(LENS), heads=heads, d_c=d_c, rope_w=rope, page_size=64, lens=LENS, kv=kv,
                     rms_mode=rms, seed=seed, device=gpu, qrows=QTOK, rms="spread", amp=2.0)


def _fp8_kw(c):
    return dict(kv_fp8=True, fp8_rms={"bf16_bytes": "bf16"}.get(c.rms_mode, c.rms_mode), k_scale=c.k_scale) \
        if c.kv == "fp8" else {}


@pytest.mark.parametrize("splits", [0, 3])
@pytest.mark.parametrize("fam", FAMILIES, ids=lambda f: f"{f[0]}-{f[1]}-{f[2]}-h{f[3]}-r{f[4]}")
def test_forward_folds_verify_rows(gpu, fam, splits):
    import qmla
    from qmla import _lib
    from qmla.decode import build_params, fold_rows
    c = _case(gpu, fam, seed=700 + fam[2] + fam[3] + fam[4] + splits)
    mode = {"bf16": _lib.RMS_BF16, "log8": _lib.RMS_LOG8, "bf16_bytes": _lib.RMS_BF16_BYTES,
            "e4m3": _lib.RMS_E4M3}[c.rms_mode]
    probe = build_params(q_nope=c.q_nope, q_pe=c.q_pe, kv_cache=c.cache, block_table=c.block_table,
                         seq_lens=c.seq_lens, out=c.q_nope, lse=None, d_c=c.d_c, rope_w=c.rope_w,
                         rms_offset=c.rms_offset, rms_mode=mode, kv=_lib.KV_FP8 if c.kv == "fp8" else _lib.KV_BF16,
                         page_size=c.page_size, sm_scale=c.sm_scale)
    fold = fold_rows(probe, QTOK)
    print(f"[fold {fam} splits {splits}] {QTOK} tokens fold {fold}", flush=True)
    assert fold == fam[5]
    o, lse = qmla.forward(c.q_nope, c.q_pe, c.cache, c.block_table, c.seq_lens, d_c=c.d_c, rope_w=c.rope_w,
                          rms_offset=c.rms_offset, page_size=c.page_size, sm_scale=c.sm_scale, qrows=QTOK,
                          num_splits=splits, **_fp8_kw(c))
    torch.cuda.synchronize()
    check_decode(f"fold {fam} splits {splits}", c, o, lse, num_splits=max(splits, 1))


@pytest.mark.parametrize("fam", [FAMILIES[0], FAMILIES[1], FAMILIES[3], FAMILIES[7]],
                         ids=lambda f: f"{f[0]}-{f[1]}-{f[2]}-h{f[3]}-r{f[4]}")
def test_reference_entry_folds_verify_rows(gpu, fam):
    """decode_attention_fwd(..., qrows=4): the reference's entry with its attn_logits partials."""
    import qmla
    c = _case(gpu, fam, seed=900 + fam[2] + fam[3])
    rows, H, dc, rope = c.q_nope.shape[0], c.heads, c.d_c, c.rope_w
    q = torch.zeros(rows, H, c.row, dtype=torch.bfloat16, device=gpu)   # [latent | rope | tail]
    q[..., :dc] = c.q_nope
    q[..., dc:dc + rope] = c.q_pe
    q[..., dc + rope:] = 7.0          # tail columns must be ignored (Lk = rms_offset)
    cache = c.cache
    o = torch.full((rows, H, dc), float("nan"), dtype=torch.bfloat16, device=gpu)
    lse = torch.zeros(rows, H, dtype=torch.float32, device=gpu)
    splits = 8
    logits = torch.zeros(rows, H, splits, dc + 1, dtype=torch.float32, device=gpu)
    kw = {}
    if c.kv == "fp8":
        cache = cache.view(torch.float8_e4m3fn)
        kw = dict(k_scale=c.k_scale, v_scale=c.k_scale, rms_bf16=c.rms_mode == "bf16_bytes",
                  rms_log8=c.rms_mode == "log8")
    qmla.decode_attention_fwd(q, cache, cache[..., :dc], o, lse, c.block_table, c.seq_lens, logits, splits,
                              c.sm_scale, c.page_size, is_mla=True, rms_offset=c.rms_offset, qrows=QTOK, **kw)
    torch.cuda.synchronize()
    check_decode(f"reference entry fold {fam}", c, o, lse, num_splits=splits)
