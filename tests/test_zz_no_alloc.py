"""qmla_decode_static: the decode with its split-K scratch in the library's own per-GPU array
instead of a caller workspace. Through the C ABI, its outputs equal qmla_decode's on the same
parameters (bit for bit: same kernels, same launch shapes), on two calls in a row with the second
on a smaller input, in the balanced and the fixed-split modes; a call whose scratch would exceed
QMLA_STATIC_SCRATCH_BYTES is refused before any device work."""
import ctypes

import pytest
import torch

from qmla import _lib
from qmla.decode import Workspace, build_params, workspace_bytes
from tests.mla_cases import check_decode, make_case, lognormal_lens


def _params(c, out, lse, splits, ws=None):
    mode = {"log8": _lib.RMS_LOG8, "bf16": _lib.RMS_BF16}[c.rms_mode]
    a = dict(q_nope=c.q_nope, q_pe=c.q_pe, kv_cache=c.cache, block_table=c.block_table, seq_lens=c.seq_lens,
             out=out, lse=lse, d_c=c.d_c, rope_w=c.rope_w, rms_offset=c.rms_offset, rms_mode=mode,
             kv=_lib.KV_FP8 if c.kv == "fp8" else _lib.KV_BF16, page_size=c.page_size, sm_scale=c.sm_scale,
             k_scale=c.k_scale, qrows=c.qrows, groups=c.groups, num_splits=splits,
             split_align=16 if splits else 0)
    if ws is not None:
        a["workspace"] = ws
        if splits:
            a["ws_strides"] = (ws.stride(0), ws.stride(1), ws.stride(2))
    return build_params(**a)


def _run_both(gpu, c, splits):
    lib = _lib.lib()
    st = torch.cuda.current_stream().cuda_stream
    rows, H = c.q_nope.shape[:2]
    dv = c.d_c // c.groups
    outs = []
    for entry in ("qmla_decode", "qmla_decode_static"):
        o = torch.full((rows, H, dv), float("nan"), dtype=torch.bfloat16, device=gpu)
        lse = torch.full((rows, H), float("nan"), dtype=torch.float32, device=gpu)
        if entry == "qmla_decode":
            if splits:
                ws = torch.empty(rows, H, splits, dv + 1, dtype=torch.float32, device=gpu)
            else:
                ws = Workspace().reserve(workspace_bytes(_params(c, o, lse, 0)), gpu)
            p = _params(c, o, lse, splits, ws)
        else:
            p = _params(c, o, lse, splits)          # no workspace: the library's scratch
        rc = getattr(lib, entry)(ctypes.byref(p), st)
        assert rc == 0, (entry, rc)
        torch.cuda.synchronize()
        outs.append((o, lse))
    return outs


@pytest.mark.gpu
@pytest.mark.parametrize("splits", [0, 4])
def test_static_scratch_matches_workspace_entry(gpu, splits):
    for step, (batch, seed) in enumerate([(48, 81), (5, 82)]):          # second call: a smaller input
        lens = lognormal_lens(batch, 6000, 0.6, 1, 30000, seed=seed)
        c = make_case(batch=batch, heads=24, d_c=512, rope_w=64, page_size=64, lens=lens, kv="fp8", rms_mode="log8",
                      seed=seed, device=gpu, amp=4.0)
        (o1, l1), (o2, l2) = _run_both(gpu, c, splits)
        print(f"[static scratch S={splits} call {step}] B={batch} tokens={c.tokens()}", flush=True)
        assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), "outputs differ from qmla_decode"
        assert torch.equal(l1, l2), "lse differs from qmla_decode"
        if step == 1:
            check_decode(f"static scratch S={splits}", c, o2, l2, num_splits=max(splits, 1))


def test_static_scratch_refuses_oversize():
    """The fixed-split partials of 32 x 24 heads x 16 splits x 1793 floats (88 MB) exceed the
    64 MiB array: refused with QMLA_ERR_WORKSPACE before any device work (fake pointers)."""
    p = _lib.DecodeParams()
    base = 0x10000
    p.q_nope, p.q_nope_stride_row, p.q_nope_stride_head = base, 24 * 1792, 1792
    p.q_pe, p.q_pe_stride_row, p.q_pe_stride_head = base + 0x1000000, 24 * 64, 64
    p.kv_cache, p.page_stride, p.token_stride = base + 0x2000000, 1600 * 1888, 1888
    p.kv_dtype, p.page_size, p.d_c, p.rope_w = _lib.KV_BF16, 1600, 1792, 64
    p.rms_offset, p.rms_mode, p.sm_scale = 1856, _lib.RMS_BF16, 0.02
    p.block_table, p.bt_stride, p.seq_lens = base + 0x3000000, 64, base + 0x4000000
    p.rows, p.heads, p.rms_heads, p.qrows, p.groups = 32, 24, 24, 1, 1
    p.out, p.out_stride_row, p.out_stride_head, p.out_dtype = base + 0x5000000, 24 * 1792, 1792, _lib.DT_BF16
    p.num_splits, p.split_align = 16, 16
    assert 32 * 24 * 16 * 1793 * 4 > _lib.STATIC_SCRATCH_BYTES
    assert _lib.lib().qmla_decode_static(ctypes.byref(p), None) == _lib.ERR_WORKSPACE
