"""The balanced plan (qmla_plan) on its own, bit for bit: per-request exclusive prefix sums of
64-token tile counts (plus the switch cost qmla_plan_switch_tiles reports for a non-empty request),
the total and the per-workgroup chunk, against numpy. Batch sizes straddle the
kernel's 1024-request batches; with verify rows the last row of a request carries its length. The
plan stands in for FlashInfer's work-split plan (qwen_mla/fi_decode.py:210-233).
"""
import numpy as np
import pytest
import torch

from tests.mla_cases import make_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_req,qrows,nwg", [(1, 1, 256), (128, 1, 256), (255, 1, 7), (1024, 1, 256), (1025, 1, 33),
                                             (1000, 4, 256), (2049, 1, 1)])
def test_plan_prefix_sums(gpu, n_req, qrows, nwg):
    from qmla import _lib
    from qmla.decode import _stream, build_params, workspace_bytes
    c = make_case(batch=n_req, heads=24, d_c=512, rope_w=64, page_size=64, lens=[1] * n_req, kv="bf16",
                  rms_mode="bf16", seed=9, device=gpu, qrows=qrows)
    g = np.random.default_rng(n_req)
    L = g.integers(0, 70000, n_req)
    L[::7] = 0
    rows = np.repeat(L, qrows) - np.tile(np.arange(qrows)[::-1], n_req)
    sl = torch.tensor(np.maximum(rows, 0), dtype=torch.int32, device=gpu)
    o = torch.empty(n_req * qrows, 24, 512, dtype=torch.bfloat16, device=gpu)
    args = dict(q_nope=c.q_nope, q_pe=c.q_pe, kv_cache=c.cache, block_table=c.block_table, seq_lens=sl, out=o,
                lse=None, d_c=512, rope_w=64, rms_offset=c.rms_offset, rms_mode=_lib.RMS_BF16, kv=_lib.KV_BF16,
                page_size=64, sm_scale=c.sm_scale, qrows=qrows, num_splits=0, num_workgroups=nwg)
    ws = torch.full((workspace_bytes(build_params(**args)) // 4,), -7, dtype=torch.int32, device=gpu)
    p = build_params(workspace=ws, **args)
    _lib.check("qmla_plan", _lib.lib().qmla_plan(p, _stream()))
    torch.cuda.synchronize()
    got = ws[:n_req + 3].cpu().numpy()
    sw = _lib.lib().qmla_plan_switch_tiles(p)
    assert sw >= 0
    tiles = (L + 63) // 64 + sw * (L > 0)
    total = int(tiles.sum())
    exp = np.concatenate([[max(-(-total // nwg), 1), total], np.cumsum(tiles) - tiles, [total]])
    print(f"[plan n_req {n_req} qrows {qrows} nwg {nwg}] total {total} tiles (switch {sw})", flush=True)
    assert np.array_equal(got, exp), np.argwhere(got != exp)[:5].ravel().tolist()


@pytest.mark.parametrize("kv,rms,d_c,n_req,nwg", [("fp8", "log8", 512, 300, 256), ("fp8", "log8", 512, 300, 7),
                                                 ("bf16", "bf16", 512, 300, 64), ("bf16", "bf16", 1792, 90, 33)])
def test_decode_kernels_store_the_plan(gpu, kv, rms, d_c, n_req, nwg):
    """The decode kernels derive the balanced plan themselves; the first workgroup stores it for the
    combine: the same words qmla_plan writes (warp-specialized, per-group and column-split kernels)."""
    from qmla import _lib
    from qmla.decode import _stream, build_params, workspace_bytes
    g = np.random.default_rng(n_req + nwg)
    L = g.integers(0, 3000, n_req)
    L[::5] = 0
    c = make_case(batch=n_req, heads=24, d_c=d_c, rope_w=64, page_size=64, lens=L.tolist(), kv=kv, rms_mode=rms,
                  seed=10, device=gpu)
    o = torch.empty(n_req, 24, d_c, dtype=torch.bfloat16, device=gpu)
    lse = torch.empty(n_req, 24, dtype=torch.float32, device=gpu)
    args = dict(q_nope=c.q_nope, q_pe=c.q_pe, kv_cache=c.cache, block_table=c.block_table, seq_lens=c.seq_lens, out=o,
                lse=lse, d_c=d_c, rope_w=64, rms_offset=c.rms_offset,
                rms_mode=_lib.RMS_LOG8 if kv == "fp8" else _lib.RMS_BF16, kv=_lib.KV_FP8 if kv == "fp8" else _lib.KV_BF16,
                page_size=64, sm_scale=c.sm_scale, k_scale=c.k_scale, num_splits=0, num_workgroups=nwg)
    ws = torch.full((workspace_bytes(build_params(**args)) // 4,), -7, dtype=torch.int32, device=gpu)
    p = build_params(workspace=ws, **args)
    _lib.check("qmla_decode_partial", _lib.lib().qmla_decode_partial(p, _stream()))
    torch.cuda.synchronize()
    got = ws[:n_req + 3].cpu().numpy()
    sw = _lib.lib().qmla_plan_switch_tiles(p)
    assert sw >= 0
    tiles = (L + 63) // 64 + sw * (L > 0)
    total = int(tiles.sum())
    exp = np.concatenate([[max(-(-total // nwg), 1), total], np.cumsum(tiles) - tiles, [total]])
    assert np.array_equal(got, exp), np.argwhere(got != exp)[:5].ravel().tolist()
