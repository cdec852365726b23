"""The C entry points recorded into a HIP graph (torch.cuda.CUDAGraph capture of the library calls
made with prebuilt parameters): every replay equals an eager call on the same inputs, bit for bit,
with eager work and input changes between the replays. Covers the balanced decode (plan, decode,
combine: three launches, no memsets), the fixed-split decode, the cache-row writer and the prep.
"""
import ctypes
import math

import pytest
import torch

from tests.mla_cases import make_case

pytestmark = pytest.mark.gpu


def _capture(fn):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()                       # one eager call on the capture stream first
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


@pytest.mark.parametrize("splits", [0, 4])
def test_decode_replays_match_eager(gpu, splits):
    import qmla
    from qmla import _lib
    from qmla.decode import Workspace, build_params, workspace_bytes
    c = make_case(batch=6, heads=24, d_c=512, rope_w=64, page_size=64, lens=[3000, 64, 1, 777, 5000, 130], kv="fp8",
                  rms_mode="log8", seed=31, device=gpu, amp=4.0)
    rows = c.q_nope.shape[0]
    out = torch.empty(rows, 24, 512, dtype=torch.bfloat16, device=gpu)
    lse = torch.empty(rows, 24, dtype=torch.float32, device=gpu)
    a = dict(q_nope=c.q_nope, q_pe=c.q_pe, kv_cache=c.cache, block_table=c.block_table, seq_lens=c.seq_lens, out=out,
             lse=lse, d_c=512, rope_w=64, rms_offset=c.rms_offset, rms_mode=_lib.RMS_LOG8, kv=_lib.KV_FP8, page_size=64,
             sm_scale=c.sm_scale, k_scale=c.k_scale, qrows=1, groups=1, num_splits=splits, split_align=16 if splits else 0)
    if splits:
        logits = torch.empty(rows, 24, splits, 513, dtype=torch.float32, device=gpu)
        p = build_params(workspace=logits, ws_strides=(logits.stride(0), logits.stride(1), logits.stride(2)), **a)
    else:
        ws = Workspace().reserve(workspace_bytes(build_params(**a)), gpu)
        p = build_params(workspace=ws, **a)
    lib = qmla.lib()

    def call():
        rc = lib.qmla_decode(p, torch.cuda.current_stream().cuda_stream)
        assert rc == 0, rc

    g = _capture(call)
    for rep in range(3):
        c.q_nope.mul_(-1.0 if rep % 2 == 0 else 0.5)      # new inputs at the same addresses
        out.fill_(7.0)
        lse.fill_(7.0)
        call()
        torch.cuda.synchronize()
        eo, el = out.clone(), lse.clone()
        out.fill_(-3.0)
        lse.fill_(-3.0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eo) and torch.equal(lse, el), rep


def test_writer_and_prep_replays_match_eager(gpu):
    import qmla
    from qmla.cache import cache_write_params
    from qmla.prep import prep_params
    from tests.mla_cases import ora
    lib = qmla.lib()
    g0 = torch.Generator().manual_seed(5)
    n = 96
    kv_c = (torch.randn(n, 512, generator=g0) * 3).to(torch.bfloat16).to(gpu)
    k_pe = torch.exp(torch.randn(n, 88, generator=g0)).to(torch.bfloat16).to(gpu)
    slots = torch.randperm(40 * 64, generator=g0)[:n].to(gpu)
    cache = torch.zeros(40, 64, 1, 608, dtype=torch.uint8, device=gpu)
    ks = torch.tensor(0.02, device=gpu)
    pw, keep_w = cache_write_params(kv_c, k_pe, cache, slots, rope_w=64, rms_heads=24, kv_fp8=True, rms="log8",
                                    k_scale=ks)
    H, hd, rd = 24, 256, 64
    q = torch.randn(n, H, hd, generator=g0).to(torch.bfloat16).to(gpu)
    kr = torch.randn(n, 4 * rd, generator=g0).to(torch.bfloat16).to(gpu)
    ku = (torch.randn(H * (hd - rd), 512, generator=g0) * 0.04).to(torch.bfloat16).to(gpu)
    gain = qmla.k_gain((torch.randn(hd, generator=g0) * 0.1).to(torch.bfloat16).to(gpu), rd)
    tab = torch.from_numpy(ora.partial_rope_table(list(range(32)), 64, 1e7, 4096)).to(torch.bfloat16).to(gpu)
    pos = torch.randint(0, 4096, (n,), generator=g0).to(gpu)
    pp, keep_p, q_out, k_out = prep_params(pos, q, kv_c, kr, ku, gain, tab, head_offset=0, rope_group=6, rope_first=0,
                                           rope_span=4, declared_rope=296, eps=1e-6)

    def call():
        st = torch.cuda.current_stream().cuda_stream
        assert lib.qmla_cache_write(ctypes.byref(pw), st) == 0
        assert lib.qmla_prep(ctypes.byref(pp), st) == 0

    g = _capture(call)
    for rep in range(3):
        kv_c.mul_(-1.0)
        q.mul_(0.5 if rep else -1.0)
        cache.fill_(0xAB)          # the writer leaves unwritten slots alone: same start for both runs
        call()
        torch.cuda.synchronize()
        ec, eq, ek = cache.clone(), q_out.clone(), k_out.clone()
        cache.fill_(0xAB)
        q_out.fill_(9.0)
        k_out.fill_(9.0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(cache, ec) and torch.equal(q_out, eq) and torch.equal(k_out, ek), rep
    assert math.isfinite(float(q_out.float().abs().max()))
