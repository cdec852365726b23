"""The backend adapter without a GPU: the verify flattening of build_decode bit for bit against the
oracle (persistent buffers reused, padding rows clamped to 0), the C parameter block forward_mqa
builds from a SimpleNamespace metadata / impl / layer carrying exactly the attributes the reference
reads (no launch), and the backend triple."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import mla_oracle as ora
from qmla import _lib
from qmla.backend import DecodeMetadataBuilder, QwenMLAHipBackend, QwenMLAHipImpl, decode_params


@pytest.mark.parametrize("q", [1, 2, 4])
def test_build_decode_matches_oracle(q):
    g = torch.Generator().manual_seed(q)
    n, width = 7, 11
    bt = torch.randint(0, 1000, (n, width), generator=g, dtype=torch.int32)
    sl = torch.tensor([0, 1, 2, 3, 17, 4096, q], dtype=torch.int32)   # 0: a graph padding request
    b = DecodeMetadataBuilder(max_rows=64)
    md = b.build_decode(bt, sl, n * q)
    ebt, esl = ora.flatten_verify(bt.numpy(), sl.numpy(), q)
    assert md._mla_q == q
    assert np.array_equal(md.block_table.numpy(), ebt) and md.block_table.dtype == torch.int32
    assert np.array_equal(md.seq_lens.numpy(), esl) and md.seq_lens.dtype == torch.int32
    if q > 1:
        ptrs = (md.block_table.data_ptr(), md.seq_lens.data_ptr())
        md2 = b.build_decode(bt.flip(0).contiguous(), sl.flip(0).contiguous(), n * q)   # next step: same buffers
        assert (md2.block_table.data_ptr(), md2.seq_lens.data_ptr()) == ptrs
        ebt2, esl2 = ora.flatten_verify(bt.flip(0).numpy(), sl.flip(0).numpy(), q)
        assert np.array_equal(md2.block_table.numpy(), ebt2) and np.array_equal(md2.seq_lens.numpy(), esl2)


def test_build_decode_rejects_ragged_token_counts():
    with pytest.raises(ValueError):
        DecodeMetadataBuilder().build_decode(torch.zeros(3, 4, dtype=torch.int32), torch.ones(3, dtype=torch.int32), 7)


def _impl(fp8=False, lse=True):
    impl = QwenMLAHipImpl(kv_lora_rank=512, scale=1 / 576 ** 0.5, need_to_return_lse_for_decode=lse)
    impl.rms_offset, impl.mla_local_heads, impl.mla_kv_fp8 = 576, 24, fp8
    impl.mla_rope_dim, impl.mla_rope_group, impl.mla_packed_rope = 64, 24, 64
    return impl


def _metadata(B, q=1, causal=True):
    dec = SimpleNamespace(seq_lens=torch.full((B,), 100, dtype=torch.int32),
                          block_table=torch.zeros(B, 4, dtype=torch.int32), _mla_q=q)
    return SimpleNamespace(causal=causal, num_decode_tokens=B, decode=dec)


@pytest.mark.parametrize("fp8,mode,code", [(False, "log8", _lib.RMS_BF16), (True, "log8", _lib.RMS_LOG8),
                                            (True, "bf16", _lib.RMS_BF16_BYTES), (True, "e4m3", _lib.RMS_E4M3)])
def test_decode_params_from_metadata(monkeypatch, fp8, mode, code):
    monkeypatch.setenv("QWEN_MLA_FP8_RMS", mode)
    B, H = 8, 24
    q = torch.zeros(B, H, 512 + 96, dtype=torch.bfloat16)          # declared rope 96: slots, rms, pad
    # vLLM's 3-D MLA cache; FP8 rows with two-byte rms codes are 16 bytes wider (the kernel stages 624)
    width = 624 if fp8 and mode == "bf16" else 608
    cache = torch.zeros(10, 64, width, dtype=torch.uint8 if fp8 else torch.bfloat16)
    layer = SimpleNamespace(_k_scale=torch.tensor(0.5))
    out = torch.empty(B, H, 512, dtype=torch.bfloat16)
    lse = torch.empty(B, H)
    md = _metadata(B, q=4)
    impl = _impl(fp8)
    impl.mla_local_heads = H = 8                                  # 8 heads x 4 verify tokens fold into 32 rows
    q, out, lse = q[:, :H], out[:, :H], lse[:, :H]
    p = decode_params(impl, q, cache, md, layer, out, lse)
    assert p.q_nope == q.data_ptr() and p.q_pe == q.data_ptr() + 512 * 2
    assert (p.d_c, p.rope_w, p.rms_offset, p.rms_mode) == (512, 64, 576, code)
    assert p.kv_dtype == (_lib.KV_FP8 if fp8 else _lib.KV_BF16)
    assert p.qrows == 4 and p.rows == B and p.heads == H and p.page_size == 64
    assert (p.page_stride, p.token_stride) == (64 * width, width)
    assert (p.k_scale is not None) == fp8
    assert p.seq_lens == md.decode.seq_lens.data_ptr() and p.block_table == md.decode.block_table.data_ptr()
    # the tuple form reads the same memory without a copy
    p2 = decode_params(impl, (q[..., :512], q[..., 512:]), cache, md, layer, out, lse)
    assert (p2.q_nope, p2.q_pe, p2.q_pe_stride_row) == (p.q_nope, p.q_pe, p.q_pe_stride_row)
    # a non-causal decode keeps one kernel row per token; so does QWEN_MLA_GROUPED_VERIFY=0
    assert decode_params(impl, q, cache, _metadata(B, 4, causal=False), layer, out, lse).qrows == 1
    monkeypatch.setenv("QWEN_MLA_GROUPED_VERIFY", "0")
    assert decode_params(impl, q, cache, md, layer, out, lse).qrows == 1


def test_decode_params_checks_the_impl():
    impl = _impl()
    impl.rms_offset = -1
    q = torch.zeros(2, 24, 576, dtype=torch.bfloat16)
    cache = torch.zeros(4, 64, 1, 608, dtype=torch.bfloat16)
    out = torch.empty(2, 24, 512, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        decode_params(impl, q, cache, _metadata(2), SimpleNamespace(), out, None)
    impl = _impl()
    impl.mla_local_heads = 12                                       # rms slots of another head count
    with pytest.raises(ValueError):
        decode_params(impl, q, cache, _metadata(2), SimpleNamespace(), out, None)


def test_backend_triple():
    assert QwenMLAHipBackend.get_name() == "QWEN_MLA_TRITON"
    assert QwenMLAHipBackend.get_impl_cls() is QwenMLAHipImpl
    assert QwenMLAHipBackend.get_builder_cls() is DecodeMetadataBuilder
    assert hasattr(QwenMLAHipImpl, "forward_mqa") and hasattr(DecodeMetadataBuilder, "build_decode")


@pytest.mark.parametrize("fp8,mode,heads,row", [(True, "log8", 24, 608), (True, "log8", 8, 592), (True, "e4m3", 24, 608),
                                                 (False, "log8", 24, 600), (True, "log8", 24, 1024)])
@pytest.mark.parametrize("qtok", [1, 2, 4])
def test_reserved_workspace_covers_the_decode(monkeypatch, fp8, mode, heads, row, qtok):
    """reserve_decode_workspace sizes the buffer with the parameters forward_mqa builds (rms format,
    verify folding, the head split of a folded 24-head x 4-token step), whatever the reserve's own
    qrows: a spec-verify decode inside graph capture must find it large enough."""
    monkeypatch.setenv("QWEN_MLA_FP8_RMS", mode)
    impl = _impl(fp8)
    impl.mla_local_heads = heads
    B = 16 * qtok
    q = torch.zeros(B, heads, 512 + 96, dtype=torch.bfloat16)
    cache = torch.zeros(10, 64, row, dtype=torch.uint8 if fp8 else torch.bfloat16)
    out = torch.empty(B, heads, 512, dtype=torch.bfloat16)
    lse = torch.empty(B, heads)
    layer = SimpleNamespace(_k_scale=torch.tensor(0.5))
    need = _lib.lib().qmla_workspace_bytes(decode_params(impl, q, cache, _metadata(B, q=qtok), layer, out, lse))
    got = impl.reserve_decode_workspace(B, "cpu", qrows=4)      # up to 4 query tokens per request
    assert got >= need, (got, need)
    assert impl._workspace.buf.numel() >= need


def test_decode_attention_fwd_refuses_a_host_scale():
    """The kernels read k_scale through a device pointer: a Python float or a tensor of another dtype
    or device is refused rather than converted (a conversion allocates, which graph capture forbids)."""
    from qmla.decode import decode_attention_fwd
    B, H = 2, 24
    q = torch.zeros(B, H, 576, dtype=torch.bfloat16)
    cache = torch.zeros(4, 64, 1, 608, dtype=torch.uint8)
    o = torch.empty(B, H, 512, dtype=torch.bfloat16)
    lse = torch.empty(B, H)
    logits = torch.empty(B, H, 4, 513)
    args = (q, cache, cache[..., :512], o, lse, torch.zeros(B, 4, dtype=torch.int32), torch.ones(B, dtype=torch.int32),
            logits, 4, 0.1, 64)
    for ks in (0.5, torch.tensor(0.5, dtype=torch.float64)):
        with pytest.raises(TypeError, match="k_scale"):
            decode_attention_fwd(*args, k_scale=ks, is_mla=True, rms_offset=576, rms_log8=True)
