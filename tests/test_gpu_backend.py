"""forward_mqa end to end on the GPU against the oracle: a SimpleNamespace attn_metadata / impl /
layer carrying the attributes the reference's decode reads, the vLLM 3-D cache, the absorbed query
as one tensor [B, H, rank + declared rope] (zeros past the packed rope, as the model writes it,
qwen3_5_mla.py:289-292) or as the (q_nope, q_pe) tuple, and spec-verify steps whose metadata goes
through build_decode's flattening first."""
from types import SimpleNamespace

import pytest
import torch

from qmla.backend import DecodeMetadataBuilder, QwenMLAHipImpl
from tests.mla_cases import check_decode, make_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kv,heads,qtok,tuple_q", [("bf16", 24, 1, False), ("fp8", 24, 1, True),
                                                  ("fp8", 8, 4, False), ("bf16", 24, 4, True)])
def test_forward_mqa(gpu, monkeypatch, kv, heads, qtok, tuple_q):
    monkeypatch.setenv("QWEN_MLA_FP8_RMS", "log8")
    lens = [3, 900, 2500, 64, 1]
    c = make_case(batch=len(lens), heads=heads, d_c=512, rope_w=64, page_size=64, lens=lens, kv=kv,
                  rms_mode="bf16" if kv == "bf16" else "log8", seed=91 + heads + qtok, device=gpu, qrows=qtok,
                  rms="spread", amp=2.0)
    rows = c.q_nope.shape[0]
    declared = 64 + heads + (-(64 + heads)) % 8
    q = torch.zeros(rows, heads, 512 + declared, dtype=torch.bfloat16, device=gpu)
    q[..., :512] = c.q_nope
    q[..., 512:576] = c.q_pe
    impl = QwenMLAHipImpl(kv_lora_rank=512, scale=c.sm_scale, need_to_return_lse_for_decode=True)
    impl.rms_offset, impl.mla_local_heads, impl.mla_kv_fp8 = 576, heads, kv == "fp8"
    impl.mla_rope_dim, impl.mla_rope_group, impl.mla_packed_rope = 64, 6, 64
    layer = SimpleNamespace(_k_scale=c.k_scale)
    # the request-level metadata vLLM hands the builder, then its flattening
    n = len(lens)
    bt_req = c.block_table.view(n, qtok, -1)[:, 0].contiguous()
    sl_req = torch.tensor(lens, dtype=torch.int32, device=gpu)
    md = DecodeMetadataBuilder(max_rows=64).build_decode(bt_req, sl_req, rows)
    assert torch.equal(md.seq_lens, c.seq_lens) and torch.equal(md.block_table, c.block_table)
    attn_metadata = SimpleNamespace(causal=True, num_decode_tokens=rows, decode=md)
    cache3 = c.cache[:, :, 0, :]                                   # vLLM's [num_blocks, block_size, head_size]
    impl.reserve_decode_workspace(rows, gpu, qrows=qtok)
    qa = (q[..., :512], q[..., 512:]) if tuple_q else q
    o, lse = impl.forward_mqa(qa, cache3, attn_metadata, layer)
    torch.cuda.synchronize()
    assert o.shape == (rows, heads, 512) and o.dtype == torch.bfloat16 and lse is not None
    check_decode(f"forward_mqa {kv} h{heads} q{qtok} tuple={tuple_q}", c, o, lse)
    impl.need_to_return_lse_for_decode = False
    o2, lse2 = impl.forward_mqa(qa, cache3, attn_metadata, layer)
    torch.cuda.synchronize()
    assert lse2 is None and torch.equal(o2.view(torch.int16), o.view(torch.int16))
