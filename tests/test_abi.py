"""The C ABI without a GPU: libqmla.so loads, exports every function include/qmla.h declares,
mirrors its struct, and rejects bad parameter blocks with the documented error codes before any
device work (fake, never dereferenced pointers)."""
from __future__ import annotations

import ctypes
import pathlib
import re

import pytest
import torch

import qmla
from qmla import _lib
from qmla.decode import build_params

HEADER = pathlib.Path(__file__).resolve().parent.parent / "include" / "qmla.h"


def _declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(qmla_\w+)\s*\(", text, flags=re.M)))


def test_header_functions_exported_and_bound():
    names = _declared_functions()
    assert "qmla_decode" in names and "qmla_cache_write" in names and "qmla_gather" in names and "qmla_prep" in names
    assert len(names) >= 10
    lib = _lib.lib()
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_version_and_constants_match_header():
    text = HEADER.read_text()
    consts = dict(re.findall(r"#define (QMLA_\w+) \(?(-?\d+)\)?", text))
    assert int(consts["QMLA_ABI_VERSION"]) == _lib.lib().qmla_version() == _lib.ABI_VERSION
    assert b"gfx950" in _lib.lib().qmla_build_info()
    for name, val in [("QMLA_ERR_NULL", _lib.ERR_NULL), ("QMLA_ERR_SHAPE", _lib.ERR_SHAPE),
                      ("QMLA_ERR_ALIGN", _lib.ERR_ALIGN), ("QMLA_ERR_WORKSPACE", _lib.ERR_WORKSPACE),
                      ("QMLA_ERR_MODE", _lib.ERR_MODE), ("QMLA_ERR_NOKERNEL", _lib.ERR_NOKERNEL),
                      ("QMLA_ERR_PAGE", _lib.ERR_PAGE),
                      ("QMLA_KV_FP8", _lib.KV_FP8), ("QMLA_RMS_LOG8", _lib.RMS_LOG8),
                      ("QMLA_RMS_E4M3", _lib.RMS_E4M3), ("QMLA_DT_F32", _lib.DT_F32)]:
        assert int(consts[name]) == val, name


def test_struct_mirror_matches_header_field_order():
    text = HEADER.read_text()
    body = text[text.index("typedef struct qmla_decode_params"):text.index("} qmla_decode_params;")]
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = []
    for decl in body.split("{", 1)[1].split(";"):
        decl = decl.strip()
        if not decl:
            continue
        names = [re.sub(r"[\*\s]", "", x).split()[-1] if x.strip() else "" for x in decl.split(",")]
        first = re.findall(r"(\w+)\s*$", decl.split(",")[0])[0]
        fields.append(first)
        fields.extend(n for n in names[1:])
    assert fields == [f[0] for f in _lib.DecodeParams._fields_]


def _valid_params(**over) -> _lib.DecodeParams:
    """A parameter block for H=24, d_c=512, rope 64, fp8 + log8, 608-byte rows, fake 16B-aligned pointers."""
    p = _lib.DecodeParams()
    base = 0x10000
    p.q_nope, p.q_nope_stride_row, p.q_nope_stride_head = base, 24 * 512, 512
    p.q_pe, p.q_pe_stride_row, p.q_pe_stride_head = base + 0x100000, 24 * 64, 64
    p.kv_cache, p.page_stride, p.token_stride = base + 0x200000, 64 * 608, 608
    p.kv_dtype, p.page_size, p.d_c, p.rope_w = _lib.KV_FP8, 64, 512, 64
    p.rms_offset, p.rms_mode = 576, _lib.RMS_LOG8
    p.sm_scale = 0.04
    p.block_table, p.bt_stride, p.seq_lens = base + 0x300000, 256, base + 0x400000
    p.rows, p.heads, p.rms_heads, p.qrows, p.groups = 8, 24, 24, 1, 1
    p.out, p.out_stride_row, p.out_stride_head, p.out_dtype = base + 0x500000, 24 * 512, 512, _lib.DT_BF16
    p.lse, p.lse_stride_row, p.lse_dtype = base + 0x600000, 24, _lib.DT_F32
    p.num_splits = 4
    p.workspace = base + 0x700000
    p.workspace_bytes = 1 << 30
    p.ws_stride_row, p.ws_stride_head, p.ws_stride_split = 24 * 4 * 513, 4 * 513, 513
    for k, v in over.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("over,code", [
    (dict(q_nope=None), _lib.ERR_NULL),
    (dict(kv_cache=None), _lib.ERR_NULL),
    (dict(q_pe=None), _lib.ERR_NULL),
    (dict(kv_dtype=7), _lib.ERR_MODE),
    (dict(rms_mode=_lib.RMS_BF16), _lib.ERR_MODE),          # bf16 rms element in an fp8 cache
    (dict(rms_offset=-1), _lib.ERR_MODE),                    # mode says rms, offset says none
    (dict(out_dtype=9), _lib.ERR_MODE),
    (dict(kv_cache=0x200008), _lib.ERR_ALIGN),               # 8-byte rows of a layout with no narrow-row kernel
    (dict(token_stride=600), _lib.ERR_ALIGN),
    (dict(kv_cache=0x200002), _lib.ERR_ALIGN),               # off 4-byte boundaries: no kernel at all
    (dict(token_stride=602), _lib.ERR_ALIGN),
    (dict(q_nope=0x100001), _lib.ERR_ALIGN),                 # queries need element alignment
    (dict(rows=9, qrows=2), _lib.ERR_SHAPE),
    (dict(heads=24, groups=5), _lib.ERR_SHAPE),
    (dict(token_stride=512, page_stride=64 * 512), _lib.ERR_SHAPE),   # row narrower than latent+rope
    (dict(d_c=384, rms_offset=448), _lib.ERR_NOKERNEL),
    (dict(workspace=None), _lib.ERR_WORKSPACE),
])
def test_error_codes(over, code):
    lib = _lib.lib()
    p = _valid_params(**over)
    assert lib.qmla_decode(ctypes.byref(p), None) == code
    if code != _lib.ERR_NOKERNEL and code != _lib.ERR_WORKSPACE:
        assert lib.qmla_decode_partial(ctypes.byref(p), None) == code
        assert lib.qmla_combine(ctypes.byref(p), None) == code


DENSE_WS = 8 * 24 * 4 * 513 * 4   # rows x heads x splits x (d_c + 1) floats of _valid_params


@pytest.mark.parametrize("over", [
    dict(workspace_bytes=DENSE_WS - 4),                        # smaller than qmla_workspace_bytes()
    dict(workspace_bytes=DENSE_WS, ws_stride_row=24 * 4 * 513 + 64),   # last partial past the end
    dict(workspace_bytes=DENSE_WS, ws_stride_head=4 * 513 + 1),
    dict(ws_stride_split=0),                                   # every stride must be positive
    dict(ws_stride_head=-513),
    dict(ws_stride_row=0),
])
def test_fixed_split_workspace_checked(over):
    """Fixed splits write attn_logits [rows, heads, S, d_c + 1] at the caller's strides: an undersized
    buffer or bad strides are rejected by every entry point before a launch."""
    lib = _lib.lib()
    p = _valid_params(**over)
    for fn in (lib.qmla_decode, lib.qmla_decode_partial, lib.qmla_combine):
        assert fn(ctypes.byref(p), None) == _lib.ERR_WORKSPACE, fn.__name__


def _layout(kv, d_c, rope, heads, rms, qrows=1, groups=1):
    """Parameter block for one cache layout (fake pointers). With 4 fixed splits and no workspace the
    entry returns ERR_WORKSPACE once it has an instance for the shape and ERR_NOKERNEL otherwise: the
    routing is checked without a launch."""
    eb = 1 if kv == _lib.KV_FP8 else 2
    rb = 2 if rms in (_lib.RMS_BF16, _lib.RMS_BF16_BYTES) else 0 if rms == _lib.RMS_NONE else 1
    row_bytes = d_c * eb + rope * eb + heads * rb
    row_bytes += (-row_bytes) % 16
    ts = row_bytes // eb
    dcg = d_c // groups
    return _valid_params(kv_dtype=kv, d_c=d_c, rope_w=rope, heads=heads, rms_heads=heads, rms_mode=rms,
                         rms_offset=-1 if rms == _lib.RMS_NONE else d_c + rope, token_stride=ts, page_stride=64 * ts, qrows=qrows, groups=groups,
                         rows=2 * qrows, q_nope_stride_row=heads * dcg, q_nope_stride_head=dcg,
                         q_pe_stride_row=heads * rope, q_pe_stride_head=rope, out_stride_row=heads * dcg,
                         out_stride_head=dcg, workspace=None, num_splits=4)


@pytest.mark.parametrize("kv,d_c,rope,heads,rms,qrows,groups,code", [
    # the plugin's deployed FP8 layouts at rank 1792 (column-split kernel, padded rope windows)
    (_lib.KV_FP8, 1792, 232, 24, _lib.RMS_LOG8, 1, 1, _lib.ERR_WORKSPACE),
    (_lib.KV_FP8, 1792, 232, 24, _lib.RMS_BF16_BYTES, 1, 1, _lib.ERR_WORKSPACE),
    (_lib.KV_FP8, 1792, 116, 12, _lib.RMS_E4M3, 1, 1, _lib.ERR_WORKSPACE),
    (_lib.KV_FP8, 1792, 64, 24, _lib.RMS_LOG8, 1, 1, _lib.ERR_WORKSPACE),
    # bf16 rank 768 with a 256-column window; bf16 rank 1792 with the reference test's partial and
    # full rope layouts (tests/test_two_pass_1792.py:12)
    (_lib.KV_BF16, 768, 232, 24, _lib.RMS_BF16, 1, 1, _lib.ERR_WORKSPACE),
    (_lib.KV_BF16, 1792, 232, 24, _lib.RMS_BF16, 1, 1, _lib.ERR_WORKSPACE),
    (_lib.KV_BF16, 1792, 116, 12, _lib.RMS_BF16, 1, 1, _lib.ERR_WORKSPACE),
    (_lib.KV_BF16, 1792, 256, 24, _lib.RMS_BF16, 1, 1, _lib.ERR_WORKSPACE),
    (_lib.KV_BF16, 1792, 256, 12, _lib.RMS_BF16, 1, 1, _lib.ERR_WORKSPACE),
    (_lib.KV_BF16, 1792, 300, 24, _lib.RMS_BF16, 1, 1, _lib.ERR_NOKERNEL),      # wider than any window
    # 24 heads x 4 verify tokens, FP8 + log8: the heads split over three workgroups per range
    (_lib.KV_FP8, 512, 64, 24, _lib.RMS_LOG8, 4, 1, _lib.ERR_WORKSPACE),
    # other rms formats: the per-group kernel splits the 96 rows over three workgroups per range
    (_lib.KV_FP8, 512, 64, 24, _lib.RMS_E4M3, 4, 1, _lib.ERR_WORKSPACE),
    # GLA-g2 with 4 verify tokens: FP8 + log8 (warp-specialized), FP8 + e4m3 / bf16-byte rms and
    # bf16 rows (per-group kernel); no instance without an rms tail
    (_lib.KV_FP8, 512, 64, 24, _lib.RMS_LOG8, 4, 2, _lib.ERR_WORKSPACE),
    (_lib.KV_FP8, 512, 64, 24, _lib.RMS_E4M3, 4, 2, _lib.ERR_WORKSPACE),
    (_lib.KV_FP8, 512, 64, 24, _lib.RMS_BF16_BYTES, 4, 2, _lib.ERR_WORKSPACE),
    (_lib.KV_BF16, 512, 64, 24, _lib.RMS_BF16, 4, 2, _lib.ERR_WORKSPACE),
    (_lib.KV_BF16, 512, 64, 24, _lib.RMS_NONE, 4, 2, _lib.ERR_NOKERNEL),
])
def test_routing_without_launch(kv, d_c, rope, heads, rms, qrows, groups, code):
    lib = _lib.lib()
    p = _layout(kv, d_c, rope, heads, rms, qrows, groups)
    assert lib.qmla_decode(ctypes.byref(p), None) == code


@pytest.mark.parametrize("kv,rms,qrows,groups,splits,tiles", [
    (_lib.KV_FP8, _lib.RMS_LOG8, 1, 1, 0, 2),     # warp-specialized decode, balanced
    (_lib.KV_FP8, _lib.RMS_LOG8, 4, 2, 0, 2),     # row-owner GLA-g2 decode, balanced
    (_lib.KV_BF16, _lib.RMS_BF16, 1, 1, 0, 2),    # bf16 warp-specialized decode, balanced
    (_lib.KV_FP8, _lib.RMS_E4M3, 1, 1, 0, 0),     # per-group kernel
    (_lib.KV_FP8, _lib.RMS_LOG8, 1, 1, 4, 0),     # fixed splits: no plan
])
def test_plan_switch_tiles(kv, rms, qrows, groups, splits, tiles):
    """The balanced plan's per-request switch charge follows the kernel the params select."""
    p = _layout(kv, 512, 64, 24, rms, qrows, groups)
    p.num_splits = splits
    assert _lib.lib().qmla_plan_switch_tiles(ctypes.byref(p)) == tiles
    p.d_c = 0
    assert _lib.lib().qmla_plan_switch_tiles(ctypes.byref(p)) < 0


@pytest.mark.parametrize("kv,d_c,rope,heads,rms,fold", [
    (_lib.KV_FP8, 512, 64, 24, _lib.RMS_LOG8, 4),          # warp-specialized: heads over 3 workgroups
    (_lib.KV_FP8, 512, 64, 24, _lib.RMS_E4M3, 4),          # per-group kernel: 96 rows over 3 workgroups
    (_lib.KV_FP8, 512, 64, 24, _lib.RMS_BF16_BYTES, 4),
    (_lib.KV_BF16, 512, 64, 24, _lib.RMS_BF16, 4),
    (_lib.KV_FP8, 768, 232, 24, _lib.RMS_LOG8, 4),         # the plugin's deployed rows (rope 232, TP 1)
    (_lib.KV_FP8, 768, 232, 24, _lib.RMS_E4M3, 4),
    (_lib.KV_FP8, 256, 232, 24, _lib.RMS_BF16_BYTES, 4),
    (_lib.KV_FP8, 768, 116, 12, _lib.RMS_LOG8, 4),         # ... rope 116, 12 heads (TP 2)
    (_lib.KV_BF16, 768, 232, 24, _lib.RMS_BF16, 4),        # column-split, 32 rows per workgroup
    (_lib.KV_FP8, 1792, 232, 24, _lib.RMS_LOG8, 4),        # column-split, 16-token tiles of 32 rows
    (_lib.KV_BF16, 1792, 232, 24, _lib.RMS_BF16, 4),       # column-split, 32 rows per workgroup
    (_lib.KV_BF16, 1792, 64, 24, _lib.RMS_BF16, 2),
    (_lib.KV_BF16, 1792, 300, 24, _lib.RMS_BF16, 1),       # no instance at all: no fold
])
def test_verify_fold_every_format(kv, d_c, rope, heads, rms, fold):
    """Spec-verify folding asks the library which fold a compiled kernel serves: 4 query tokens x 24
    heads fold into one request for every cache format and deployed layout up to rank 768 and on the
    rank-1792 rope-window layouts (2 on the rank-1792 rope-64 instances with 16 rows per workgroup
    and per-row rms reads), so the cache is read once per
    request, or once per pair of tokens, instead of once per token (no launch, no pointers). The
    reference folds 2 tokens at 24 heads (64-row groups, mla_decode_attention.py:1291-1300)."""
    from qmla.decode import fold_rows
    p = _layout(kv, d_c, rope, heads, rms, 1, 1)
    p.rows = 8 * 4
    p.q_nope = p.q_pe = p.kv_cache = p.block_table = p.seq_lens = p.out = None   # shape questions only
    assert fold_rows(p, 4) == fold
    assert p.qrows == 1                                                       # left as it was
    p.qrows = fold
    assert _lib.lib().qmla_decode_supported(ctypes.byref(p)) == (_lib.OK if fold > 1 else _lib.ERR_NOKERNEL)


def test_null_params_and_balanced_workspace_errors():
    lib = _lib.lib()
    assert lib.qmla_decode(None, None) == _lib.ERR_NULL
    assert lib.qmla_workspace_bytes(None) == 0
    p = _valid_params(num_splits=0, num_workgroups=16, workspace_bytes=0)
    assert lib.qmla_plan(ctypes.byref(p), None) == _lib.ERR_WORKSPACE
    p = _valid_params(num_splits=3)
    assert lib.qmla_plan(ctypes.byref(p), None) == _lib.ERR_MODE


def test_workspace_bytes_arithmetic():
    lib = _lib.lib()
    p = _valid_params(num_splits=4)
    assert lib.qmla_workspace_bytes(ctypes.byref(p)) == 8 * 24 * 4 * 513 * 4
    p = _valid_params(num_splits=1)
    assert lib.qmla_workspace_bytes(ctypes.byref(p)) == 0
    small = lib.qmla_workspace_bytes(ctypes.byref(_valid_params(num_splits=0, num_workgroups=16)))
    big = lib.qmla_workspace_bytes(ctypes.byref(_valid_params(num_splits=0, num_workgroups=64)))
    # balanced: (workgroups + requests) partial slots of H x (d_c + lse) floats, plus the plan
    assert big - small >= 48 * 24 * 513 * 4
    assert small >= (16 + 8) * 24 * 513 * 4


def test_build_params_reads_real_strides():
    q = torch.empty(6, 24, 576, dtype=torch.bfloat16)
    qn, qp = q[..., :512], q[..., 512:]
    cache = torch.empty(10, 64, 1, 608, dtype=torch.uint8)[2:9]       # a view: page stride from the tensor
    bt = torch.zeros(6, 40, dtype=torch.int32)
    sl = torch.zeros(6, dtype=torch.int32)
    out = torch.empty(6, 24, 512, dtype=torch.bfloat16)
    lse = torch.empty(6, 24)
    p = build_params(q_nope=qn, q_pe=qp, kv_cache=cache, block_table=bt, seq_lens=sl, out=out, lse=lse, d_c=512,
                     rope_w=64, rms_offset=576, rms_mode=_lib.RMS_LOG8, kv=_lib.KV_FP8, page_size=64,
                     sm_scale=0.1, qrows=2)
    assert (p.q_nope_stride_row, p.q_nope_stride_head) == (24 * 576, 576)
    assert p.q_pe == qn.data_ptr() + 512 * 2
    assert (p.page_stride, p.token_stride) == (64 * 608, 608)
    assert p.kv_cache == cache.data_ptr() and p.bt_stride == 40
    assert (p.rows, p.heads, p.rms_heads, p.qrows) == (6, 24, 24, 2)
    assert p.out_dtype == _lib.DT_BF16 and p.lse_dtype == _lib.DT_F32
    flat = torch.empty(640, 1, 608, dtype=torch.uint8)                  # 3-D [pages*P, 1, row]
    p3 = build_params(q_nope=qn, q_pe=qp, kv_cache=flat, block_table=bt, seq_lens=sl, out=out, lse=None,
                      d_c=512, rope_w=64, rms_offset=576, rms_mode=_lib.RMS_LOG8, kv=_lib.KV_FP8, page_size=64,
                      sm_scale=0.1)
    assert (p3.page_stride, p3.token_stride) == (64 * 608, 608) and p3.lse is None
    # the page bound: pages of the 4-D view, tokens / page_size of the 3-D cache; no status word
    assert p.num_pages == 7 and p3.num_pages == 10 and not p.status
    status = torch.zeros(1, dtype=torch.int32)
    p4 = build_params(q_nope=qn, q_pe=qp, kv_cache=flat, block_table=bt, seq_lens=sl, out=out, lse=None,
                      d_c=512, rope_w=64, rms_offset=576, rms_mode=_lib.RMS_LOG8, kv=_lib.KV_FP8, page_size=64,
                      sm_scale=0.1, status=status)
    assert p4.status == status.data_ptr()
    with pytest.raises(TypeError):
        build_params(q_nope=qn, q_pe=qp, kv_cache=flat, block_table=bt, seq_lens=sl, out=out, lse=None,
                     d_c=512, rope_w=64, rms_offset=576, rms_mode=_lib.RMS_LOG8, kv=_lib.KV_FP8, page_size=64,
                     sm_scale=0.1, status=torch.zeros(1, dtype=torch.int64))
    # the kernels store into *status from the device: a status word off the cache's device (a host
    # tensor beside a device cache, here a meta tensor beside a host one) is refused
    with pytest.raises(TypeError):
        build_params(q_nope=qn, q_pe=qp, kv_cache=flat, block_table=bt, seq_lens=sl, out=out, lse=None,
                     d_c=512, rope_w=64, rms_offset=576, rms_mode=_lib.RMS_LOG8, kv=_lib.KV_FP8, page_size=64,
                     sm_scale=0.1, status=torch.zeros(1, dtype=torch.int32, device="meta"))


def test_negative_page_count_rejected():
    lib = _lib.lib()
    p = _valid_params(num_splits=4, num_pages=-1)
    assert lib.qmla_decode(ctypes.byref(p), None) == _lib.ERR_SHAPE


def _bp_args(**over):
    q = torch.empty(6, 24, 576, dtype=torch.bfloat16)
    a = dict(q_nope=q[..., :512], q_pe=q[..., 512:], kv_cache=torch.empty(8, 64, 1, 608, dtype=torch.uint8),
             block_table=torch.zeros(6, 40, dtype=torch.int32), seq_lens=torch.zeros(6, dtype=torch.int32),
             out=torch.empty(6, 24, 512, dtype=torch.bfloat16), lse=torch.empty(6, 24), d_c=512, rope_w=64,
             rms_offset=576, rms_mode=_lib.RMS_LOG8, kv=_lib.KV_FP8, page_size=64, sm_scale=0.1)
    a.update(over)
    return a


@pytest.mark.parametrize("over,exc", [
    (dict(block_table=torch.zeros(6, 40, dtype=torch.int64)), TypeError),
    (dict(seq_lens=torch.zeros(6, dtype=torch.int64)), TypeError),
    (dict(seq_lens=torch.zeros(12, dtype=torch.int32)[::2]), ValueError),          # strided lengths
    (dict(block_table=torch.zeros(40, 6, dtype=torch.int32).t()), ValueError),      # column stride 6
    (dict(out=torch.empty(6, 512, 24, dtype=torch.bfloat16).transpose(1, 2)), ValueError),
    (dict(lse=torch.empty(24, 6).t()), ValueError),
    (dict(kv_cache=torch.empty(8, 64, 1, 1216, dtype=torch.uint8)[..., ::2]), ValueError),
    (dict(q_nope=torch.empty(6, 24, 1024, dtype=torch.bfloat16)[..., ::2]), ValueError),
    (dict(q_nope=torch.empty(6, 24, 512, dtype=torch.float16)), TypeError),
])
def test_build_params_rejects_unreadable_layouts(over, exc):
    """The kernels read int32 metadata and unit-stride rows; anything else raises rather than being
    converted (a conversion would allocate inside graph capture) or silently misread."""
    with pytest.raises(exc):
        build_params(**_bp_args(**over))


def test_product_path_refuses_cpu_tensors():
    case_q = torch.zeros(1, 24, 512, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        qmla.forward(case_q, torch.zeros(1, 24, 64, dtype=torch.bfloat16),
                     torch.zeros(1, 64, 1, 608, dtype=torch.uint8), torch.zeros(1, 1, dtype=torch.int32),
                     torch.ones(1, dtype=torch.int32), page_size=64, sm_scale=0.1, kv_fp8=True)


@pytest.mark.parametrize("name,mirror", [("qmla_cache_write_params", _lib.CacheWriteParams),
                                         ("qmla_gather_params", _lib.GatherParams),
                                         ("qmla_prep_params", _lib.PrepParams)])
def test_cache_struct_mirrors_match_header(name, mirror):
    text = HEADER.read_text()
    body = text[text.index("typedef struct " + name):text.index("} " + name + ";")]
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = []
    for decl in body.split("{", 1)[1].split(";"):
        decl = decl.strip()
        if not decl:
            continue
        parts = decl.split(",")
        fields.append(re.findall(r"(\w+)\s*$", parts[0])[0])
        fields.extend(re.sub(r"[\*\s]", "", x) for x in parts[1:])
    assert fields == [f[0] for f in mirror._fields_]


def _write_params(**over) -> _lib.CacheWriteParams:
    p = _lib.CacheWriteParams()
    base = 0x10000
    p.kv_c, p.kv_c_stride, p.k_pe, p.k_pe_stride = base, 512, base + 0x100000, 96
    p.slots, p.n, p.d_c, p.rope_w, p.rms_heads = base + 0x200000, 8, 512, 64, 24
    p.kv_dtype, p.rms_mode, p.k_scale = _lib.KV_FP8, _lib.RMS_LOG8, base + 0x300000
    p.cache, p.page_stride, p.token_stride, p.page_size, p.num_slots = base + 0x400000, 64 * 608, 608, 64, 6400
    for k, v in over.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("over,code", [
    (dict(kv_c=None), _lib.ERR_NULL),
    (dict(k_scale=None), _lib.ERR_NULL),
    (dict(kv_dtype=5), _lib.ERR_MODE),
    (dict(rms_mode=_lib.RMS_BF16), _lib.ERR_MODE),                          # bf16 element in an fp8 row
    (dict(kv_dtype=_lib.KV_BF16, rms_mode=_lib.RMS_LOG8), _lib.ERR_MODE),
    (dict(d_c=508), _lib.ERR_SHAPE),
    (dict(token_stride=592, page_stride=64 * 592), _lib.ERR_SHAPE),        # 600 bytes do not fit
    (dict(rms_mode=_lib.RMS_BF16_BYTES), _lib.ERR_SHAPE),                   # 624 bytes do not fit 608
    (dict(k_pe_stride=80), _lib.ERR_SHAPE),                                 # rope + 24 codes do not fit
    (dict(kv_c=0x10008), _lib.ERR_ALIGN),
    (dict(kv_c_stride=516), _lib.ERR_ALIGN),
    (dict(n=0), _lib.OK),
])
def test_cache_write_error_codes(over, code):
    p = _write_params(**over)
    assert _lib.lib().qmla_cache_write(ctypes.byref(p), None) == code
    assert _lib.lib().qmla_cache_write(None, None) == _lib.ERR_NULL


def _gather_params(**over) -> _lib.GatherParams:
    p = _lib.GatherParams()
    base = 0x10000
    p.cache, p.page_stride, p.token_stride, p.page_size, p.num_pages = base, 64 * 608, 608, 64, 100
    p.kv_dtype, p.rms_mode, p.rms_offset, p.rms_heads, p.scale = _lib.KV_FP8, _lib.RMS_LOG8, 576, 24, base + 0x100000
    p.block_table, p.bt_stride, p.num_seqs, p.bt_cols = base + 0x200000, 16, 4, 16
    p.cu_seq_lens, p.token_to_seq, p.num_tokens = base + 0x300000, base + 0x400000, 100
    p.dst, p.dst_stride, p.dst_dtype = base + 0x500000, 608, _lib.DT_BF16
    for k, v in over.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("over,code", [
    (dict(cache=None), _lib.ERR_NULL),
    (dict(scale=None), _lib.ERR_NULL),
    (dict(dst_dtype=_lib.DT_F32), _lib.ERR_MODE),
    (dict(rms_mode=_lib.RMS_NONE), _lib.ERR_MODE),
    (dict(kv_dtype=_lib.KV_BF16, row_elems=0), _lib.ERR_SHAPE),
    (dict(kv_dtype=_lib.KV_BF16, row_elems=600), _lib.ERR_SHAPE),        # 1200 bytes > 608-byte rows
    (dict(rms_offset=600), _lib.ERR_SHAPE),                           # 24 codes past the 608-byte row
    (dict(rms_offset=0), _lib.ERR_SHAPE),
    (dict(dst_stride=500), _lib.ERR_SHAPE),
    (dict(bt_stride=8), _lib.ERR_SHAPE),
    (dict(dst=0x500008), _lib.ERR_ALIGN),
    (dict(dst_stride=604), _lib.ERR_ALIGN),
    (dict(num_tokens=0), _lib.OK),
])
def test_gather_error_codes(over, code):
    p = _gather_params(**over)
    assert _lib.lib().qmla_gather(ctypes.byref(p), None) == code
    assert _lib.lib().qmla_gather(None, None) == _lib.ERR_NULL


def _prep_params(**over) -> _lib.PrepParams:
    """A valid description of 24 heads x 256 (rope 64 first), 4 rope groups, d_c 512 (never launched:
    every case below fails validation or has no tokens)."""
    p = _lib.PrepParams()
    base = 0x10000
    p.q, p.q_token_stride, p.q_head_stride = base, 24 * 512, 512
    p.latent, p.latent_stride = base + 0x100000, 512
    p.k_rope, p.k_rope_stride = base + 0x200000, 256
    p.k_up, p.k_gain = base + 0x300000, base + 0x400000
    p.cos_sin, p.cos_sin_dtype, p.max_pos = base + 0x500000, _lib.DT_BF16, 4096
    p.positions, p.pos_row_stride, p.pos_rows, p.rope_sec = base + 0x600000, 0, 1, None
    p.n, p.heads, p.head_dim, p.rope_dim, p.kv_heads, p.d_c = 8, 24, 256, 64, 4, 512
    p.head_offset, p.rope_group, p.rope_first, p.rope_span, p.declared_rope = 0, 6, 0, 4, 296
    p.eps = 1e-6
    p.q_out, p.q_out_token_stride, p.q_out_head_stride = base + 0x700000, 24 * 488, 488
    p.k_pe, p.k_pe_stride = base + 0x800000, 296
    for k, v in over.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("over,code", [
    (dict(q=None), _lib.ERR_NULL),
    (dict(k_gain=None), _lib.ERR_NULL),
    (dict(pos_rows=3, pos_row_stride=8), _lib.ERR_NULL),                  # M-RoPE without rope_sec
    (dict(pos_rows=2), _lib.ERR_SHAPE),
    (dict(cos_sin_dtype=7), _lib.ERR_MODE),
    (dict(d_c=448), _lib.ERR_SHAPE),                                      # K halves of 64-wide blocks
    (dict(head_dim=64), _lib.ERR_SHAPE),                                  # no nope part
    (dict(rope_first=1), _lib.ERR_SHAPE),                                 # head 0's group not cached
    (dict(rope_span=5), _lib.ERR_SHAPE),                                  # more groups than k_rope holds
    (dict(declared_rope=272), _lib.ERR_SHAPE),                            # rope 256 + 24 rms do not fit
    (dict(head_offset=12, rope_first=2, rope_span=1), _lib.ERR_SHAPE),    # heads 12..35 span 4 groups
    (dict(q_out_head_stride=480), _lib.ERR_SHAPE),
    (dict(k_pe_stride=200), _lib.ERR_SHAPE),
    (dict(latent=0x100008 + 0x10000), _lib.ERR_ALIGN),
    (dict(latent_stride=516), _lib.ERR_ALIGN),
    (dict(q_head_stride=513, q_token_stride=24 * 513), _lib.ERR_ALIGN),
    (dict(n=0), _lib.OK),
])
def test_prep_error_codes(over, code):
    p = _prep_params(**over)
    assert _lib.lib().qmla_prep(ctypes.byref(p), None) == code
    assert _lib.lib().qmla_prep(None, None) == _lib.ERR_NULL


@pytest.mark.parametrize("rank", [256, 768, 1792])
def test_unpadded_rows_take_narrow_row_kernels(rank):
    """The reference's standalone numerics test decodes rows of rank + 256 rope + 12 rms bf16 elements
    with no padding (tests/test_decode_numerics.py:60-67, 89-91): 1048 / 2072 / 4120 bytes, on 8-byte
    boundaries. The plugin pads every cache row to 16 elements for its 128-bit path
    (qwen_mla/mla_impl.py:252-271, cp_async_safe in qwen_mla/fi_decode.py:117-127); here such rows
    route to the narrow-row instances (4 bytes a lane), which exist for exactly these layouts. Rows
    off 4-byte boundaries, and narrow rows of any other layout, are refused with QMLA_ERR_ALIGN
    before any device work, and the Python entries raise it (no launch here)."""
    from qmla.layout import row_dma_safe
    heads, page = 12, 400
    entry = rank + 256 + heads
    assert not row_dma_safe(entry, page, rank, rank + 256, 2)
    p = _layout(_lib.KV_BF16, rank, 256, heads, _lib.RMS_BF16)
    p.token_stride, p.page_stride, p.page_size = entry, entry * page, page
    assert _lib.lib().qmla_decode_supported(ctypes.byref(p)) == _lib.OK
    p.page_size, p.page_stride = 401, entry * 401          # pages off 16-byte boundaries as well
    assert _lib.lib().qmla_decode_supported(ctypes.byref(p)) == _lib.OK
    # the 24-head rows of the same test are on 16-byte boundaries: the ordinary kernels
    p24 = _layout(_lib.KV_BF16, rank, 256, 24, _lib.RMS_BF16)
    p24.token_stride, p24.page_stride, p24.page_size = rank + 256 + 24, (rank + 256 + 24) * page, page
    assert _lib.lib().qmla_decode_supported(ctypes.byref(p24)) == _lib.OK
    # a narrow row of a layout no narrow-row instance serves (rope 64), and rows on 2-byte boundaries
    pn = _layout(_lib.KV_BF16, rank, 64, heads, _lib.RMS_BF16)
    pn.token_stride, pn.page_stride, pn.page_size = rank + 64 + heads, (rank + 64 + heads) * page, page
    assert _lib.lib().qmla_decode_supported(ctypes.byref(pn)) == _lib.ERR_ALIGN
    p.token_stride, p.page_stride = entry + 1, (entry + 1) * page
    assert _lib.lib().qmla_decode_supported(ctypes.byref(p)) == _lib.ERR_ALIGN
    # what the Python entries raise on it (the error names the alignment)
    with pytest.raises(RuntimeError, match="ALIGN"):
        _lib.check("qmla_decode_supported", _lib.lib().qmla_decode_supported(ctypes.byref(p)))
