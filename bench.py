#!/usr/bin/env python3
"""MLA decode throughput on one MI355X: tokens/s and achieved HBM GB/s.

Default workload (the headline metric): FP8 e4m3 latent KV with 1-byte log2 rms codes, B=128
decode rows, 24 heads sharing one latent row, d_c=512, d_r=64, 64-token pages behind a
random-permutation block table, context lengths lognormal (median 16384, sigma 0.5) clipped to
[1024, 65536], latent/rope drawn N(0,1) x4 against a per-layer scale calibrated on the unscaled
draw, seed 2. Inputs are resident in HBM before timing.

Prints ONE JSON line. `value` = decode rows per second of the whole call (plan + decode + combine)
at one layer; `roofline` reports the decode kernel's algorithmic bytes over its own average
duration (HIP events on the stream it runs on); `cpu_baseline` times the CPU oracle on a fixed
sample of the same workload on this host's cores.

    python bench.py [--steps K] [--warmup W] [--workload fp8_b128|bf16_b64|gla_b48|wide_b32] [--no-cpu]
    python bench.py --path write_n16384|gather_n16384|prep_b128     (the kernels beside the decode)
"""
from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import statistics
import sys
import time

REPO = pathlib.Path(__file__).resolve().parent
for p in (REPO, REPO / "qwen-mla-vllm_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

METRIC = "MLA decode tokens/s + achieved HBM GB/s (% peak), B=128 ctx16k fp8 latent KV"
HBM_PEAK_GBPS = 8000.0

WORKLOADS = {
    # name: (make_case kwargs, description)
    "fp8_b128": dict(batch=128, heads=24, d_c=512, rope_w=64, page_size=64, kv="fp8", rms_mode="log8", seed=2,
                     amp=4.0, lens=("lognormal", 16384, 0.5, 1024, 65536)),
    "bf16_b64": dict(batch=64, heads=24, d_c=512, rope_w=64, page_size=64, kv="bf16", rms_mode="bf16", seed=1,
                     amp=1.0, lens=("uniform", 4096, 32768)),
    "gla_b48": dict(batch=48, heads=24, d_c=512, rope_w=64, page_size=64, kv="fp8", rms_mode="log8", seed=4,
                    amp=1.0, lens=("uniform", 8192, 32768), qrows=4, groups=2),
    # MTP verify on plain MLA: 64 requests x 4 query tokens x 24 heads (96 rows per request, folded
    # so each cached row is read once from HBM: the heads split over 3 workgroups on one XCD)
    "verify_b64x4": dict(batch=64, heads=24, d_c=512, rope_w=64, page_size=64, kv="fp8", rms_mode="log8", seed=5,
                         amp=4.0, lens=("lognormal", 16384, 0.5, 1024, 65536), qrows=4),
    # the same verify step on a bf16 cache: the wide-row kernel splits the heads over 3 workgroups
    # that read each token range together
    "verify_bf16_b64x4": dict(batch=64, heads=24, d_c=512, rope_w=64, page_size=64, kv="bf16", rms_mode="bf16",
                              seed=5, amp=1.0, lens=("lognormal", 16384, 0.5, 1024, 65536), qrows=4),
    # the shapes of the reference's own kernel timings (qwen_mla/kernels/qwen_mla.cuh:1450-1454,
    # ops/mla_decode_attention.py:925-927): B 64 x ctx 32k, 12 heads (TP 2 rank-local), bf16 rows of
    # [latent | packed rope 116 | 12 bf16 rms] (the 128-column window after the latent), ranks 256,
    # 768 and 1792; balanced split mode
    "pub_r256_h12": dict(batch=64, heads=12, d_c=256, rope_w=116, page_size=64, kv="bf16", rms_mode="bf16",
                         seed=11, amp=1.0, lens=("fixed", 32768)),
    "pub_r768_h12": dict(batch=64, heads=12, d_c=768, rope_w=116, page_size=64, kv="bf16", rms_mode="bf16",
                         seed=12, amp=1.0, lens=("fixed", 32768)),
    "pub_r1792_h12": dict(batch=64, heads=12, d_c=1792, rope_w=116, page_size=64, kv="bf16", rms_mode="bf16",
                          seed=13, amp=1.0, lens=("fixed", 32768)),
    # the plugin's deployed FP8 row at TP 1: rank 768, packed rope 232, 24 log8 rms codes (1024 bytes),
    # with the headline's batch and lengths
    "fp8_r768_b128": dict(batch=128, heads=24, d_c=768, rope_w=232, page_size=64, kv="fp8", rms_mode="log8",
                          seed=14, amp=4.0, lens=("lognormal", 16384, 0.5, 1024, 65536)),
    # the plugin's deployed rows at rank 1792 (tests/test_fp8_kv.py:136-138, tests/test_two_pass_1792.py:
    # 12-19): packed rope 232, 24 heads; FP8 with log8 codes at the headline's batch and lengths, and
    # bf16 at B 64 (column-split kernel)
    "fp8_r1792_b128": dict(batch=128, heads=24, d_c=1792, rope_w=232, page_size=64, kv="fp8", rms_mode="log8",
                           seed=16, amp=4.0, lens=("lognormal", 16384, 0.5, 1024, 65536)),
    "bf16_r1792_b64": dict(batch=64, heads=24, d_c=1792, rope_w=232, page_size=64, kv="bf16", rms_mode="bf16",
                           seed=17, amp=1.0, lens=("lognormal", 16384, 0.5, 1024, 65536)),
    # wide latent: 16 fixed splits in the reference's attn_logits layout, then the combine
    "wide_b32": dict(batch=32, heads=24, d_c=1792, rope_w=64, page_size=1600, kv="bf16", rms_mode="bf16", seed=3,
                     amp=1.0, lens=("fixed", 65536), splits=16),
}
CPU_EVERY = {"wide_b32": 8, "pub_r256_h12": 4, "pub_r768_h12": 8, "pub_r1792_h12": 16, "fp8_r1792_b128": 16,
             "bf16_r1792_b64": 16}
GRAPH_CALLS = 16   # decode calls recorded into one HIP graph (one per layer of a 16-layer forward)


def make_workload(name, device):
    from qmla.synth import lognormal_lens, make_case, uniform_lens
    w = dict(WORKLOADS[name])
    spec = w.pop("lens")
    w.pop("splits", None)
    if spec[0] == "lognormal":
        lens = lognormal_lens(w["batch"], spec[1], spec[2], spec[3], spec[4], seed=w["seed"])
    elif spec[0] == "fixed":
        lens = [spec[1]] * w["batch"]
    else:
        lens = uniform_lens(w["batch"], spec[1], spec[2], seed=w["seed"])
    return make_case(lens=lens, device=device, rms="row", **w), spec


def decode_call(case, splits, dev):
    """The exact call the bench times: qmla_decode on prebuilt parameters, balanced split mode with a
    reserved workspace, or `splits` fixed splits with the reference's attn_logits [B, H, S, Dv+1]
    partials. Returns (params, out, lse, buffers to keep alive)."""
    import torch
    from qmla import _lib
    from qmla.decode import Workspace, build_params, workspace_bytes
    rows, H = case.q_nope.shape[0], case.heads
    dv = case.d_c // case.groups
    out = torch.empty(rows, H, dv, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(rows, H, dtype=torch.float32, device=dev)
    kv = _lib.KV_FP8 if case.kv == "fp8" else _lib.KV_BF16
    mode = {"bf16": _lib.RMS_BF16, "log8": _lib.RMS_LOG8, "bf16_bytes": _lib.RMS_BF16_BYTES,
            "e4m3": _lib.RMS_E4M3, "none": _lib.RMS_NONE}[case.rms_mode]
    args_p = dict(q_nope=case.q_nope, q_pe=case.q_pe, kv_cache=case.cache, block_table=case.block_table,
                  seq_lens=case.seq_lens, out=out, lse=lse, d_c=case.d_c, rope_w=case.rope_w,
                  rms_offset=case.rms_offset, rms_mode=mode, kv=kv, page_size=case.page_size,
                  sm_scale=case.sm_scale, k_scale=case.k_scale, qrows=case.qrows, groups=case.groups,
                  num_splits=0, split_align=0)
    if splits:
        logits = torch.empty(rows, H, splits, dv + 1, dtype=torch.float32, device=dev)
        args_p.update(num_splits=splits, split_align=16 if case.page_size % 16 == 0 else 0)
        p = build_params(workspace=logits, ws_strides=(logits.stride(0), logits.stride(1), logits.stride(2)),
                         **args_p)
        return p, out, lse, (logits,)
    ws = Workspace().reserve(workspace_bytes(build_params(**args_p)), dev)
    return build_params(workspace=ws, **args_p), out, lse, (ws,)


def kernel_bytes(case) -> int:
    """Algorithmic bytes the decode kernel reads: cached rows (latent + rope + rms, padding
    excluded), queries, block-table entries and lengths."""
    import torch
    e = 1 if case.kv == "fp8" else 2
    r = 2 if case.rms_mode in ("bf16", "bf16_bytes") else 1
    n_req = case.seq_lens.shape[0] // case.qrows
    L = case.seq_lens.view(n_req, case.qrows)[:, -1].to(torch.int64)
    toks = int(L.sum())
    rows, H = case.q_nope.shape[0], case.heads
    dv = case.d_c // case.groups
    pages = int(((L + case.page_size - 1) // case.page_size).sum())
    return toks * (case.d_c * e + case.rope_w * e + H * r) + rows * H * (dv + case.rope_w) * 2 + pages * 4 + rows * 4


def measured_traffic(workload: str):
    """HBM bytes per decode launch from the committed counter summary of this workload
    (FETCH_SIZE + WRITE_SIZE, each scaled by what it reads for a 1 GiB copy), or None."""
    f = REPO / "profiles" / f"traffic_mla_decode_{workload}.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            return int(line.split(":", 1)[1])
    return None


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(case, sample_every: int, budget_s: float):
    """The CPU oracle on a fixed sample of the workload's requests (every k-th), timed on this host's
    cores; returns decode rows per second scaled per request."""
    import torch
    from oracle import mla_oracle as ora
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    from qmla.synth import compact_requests
    n_req = case.seq_lens.shape[0] // case.qrows
    picks = list(range(0, n_req, sample_every))
    cache, new_bt, sll, qn, qp, rows = compact_requests(case, picks)
    P = case.page_size
    rms_map = {"bf16": ora.RMS_BF16, "log8": ora.RMS_LOG8, "bf16_bytes": ora.RMS_BF16_BYTES,
               "e4m3": ora.RMS_E4M3, "none": ora.RMS_NONE}
    ks = float(case.k_scale.cpu()) if case.k_scale is not None else 1.0

    def run():
        ora.mla_decode(qn, qp, cache, new_bt, sll, page_size=P, d_c=case.d_c, rope_w=case.rope_w,
                       rms_offset=case.rms_offset, kv=case.kv, rms_mode=rms_map[case.rms_mode], k_scale=ks,
                       sm_scale=case.sm_scale, rms_heads=case.heads, groups=case.groups)

    t, k = _cpu_runs(run, budget_s)
    toks = int(sll.to(torch.int64).sum())
    return {"value": round(len(rows) / t, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "cpu": cpu_model(),
            "sample": f"{len(picks)} of {n_req} requests (every {sample_every}th, {len(rows)} rows, "
                      f"{toks} cached tokens), fp32 torch oracle, {CPU_WARMUP} warm-up runs then the median "
                      f"of {k} ({t:.2f} s each), scaled per request"}


CPU_WARMUP, CPU_RUNS = 2, 5


def _cpu_runs(fn, budget_s):
    """CPU_WARMUP untimed runs, then the median of CPU_RUNS timed ones (fewer, but at least one,
    when a run takes longer than the budget allows)."""
    for _ in range(CPU_WARMUP):
        fn()
    times, t_all = [], time.perf_counter()
    while True:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= CPU_RUNS or time.perf_counter() - t_all > budget_s:
            return statistics.median(times), len(times)


def cpu_reference_small():
    """The CPU-runnable reference configuration timed in full on this host's cores: B=4 rows, 24
    heads sharing one latent row, d_c 512, d_r 64, 2048 tokens each, bf16 cache in 16-token pages
    behind a random-permutation block table, N(0,1) inputs with seed 0, row-RMS divisor, fp32
    softmax, bf16 output; the fp32 torch oracle (decode rows per second)."""
    import torch
    from oracle import mla_oracle as ora
    from qmla.synth import make_case
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    from qmla.synth import compact_requests
    c = make_case(batch=4, heads=24, d_c=512, rope_w=64, page_size=16, lens=[2048] * 4, kv="bf16",
                  rms_mode="bf16", seed=0, device="cpu", rms="row", amp=1.0)
    cache, bt, sl, qn, qp, _ = compact_requests(c, list(range(4)))

    def run():
        o, _ = ora.mla_decode(qn, qp, cache, bt, sl, page_size=16, d_c=512, rope_w=64, rms_offset=c.rms_offset,
                              kv="bf16", rms_mode=ora.RMS_BF16, k_scale=1.0, sm_scale=c.sm_scale, rms_heads=24,
                              groups=1)
        o.to(torch.bfloat16)

    t, k = _cpu_runs(run, 20.0)
    return {"value": round(4 / t, 2), "unit": "tokens/s", "cores": cores, "kind": "port", "cpu": cpu_model(),
            "sample": f"all of it: B 4 x 2048 tokens, bf16 cache, P 16, fp32 torch oracle, {CPU_WARMUP} warm-up runs "
                      f"then the median of {k} ({t * 1e3:.1f} ms each)"}


# ------------------------------------------------------------------------------------------------
# the kernels either side of the decode: cache-row writer, prefill context gather, decode prep
# ------------------------------------------------------------------------------------------------
ADJACENT = {
    # FP8 log8 rows for a 16384-token prefill chunk written to random free slots
    "write_n16384": dict(n=16384, heads=24, d_c=512, rope_w=64, page_size=64, seed=5),
    # ... a 262144-token prefill (long prompts), where launch and ramp no longer dominate
    "write_n262144": dict(n=262144, heads=24, d_c=512, rope_w=64, page_size=64, seed=5),
    # 4 x 4096 cached tokens of FP8 log8 rows gathered into a bf16 workspace
    "gather_n16384": dict(n=16384, seqs=4, heads=24, d_c=512, rope_w=64, page_size=64, seed=6),
    # ... 4 x 65536 cached tokens
    "gather_n262144": dict(n=262144, seqs=4, heads=24, d_c=512, rope_w=64, page_size=64, seed=6),
    # the decode step's q / k_pe prep at B=128: 24 heads of 256, rope 64 in 4 groups, d_c 512
    "prep_b128": dict(n=128, heads=24, head_dim=256, rd=64, kv_heads=4, rope_group=6, d_c=512, declared=296,
                      max_pos=65536, seed=7),
}


def _time_launches(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t = time.perf_counter()
    e0.record(st)
    for _ in range(steps):
        fn()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, time.perf_counter() - t


def adjacent(args):
    """One JSON line for a kernel either side of the decode: rows per second of one launch with
    inputs resident in HBM (the C entry point called with prebuilt parameters, K launches back to
    back), algorithmic bytes over its average duration (HIP events on the stream it runs on) against
    the HBM peak, and the oracle on the same rows on this host's cores."""
    import numpy as np
    import torch
    import qmla
    from oracle import mla_oracle as ora
    import ctypes
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib, st = qmla.lib(), torch.cuda.current_stream().cuda_stream
    w = ADJACENT[args.path_workload]
    g = torch.Generator().manual_seed(w["seed"])
    kind = args.path_workload.split("_")[0]
    if kind == "write":
        n, H, d_c, W, P = w["n"], w["heads"], w["d_c"], w["rope_w"], w["page_size"]
        kv_c = (torch.randn(n, d_c, generator=g) * 4).to(torch.bfloat16)
        k_pe = torch.empty(n, W + H, dtype=torch.bfloat16)
        k_pe[:, :W] = (torch.randn(n, W, generator=g) * 4).to(torch.bfloat16)
        k_pe[:, W:] = torch.exp(torch.randn(n, H, generator=g) * 0.6).to(torch.bfloat16)
        pages = n // P * 2
        slots = torch.randperm(pages * P, generator=g)[:n]
        cache = torch.zeros(pages, P, 1, 608, dtype=torch.uint8, device=dev)
        ks = torch.tensor(kv_c.float().abs().max().item() / 448.0, device=dev)
        a = (kv_c.to(dev), k_pe.to(dev), cache, slots.to(dev))
        from qmla.cache import cache_write_params
        prm, keep = cache_write_params(*a, rope_w=W, rms_heads=H, kv_fp8=True, rms="log8", k_scale=ks)
        fn = lambda: lib.qmla_cache_write(ctypes.byref(prm), st)
        alg = n * ((d_c + W + H) * 2 + (d_c + W + H) + 8)          # bf16 inputs + fp8 row + slot id
        kc, kp = kv_c.float().numpy(), k_pe.float().numpy()
        ksf = float(ks.cpu())
        cpu_fn = lambda: ora.fp8_row_bytes(kc, kp, packed_rope=W, n_heads=H, k_scale=ksf, rms_mode=ora.RMS_LOG8)
        cpu_rows, sample = n, f"all {n} rows, numpy oracle (fp8_row_bytes)"
        cfg = {"workload": f"mla_cache_write_n{n}", "tokens": n, "heads": H, "d_c": d_c, "d_r": W,
               "kv": "fp8", "rms": "log8", "row_bytes": 608}
        metric, dtype = "MLA FP8 cache-row writer rows/s + achieved HBM GB/s", "bf16->e4m3"
    elif kind == "gather":
        from qmla.synth import make_case
        n, S, H, P = w["n"], w["seqs"], w["heads"], w["page_size"]
        c = make_case(batch=S, heads=H, d_c=w["d_c"], rope_w=w["rope_w"], page_size=P, lens=[n // S] * S, kv="fp8",
                      rms_mode="log8", seed=w["seed"], device=dev, rms="spread")
        lens = torch.full((S,), n // S, dtype=torch.int64)
        cu = torch.zeros(S + 1, dtype=torch.int32)
        cu[1:] = torch.cumsum(lens, 0).to(torch.int32)
        t2s = torch.repeat_interleave(torch.arange(S, dtype=torch.int32), lens)
        dst = torch.empty(n, c.row, dtype=torch.bfloat16, device=dev)
        cud, t2sd = cu.to(dev), t2s.to(dev)
        mla_rms = (c.rms_offset, H, "log8")
        from qmla.cache import gather_params
        prm, keep = gather_params(src_cache=c.cache, dst=dst, block_table=c.block_table, cu_seq_lens=cud,
                                  token_to_seq=t2sd, num_tokens=n, kv_cache_dtype="fp8", scale=c.k_scale,
                                  mla_rms=mla_rms)
        fn = lambda: lib.qmla_gather(ctypes.byref(prm), st)
        width = c.rms_offset + H
        alg = n * (width + 2 * width + 4) + S * (n // S // P) * 4 + (S + 1) * 4
        cb = c.cache.cpu().contiguous().view(torch.uint8).reshape(c.cache.shape[0], P, -1).numpy()
        btn, ks = c.block_table.cpu().numpy(), float(c.k_scale.cpu())
        cpu_fn = lambda: ora.gather_context(cb, btn, cu.numpy(), t2s.numpy(), n, None, kv="fp8", scale=ks,
                                            rms_offset=c.rms_offset, n_heads=H, rms_mode=ora.RMS_LOG8)
        cpu_rows, sample = n, f"all {n} rows, numpy oracle (gather_context)"
        cfg = {"workload": f"mla_gather_n{n}", "tokens": n, "seqs": S, "heads": H, "d_c": w["d_c"],
               "d_r": w["rope_w"], "page_size": P, "kv": "fp8", "rms": "log8", "dst": "bf16"}
        metric, dtype = "MLA prefill context gather rows/s + achieved HBM GB/s", "e4m3->bf16"
    else:
        n, H, hd, rd, kvh, d_c, decl = (w[k] for k in ("n", "heads", "head_dim", "rd", "kv_heads", "d_c", "declared"))
        nope = hd - rd
        q = torch.randn(n, H, hd, generator=g).to(torch.bfloat16)
        lat = torch.randn(n, d_c, generator=g).to(torch.bfloat16)
        kr = torch.randn(n, kvh * rd, generator=g).to(torch.bfloat16)
        ku = (torch.randn(H * nope, d_c, generator=g) * d_c ** -0.5).to(torch.bfloat16)
        wn = (torch.randn(hd, generator=g) * 0.1).to(torch.bfloat16)
        tab = qmla.partial_rope_table(list(range(rd // 2)), rd, 1e7, w["max_pos"]).to(torch.bfloat16)
        pos = torch.randint(0, w["max_pos"], (n,), generator=g)
        a = [t.to(dev) for t in (pos, q, lat, kr, ku)]
        gain = qmla.k_gain(wn.to(dev), rd)
        tabd = tab.to(dev)
        q_out = torch.empty(n, H, nope + decl, dtype=torch.bfloat16, device=dev)
        k_pe = torch.empty(n, decl, dtype=torch.bfloat16, device=dev)
        from qmla.prep import prep_params
        prm, keep, _, _ = prep_params(*a, gain, tabd, head_offset=0, rope_group=w["rope_group"], rope_first=0,
                                      rope_span=kvh, declared_rope=decl, eps=1e-6, q_out=q_out, k_pe=k_pe)
        fn = lambda: lib.qmla_prep(ctypes.byref(prm), st)
        alg = (n * H * hd * 2 + n * d_c * 2 + n * kvh * rd * 2 + H * nope * d_c * 2 + rd * 4 + n * 8 + n * rd * 2
               + n * H * (nope + decl) * 2 + n * decl * 2)
        qn, ln, krn, kun, wnn, tabn = (t.float().numpy() for t in (q, lat, kr, ku, wn, tab))
        krn = krn.reshape(n, kvh, rd)
        posn = pos.numpy()
        cpu_fn = lambda: ora.mla_decode_prep(qn, ln, krn, kun, wnn, tabn, posn, head_offset=0,
                                             rope_group=w["rope_group"], rope_first=0, rope_span=kvh,
                                             declared_rope=decl, eps=1e-6)
        cpu_rows, sample = n, f"all {n} tokens, numpy oracle (mla_decode_prep, float64 up-projection)"
        cfg = {"workload": "mla_decode_prep_b128", "tokens": n, "heads": H, "head_dim": hd,
               "rope_dim": rd, "rope_groups": kvh, "d_c": d_c, "declared_rope": decl}
        metric, dtype = "MLA decode q/k_pe prep tokens/s + achieved HBM GB/s", "bf16"
    def launch():
        rc = fn()
        if rc != 0:
            raise RuntimeError(f"{kind} launch failed: {rc}")

    ms, wall = _time_launches(launch, args.steps, args.warmup)
    if args.copy_calib_mib:
        src = torch.empty(args.copy_calib_mib << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst_c = torch.empty_like(src)
        for _ in range(3):
            dst_c.copy_(src)
        torch.cuda.synchronize()
    n_rows = w["n"]
    gbps = alg / (ms / 1e3) / 1e9
    traffic = None
    f = REPO / "profiles" / f"traffic_{cfg['workload']}.md"
    if f.exists():
        for line in f.read_text().splitlines():
            if line.startswith("hbm_bytes_per_launch:"):
                traffic = int(line.split(":", 1)[1])
    cpu = None
    if not args.no_cpu:
        from threadpoolctl import threadpool_limits
        with threadpool_limits(1):                      # numpy / BLAS on one thread: cores = 1
            t, k = _cpu_runs(cpu_fn, min(args.cpu_budget, 10.0))
        cpu = {"value": round(cpu_rows / t, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
               "cpu": cpu_model(), "sample": f"{sample}, {CPU_WARMUP} warm-up runs then the median of {k} ({t:.3f} s each)"}
    print(json.dumps({
        "metric": metric, "value": round(n_rows / (ms / 1e3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": "synthetic", "config": cfg,
        "kernel_us": round(ms * 1e3, 3), "wall_s_timed": round(wall, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": traffic, "algorithmic_bytes_per_launch": alg},
        "cpu_baseline": cpu}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--workload", default="fp8_b128", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP-graph replay timing")
    ap.add_argument("--unfold", action="store_true",
                    help="verify workloads: decode every query token as a request of its own (no folding), "
                         "the way a caller without folding reads the cache once per token")
    ap.add_argument("--settle-ms", type=float, default=250.0,
                    help="run the call back to back this long before the warm-up steps (clock ramp)")
    ap.add_argument("--cpu-every", type=int, default=0, help="oracle on every k-th request (0: per workload)")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="also run a plain device copy of this many MiB (FETCH/WRITE_SIZE calibration)")
    ap.add_argument("--path", dest="path_workload", default=None, choices=sorted(ADJACENT),
                    help="time a kernel either side of the decode instead (writer, gather, prep)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "the benchmark measures one GPU only: the decode shards by request "
                                   "(no collectives); run with --gpus 1"}))
        sys.exit(2)

    if args.path_workload:
        adjacent(args)
        return
    import torch
    import qmla
    from qmla import _lib

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    case, spec = make_workload(args.workload, dev)
    rows, H = case.q_nope.shape[0], case.heads
    splits = WORKLOADS[args.workload].get("splits", 0)
    if args.unfold:
        case.qrows = 1                      # the flattened rows are requests of their own
    p, out, lse, keep = decode_call(case, splits, dev)
    lib = qmla.lib()
    st = torch.cuda.current_stream().cuda_stream

    def step():
        _lib.check("qmla_decode", lib.qmla_decode(p, st))

    # clock settle: the GPU's clocks ramp over the first tens of milliseconds of load, so the call
    # runs back to back for --settle-ms of wall time before the W warm-up steps
    settle_calls = 0
    t_settle = time.perf_counter()
    while (time.perf_counter() - t_settle) * 1e3 < args.settle_ms:
        for _ in range(20):
            step()
        settle_calls += 20
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # timed region 1: the whole call, K steps back to back
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    t_wall = time.perf_counter() - t_wall
    ms = e0.elapsed_time(e1) / args.steps

    # timed region 2: the same call stage by stage, events around the decode kernel
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
            torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for a, b, c in evs:
        if not splits:
            _lib.check("qmla_plan", lib.qmla_plan(p, st))
        a.record()
        _lib.check("qmla_decode_partial", lib.qmla_decode_partial(p, st))
        b.record()
        _lib.check("qmla_combine", lib.qmla_combine(p, st))
        c.record()
    torch.cuda.synchronize()
    part_ms = statistics.mean(a.elapsed_time(b) for a, b, _ in evs)
    comb_ms = statistics.mean(b.elapsed_time(c) for _, b, c in evs)

    # timed region 3: the call as the serving loop runs it, inside a captured HIP graph. A model's
    # decode graph holds one call per layer, so GRAPH_CALLS calls are recorded into one graph (the
    # graph launch is paid once per forward, not per call) and the graph is replayed until K calls
    # have run; graph_ms_per_step is per call
    graph_ms = None
    if not args.no_graph:
        g = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cap):
            step_on = lambda: _lib.check("qmla_decode", lib.qmla_decode(p, torch.cuda.current_stream().cuda_stream))
            step_on()
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=cap):
                for _ in range(GRAPH_CALLS):
                    step_on()
        torch.cuda.current_stream().wait_stream(cap)
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        reps = max(1, -(-args.steps // GRAPH_CALLS))
        g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        g0.record()
        for _ in range(reps):
            g.replay()
        g1.record()
        torch.cuda.synchronize()
        graph_ms = g0.elapsed_time(g1) / (reps * GRAPH_CALLS)
        del g

    # timed region 4: cold L2 / MALL -- 512 MiB written between calls, each call timed on its own
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    cold = []
    for _ in range(args.steps):
        flush.fill_(1)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        step()
        b.record()
        cold.append((a, b))
    torch.cuda.synchronize()
    cold_ms = statistics.median(a.elapsed_time(b) for a, b in cold)
    del flush

    if args.copy_calib_mib:
        n = args.copy_calib_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()

    n_req = rows // case.qrows
    toks_cached = int(case.seq_lens.view(n_req, case.qrows)[:, -1].to(torch.int64).sum())
    from qmla.synth import algorithmic_bytes
    call_bytes = algorithmic_bytes(case)
    k_bytes = kernel_bytes(case)
    value = rows / (ms / 1e3)
    gbps = call_bytes / (ms / 1e3) / 1e9
    k_gbps = k_bytes / (part_ms / 1e3) / 1e9
    traffic = measured_traffic(args.workload)

    # the warp-specialized kernel's fp8 score path serves fp8 + log8 rows, d_c 512, rope 64: one latent
    # group with at most 32 rows per workgroup (a request's heads split over up to 4 workgroups), or
    # GLA-g2 with at most 48 rows per group
    ws_rows = case.qrows * case.heads // case.groups
    ws_fp8 = (case.kv == "fp8" and case.rms_mode == "log8" and case.d_c // case.groups in (512, 256)
              and case.rope_w == 64
              and (ws_rows <= 48 if case.groups == 2 else
                   any(case.heads % hs == 0 and ws_rows // hs <= 32 for hs in range(1, 5))))
    cpu = cpu_small = None
    if not args.no_cpu:
        cpu = cpu_baseline(case, args.cpu_every or CPU_EVERY.get(args.workload, 2), args.cpu_budget)
        if args.workload == "fp8_b128":
            cpu_small = cpu_reference_small()

    if spec[0] == "lognormal":
        ctx = f"lognormal median {spec[1]} sigma {spec[2]} clipped [{spec[3]}, {spec[4]}]"
    elif spec[0] == "fixed":
        ctx = f"{spec[1]} each"
    else:
        ctx = f"uniform [{spec[1]}, {spec[2]}]"
    res = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8+fp16" if ws_fp8 else "bf16",
        "storage": (("e4m3 latent/rope + u8 log8 rms; scores on the fp8 MFMAs (cache bytes as stored, query as "
                     "e4m3 hi+lo, 8 significant bits), P.V on the fp16 MFMAs (V exact, P with 11 significant "
                     "bits), fp32 accumulate and softmax")
                    if ws_fp8 else
                    "e4m3 latent/rope + u8 log8 rms; bf16 MFMA operands, fp32 accumulate and softmax"
                    if case.kv == "fp8" else "bf16 cache; bf16 MFMA operands, fp32 accumulate and softmax"),
        "data": "synthetic",
        "config": {"workload": f"mla_decode_{args.workload}", "batch": n_req, "rows": rows, "heads": H,
                   "d_c": case.d_c, "d_r": case.rope_w, "page_size": case.page_size, "kv": case.kv,
                   "rms": case.rms_mode, "ctx": ctx, "cached_tokens": toks_cached, "qrows": case.qrows,
                   "groups": case.groups, "split": f"fixed {splits} + combine" if splits else "balanced", "row_bytes": case.row * (1 if case.kv == "fp8" else 2)},
        # the whole call (plan + decode + combine) against the HBM peak: the metric's GB/s
        "call_gbps": round(gbps, 1),
        "call_hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "decode_kernel_us": round(part_ms * 1e3, 2),
        "combine_us": round(comb_ms * 1e3, 2),
        "graph_ms_per_step": None if graph_ms is None else round(graph_ms, 4),
        "graph_calls_per_graph": GRAPH_CALLS,
        "graph_call_hbm_frac": None if graph_ms is None else round(call_bytes / (graph_ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
        "cold_l2_ms_per_call": round(cold_ms, 4),
        "settle_calls": settle_calls,
        "wall_s_timed": round(t_wall, 3),
        "roofline": {"bound": "hbm", "achieved": round(k_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(k_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": k_bytes},
        "cpu_baseline": cpu,
        # the CPU-runnable reference configuration (B 4 x 2048, bf16, 16-token pages), timed in full
        "cpu_reference_b4_ctx2048": cpu_small,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
