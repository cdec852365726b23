"""Writes tests/golden/codes.json: byte-format vectors produced by torch's own conversions.

* e4m3fn: `x.to(torch.float8_e4m3fn)` of clamped float32 inputs (the FP8 row writer's call,
  qwen_mla/mla_impl.py:329-332) and the float value of every code.
* log8: the writer's float32 torch arithmetic (qwen_mla/mla_impl.py:333-336) on rms values at and
  around code boundaries.
* bf16: `x.to(torch.bfloat16)` bit patterns, including exact ties.

Run from the repository root: python tests/golden/make_codes.py
"""
from __future__ import annotations

import json
import math
import pathlib

import torch

OUT = pathlib.Path(__file__).resolve().parent / "codes.json"


def main() -> None:
    g = torch.Generator().manual_seed(1234)
    f8 = torch.float8_e4m3fn
    x = torch.cat([torch.randn(512, generator=g) * torch.exp2(torch.rand(512, generator=g) * 20 - 11),
                   torch.tensor([0.0, 1.0625, 1.1875, 448.0, -448.0, 2.0 ** -9, 1.5 * 2.0 ** -9, 464.0 - 1e-3,
                                 240.0, 0.5 * 2.0 ** -9])]).float().clamp(-448.0, 448.0)
    codes = x.to(f8).view(torch.uint8)
    vals = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(f8).float()
    lo, hi = -3.0, 3.0
    k = torch.arange(256, dtype=torch.float64)
    edges = torch.exp2(lo + (k + 0.5) * (hi - lo) / 255)      # boundaries between codes
    r = torch.cat([torch.exp2(torch.rand(400, generator=g, dtype=torch.float64) * 8 - 4),
                   edges * (1 + 1e-5), edges * (1 - 1e-5), torch.tensor([1.0, 0.125, 8.0, 1e-3, 1e3, 0.0])]).float()
    code = (r.clamp_min(1e-30).log2() - lo) * (255.0 / (hi - lo))
    log8 = code.round_().clamp_(0, 255).to(torch.uint8)
    b = torch.randn(256, generator=g) * torch.exp2(torch.rand(256, generator=g) * 40 - 20)
    bb = b.bfloat16().float()
    b = torch.cat([b, bb * (1 + 2.0 ** -9), bb * (1 - 2.0 ** -9)]).float()
    bits = b.bfloat16().view(torch.int16).to(torch.int32) & 0xFFFF
    doc = {
        "e4m3_inputs": [float(v) for v in x.tolist()],
        "e4m3_codes": [int(v) for v in codes.tolist()],
        "e4m3_values": [None if math.isnan(v) else float(v) for v in vals.tolist()],
        "log8_inputs": [float(v) for v in r.tolist()],
        "log8_codes": [int(v) for v in log8.tolist()],
        "bf16_inputs": [float(v) for v in b.tolist()],
        "bf16_bits": [int(v) for v in bits.tolist()],
    }
    OUT.write_text(json.dumps(doc))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
