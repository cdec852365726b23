"""Pins the oracle's byte arithmetic: e4m3fn decode/encode, bf16 rounding and the log8 rms code.

The e4m3fn and bf16 checks compare against torch's own float8_e4m3fn / bfloat16 conversions (an
independent implementation of the same OCP / IEEE rounding rules); the log8 checks use the known
answers of the reference (qwen_mla/mla_impl.py:126-132: range [0.125, 8], about 0.8% worst-case
relative error) and properties the code must have (monotone, round-trip idempotent, nearest code).
"""
from __future__ import annotations

import json
import math
import pathlib

import numpy as np
import pytest
import torch

from oracle import mla_oracle as ora

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
F8 = getattr(torch, "float8_e4m3fn", None)
pytestmark = pytest.mark.skipif(F8 is None, reason="torch without float8_e4m3fn")


def test_e4m3_decode_matches_torch_all_codes():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(F8).float().numpy()
    got = ora.e4m3_decode(codes.numpy())
    nan = np.isnan(ref)
    assert np.array_equal(nan, np.isnan(got))
    assert nan.sum() == 2                       # 0x7F and 0xFF
    assert np.array_equal(ref[~nan], got[~nan])


def test_e4m3_known_answers():
    ka = {1.0: 0x38, 2.0: 0x40, -2.0: 0xC0, 448.0: 0x7E, -448.0: 0xFE, 2.0 ** -9: 0x01,
          2.0 ** -6: 0x08, 0.0: 0x00, 1.125: 0x39, 240.0: 0x77}
    x = np.array(list(ka), dtype=np.float32)
    got = ora.e4m3_encode(x)
    assert [int(v) for v in got] == [ka[k] for k in ka]
    # ties round to even: 1 + 1/16 sits halfway between 1 (even mantissa) and 1.125
    assert int(ora.e4m3_encode(np.array([1.0625], np.float32))[0]) == 0x38
    assert int(ora.e4m3_encode(np.array([1.1875], np.float32))[0]) == 0x3A
    # subnormal tie: 1.5 * 2^-9 -> 2 * 2^-9 (even)
    assert int(ora.e4m3_encode(np.array([1.5 * 2.0 ** -9], np.float32))[0]) == 0x02


def _e4m3_probe_values(seed: int) -> np.ndarray:
    """Every representable value, every midpoint between neighbours (the tie cases), values a hair
    either side of each midpoint, random normals over many octaves and the saturation region."""
    reps = np.unique(np.abs(ora.E4M3_TABLE[~np.isnan(ora.E4M3_TABLE)]).astype(np.float64))
    mids = (reps[:-1] + reps[1:]) / 2
    eps = np.concatenate([mids * (1 + 2.0 ** -20), mids * (1 - 2.0 ** -20)])
    rng = np.random.default_rng(seed)
    rnd = rng.standard_normal(200_000) * np.exp2(rng.uniform(-12, 9, 200_000))
    v = np.concatenate([reps, mids, eps, rnd, np.linspace(400, 448, 997)])
    v = np.concatenate([v, -v]).astype(np.float32)
    return np.clip(v, -448.0, 448.0)


def test_e4m3_encode_matches_torch():
    x = _e4m3_probe_values(0)
    ref = torch.from_numpy(x).to(F8).view(torch.uint8).numpy()
    got = ora.e4m3_encode(x)
    bad = np.nonzero(ref != got)[0]
    assert bad.size == 0, [(float(x[i]), int(ref[i]), int(got[i])) for i in bad[:8]]


def test_e4m3_encode_decode_roundtrip_all_codes():
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF, 0x80)], dtype=np.uint8)
    assert np.array_equal(ora.e4m3_encode(ora.e4m3_decode(codes)), codes)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(100_000) * np.exp2(rng.uniform(-30, 30, 100_000))).astype(np.float32)
    # exact ties: bf16 value + half an ulp
    base = torch.from_numpy(x[:1000]).bfloat16().float().numpy()
    ulp = np.abs(base) * 2.0 ** -8
    x = np.concatenate([x, base + ulp / 2, base - ulp / 2, np.array([0.0, -0.0, 1e-40, 3.4e38], np.float32)])
    x = x.astype(np.float32)
    ref = torch.from_numpy(x).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ora.f32_to_bf16_bits(x), ref)
    assert np.array_equal(ora.bf16_bits_to_f32(ref), torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_log8_known_answers():
    dec = ora.log8_decode(np.arange(256))
    assert dec[0] == np.float32(0.125) and dec[255] == np.float32(8.0)
    assert abs(float(dec[128]) - 2.0 ** (-3 + 128 * 6 / 255)) < 1e-6
    # 1.0: (0 + 3) * 42.5 = 127.5, a tie: round-half-even -> 128
    assert int(ora.log8_encode(np.array([1.0], np.float32))[0]) == 128
    enc = ora.log8_encode(np.array([0.125, 8.0, 1e-3, 1e3, 0.0, -1.0], np.float32))
    assert enc.tolist() == [0, 255, 0, 255, 0, 0]


def test_log8_properties():
    codes = np.arange(256)
    dec = ora.log8_decode(codes)
    assert np.all(np.diff(dec) > 0)                                   # monotone
    assert np.array_equal(ora.log8_encode(dec), codes.astype(np.uint8))  # idempotent round trip
    rng = np.random.default_rng(2)
    r = np.exp2(rng.uniform(-3, 3, 100_000)).astype(np.float32)
    back = ora.log8_decode(ora.log8_encode(r))
    rel = np.abs(back / r - 1)
    half_step = 2.0 ** (3.0 / 255) - 1                                # 0.819%
    assert rel.max() <= half_step * 1.0001
    assert rel.max() > 0.8e-2                                         # the quoted ~0.8% is reached
    # the chosen code is the nearest one in log space
    lg = np.log2(r.astype(np.float64))
    code = ora.log8_encode(r).astype(np.float64)
    assert np.all(np.abs(lg - (-3 + code * 6 / 255)) <= 3 / 255 + 1e-6)


def test_golden_known_answers():
    """The committed fixture (tests/golden/codes.json, written by tests/golden/make_codes.py from
    torch's conversions and the reference's docstring constants) agrees with the oracle."""
    g = json.loads((GOLDEN / "codes.json").read_text())
    x = np.array(g["e4m3_inputs"], np.float32)
    assert ora.e4m3_encode(x).tolist() == g["e4m3_codes"]
    assert [float(v) if not math.isnan(v) else None for v in ora.e4m3_decode(np.arange(256))] == \
        [v for v in g["e4m3_values"]]
    r = np.array(g["log8_inputs"], np.float32)
    assert ora.log8_encode(r).tolist() == g["log8_codes"]
    b = np.array(g["bf16_inputs"], np.float32)
    assert ora.f32_to_bf16_bits(b).tolist() == g["bf16_bits"]
