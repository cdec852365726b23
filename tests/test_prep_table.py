"""qmla.prep.partial_rope_table on the CPU: the cos/sin table of the kept rope subspaces
(qwen_mla/partial_rope.py:52-76).

* The property the reference states for its float32 convention (partial_rope.py:61-64): the
  partial table is bit-identical to the matching columns of the full-width table (torch.equal), for
  contiguous, strided and shuffled keep lists.
* Against the oracle's table (cos / sin of the float32 angle evaluated in float64 and rounded once):
  within a few float32 ulps of the angle's own rounding.
* Closed forms: row 0 is [1 ... 1 | 0 ... 0]; cos^2 + sin^2 = 1 to float32 rounding; subspace i turns
  at theta^(-2 i / 64) radians per position.
"""
import math

import numpy as np
import pytest
import torch

from oracle import mla_oracle as ora
from qmla.prep import partial_rope_table


@pytest.mark.parametrize("keep", [list(range(29)), list(range(0, 32, 2)), [31, 0, 17, 5, 9], list(range(32))])
def test_partial_table_is_the_full_table_sliced(keep):
    full = partial_rope_table(list(range(32)), 64, 1e7, 4096)
    part = partial_rope_table(keep, 64, 1e7, 4096)
    cols = keep + [32 + k for k in keep]
    assert part.dtype == torch.float32 and part.shape == (4096, 2 * len(keep))
    assert torch.equal(part, full[:, cols])


def test_against_the_oracle_table():
    """The oracle rounds each inverse frequency once from float64; torch's float32 pow (the
    reference's arithmetic, which the table follows bit for bit) may land one ulp away, and the
    angle t * inv carries that ulp times t, then one ulp of the float32 angle when the two products
    round apart. So the bound grows with the position: t * ulp(inv) + ulp(angle) plus a few ulps of
    cos / sin themselves."""
    keep = [0, 3, 7, 12, 20, 28, 31]
    n = 65536
    t = partial_rope_table(keep, 64, 1e7, n).numpy().astype(np.float64)
    o = ora.partial_rope_table(keep, 64, 1e7, n).astype(np.float64)
    inv = np.array([1e7 ** (-2 * k / 64) for k in keep])
    ulp = np.spacing(inv.astype(np.float32)).astype(np.float64)
    pos = np.arange(n, dtype=np.float64)[:, None]
    dang = pos * ulp + np.spacing((pos * inv).astype(np.float32)).astype(np.float64)
    bound = np.concatenate([dang, dang], axis=1) + 4 * float(np.finfo(np.float32).eps)
    assert (np.abs(t - o) <= bound).all()
    # most positions see the same angle: the two agree to float32 rounding there
    assert np.median(np.abs(t - o)) <= 2 * float(np.finfo(np.float32).eps)


def test_closed_forms():
    t = partial_rope_table(list(range(32)), 64, 1e6, 3000).double()
    assert torch.equal(t[0, :32], torch.ones(32, dtype=torch.float64)) and torch.equal(t[0, 32:], torch.zeros(32, dtype=torch.float64))
    assert (t[:, :32] ** 2 + t[:, 32:] ** 2 - 1).abs().max().item() < 1e-6
    # position 1: angle = inverse frequency of each subspace
    inv = [1e6 ** (-2 * i / 64) for i in range(32)]
    assert max(abs(math.atan2(t[1, 32 + i].item(), t[1, i].item()) - inv[i]) for i in range(32)) < 1e-6
