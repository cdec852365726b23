"""qmla: MI355X-native (gfx950) absorbed-MLA latent-KV decode attention.

Host side in Python on PyTorch-ROCm; the compute runs in hand-written HIP kernels of libqmla.so
behind the C ABI of include/qmla.h. See decode.py for the two call surfaces.
"""
from . import backend, layout  # noqa: F401
from .cache import cache_write, do_kv_cache_update, gather_cache  # noqa: F401
from ._lib import lib  # noqa: F401
from .decode import Workspace, build_params, decode_attention_fwd, forward, workspace_bytes  # noqa: F401
from .prep import k_gain, mla_decode_prep, partial_rope_table  # noqa: F401

__all__ = ["backend", "layout", "lib", "cache_write", "do_kv_cache_update", "gather_cache", "decode_attention_fwd", "forward", "build_params", "workspace_bytes", "Workspace",
           "mla_decode_prep", "k_gain", "partial_rope_table"]
