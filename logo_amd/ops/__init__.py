"""Selected-query full-attention operators for LoGo on MI355X.

Same public names as logo/ops/__init__.py:14-23, plus the local/dense
branches that run on the same HIP kernels.
"""

from .common import (
    SelInfo,
    assert_close,
    build_selection,
    compute_q_start_blk,
    get_abs_err,
    get_err_ratio,
    prepare_chunk_indices,
)
from .dense import sdpa_causal_ref, sq_full_attn_dense_ref
from .sq_attn import dense_causal_attn, sq_full_attn, swa_attn

__all__ = [
    "sq_full_attn",
    "sq_full_attn_dense_ref",
    "sdpa_causal_ref",
    "build_selection",
    "SelInfo",
    "get_abs_err",
    "get_err_ratio",
    "assert_close",
    "prepare_chunk_indices",
    "compute_q_start_blk",
    "swa_attn",
    "dense_causal_attn",
]
