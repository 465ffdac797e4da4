"""icsa_hip: MI355X (gfx950) in-context sparse attention, the reference package's API with a
HIP backend.

The package has its own name so that the reference's ``in_context_sparse_attention``
package can import it (its ``backend='hip'`` branch).  It mirrors that package's
``__init__.py`` (``Backend``,
``editing_sparse_attention``, ``editing_sparse_attention_tilelang``) and adds the kernel-host
functions of the HIP backend.  Importing does not load the native library; the first GPU
call does, and fails loudly if ``libicsa.so`` has not been built.
"""
from .editing_sparse_attention import (  # noqa: F401
    Backend,
    derived_sizes,
    editing_sparse_attention,
    editing_sparse_attention_tilelang,
)
from .hip_host import (  # noqa: F401
    IcsaArgumentError,
    flash_attn_func,
    gather_kv,
    pool,
    SparsePiecewiseAttn1stIntervalsFunction,
    sparse_piecewise_attn_1st_intervals,
    sparse_piecewise_attn_1st_intervals_bwd_hip,
    sparse_piecewise_attn_1st_intervals_fwd_hip,
    sparse_piecewise_attn_1st_intervals_hip,
    sparse_piecewise_attn_tilelang_hosttopk_hip,
)

__all__ = [
    'Backend',
    'editing_sparse_attention',
    'editing_sparse_attention_tilelang',
    'sparse_piecewise_attn_1st_intervals_hip',
    'sparse_piecewise_attn_tilelang_hosttopk_hip',
    'sparse_piecewise_attn_1st_intervals',
    'SparsePiecewiseAttn1stIntervalsFunction',
    'sparse_piecewise_attn_1st_intervals_fwd_hip',
    'sparse_piecewise_attn_1st_intervals_bwd_hip',
    'flash_attn_func',
    'derived_sizes',
    'IcsaArgumentError',
]
