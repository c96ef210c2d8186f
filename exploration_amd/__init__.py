"""MI355X (gfx950) drop-in for the attention operators of Stack (``st.ops``).

Public entry points (same signatures as the reference's ``st.ops``):

* ``dense_attention`` / ``triton_supported`` (``st/ops/attention.py:142-176``)
* ``sparse_attention`` / ``TensorPages`` (``st/ops/sparse.py:75-174``)

plus ``PagedKV`` (page-table KV cache), the internal equivalents
``dense_hip``, ``block_scores``, ``select_blocks``, ``sparse_pop`` and
``launch_report``. The kernels live in ``libst_attn.so`` (C ABI in
``include/st_attn.h``); importing the package does not load it.
"""
from .attention import dense_attention, dense_hip, hip_supported, triton_supported
from .sparse import PagedKV, TensorPages, block_scores, select_blocks, sparse_attention, sparse_pop


def launch_report():
    """Operator-level records (kernel = operator, with dtype, head_dim and
    block size) followed by the library's per-kernel launch records (tiles,
    waves, LDS buffers, registers, LDS bytes, workgroups; the reference's
    ``st/ops/kernels/launch.py:52-56`` fields)."""
    from . import _lib, attention, sparse
    native = _lib.native_launch_report() if _lib._lib is not None else []
    return attention.launch_report() + sparse.launch_report() + native


__all__ = ["dense_attention", "dense_hip", "hip_supported", "triton_supported", "sparse_attention",
           "TensorPages", "PagedKV", "block_scores", "select_blocks", "sparse_pop", "launch_report"]
__version__ = "0.1.0"
