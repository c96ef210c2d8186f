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
    from . import attention, sparse
    return attention.launch_report() + sparse.launch_report()


__all__ = ["dense_attention", "dense_hip", "hip_supported", "triton_supported", "sparse_attention",
           "TensorPages", "PagedKV", "block_scores", "select_blocks", "sparse_pop", "launch_report"]
__version__ = "0.1.0"
