"""oal_amd: MI355X (gfx950) HIP implementation of OAL grouped quadratic attention.

Drop-in for the reference ``oal_attention`` operator surface:

* ``oal_amd.oal_attention`` (``oal_attention.oal_attention``)
* ``oal_amd.hd_attention.grouped_causal_attention``
* ``oal_amd.hd_block_gemm_adapters.prepare_grouped_hd_block_gemm`` /
  ``run_prepared_grouped_hd_block_gemm``
* ``oal_amd.hd_block_gemm_autograd._HDParallelBlockGemmFunction``
* ``oal_amd.hd_block_gemm.build_hd_block_gemm_plan`` / ``canonical_pair_layout``

The arithmetic runs in ``liboal_amd.so`` (hand-written HIP kernels behind the
C ABI in ``include/oal_amd.h``); PyTorch supplies device memory and streams.
"""

from .grouped_quadratic import oal_attention

__all__ = ["oal_attention"]
