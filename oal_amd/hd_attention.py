"""Public causal OAL entry point for the HD family (reference oal_attention/hd_attention.py)."""

from .hd_block_gemm_adapters import grouped_causal_attention

__all__ = ("grouped_causal_attention",)
