"""Plan and pair-layout objects of the HD Block-GEMM surface.

The reference planner (``oal_attention/hd_block_gemm.py:223-537``,
``hd_block_gemm_plan.py:84-713``) sizes Python wave loops, named buffers and
backend tokens for its cuBLAS/Triton schedule. Here the schedule lives inside
the HIP kernels (fixed token block, fused scans), so the plan only validates
geometry and records the caller's options: every field the caller reads
(``qwen_lora_experiment/attention/hd_runtime.py:95-116``) stays a readable
attribute, and ``requested_gradient_mask`` keeps its meaning for the autograd
boundary.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass, field
from math import ceil

import torch

_PRECISIONS = ("fp32_ieee", "bf16_tensorcore")
# Token block (chunk) of every HIP kernel, liboal_amd.so's oal_chunk_size().
KERNEL_TOKEN_BLOCK = 64


@dataclass(frozen=True)
class CanonicalPairLayout:
    """Lower-triangular row-major pair order p(r, c) = r(r+1)/2 + c, r >= c.

    Same order and multiplicities as ``hd_block_gemm_cache.py:105-121``.
    """

    head_dimension: int
    rows: tuple[int, ...]
    columns: tuple[int, ...]
    multiplicity: tuple[float, ...]
    layout_id: str

    @property
    def pair_count(self) -> int:
        return len(self.rows)


_LAYOUTS: dict[int, CanonicalPairLayout] = {}


def canonical_pair_layout(head_dimension: int) -> CanonicalPairLayout:
    if head_dimension not in _LAYOUTS:
        rows, cols = [], []
        for r in range(head_dimension):
            for c in range(r + 1):
                rows.append(r)
                cols.append(c)
        mult = tuple(1.0 if r == c else 2.0 for r, c in zip(rows, cols))
        digest = hashlib.sha256(f"tril-row-major:{head_dimension}".encode()).hexdigest()[:16]
        _LAYOUTS[head_dimension] = CanonicalPairLayout(
            head_dimension, tuple(rows), tuple(cols), mult, f"pairs-{head_dimension}-{digest}"
        )
    return _LAYOUTS[head_dimension]


@dataclass(frozen=True)
class HDParallelBlockPlan:
    """Frozen description of one Q/K/V geometry and the requested options."""

    batch_size: int
    query_heads: int
    key_value_heads: int
    sequence_length: int
    head_dimension: int
    value_dimension: int
    input_dtype: str
    device: str
    precision: str
    requested_gradient_mask: tuple[bool, bool, bool, bool, bool, bool]
    token_block: int
    feature_wave_blocks: int
    memory_budget_bytes: int | None
    model_residency_bytes: int
    options: tuple[tuple[str, object], ...]
    require_positive_denominator: bool = True
    requested_token_block: int | None = None
    feature_dimension: int = field(init=False)
    pair_count: int = field(init=False)
    number_blocks: int = field(init=False)
    gqa_ratio: int = field(init=False)
    pair_layout_id: str = field(init=False)
    plan_id: str = field(init=False)

    def __post_init__(self) -> None:
        d = self.head_dimension
        object.__setattr__(self, "pair_count", d * (d + 1) // 2)
        object.__setattr__(self, "feature_dimension", 1 + d + d * (d + 1) // 2)
        object.__setattr__(self, "number_blocks", ceil(self.sequence_length / self.token_block))
        object.__setattr__(self, "gqa_ratio", self.query_heads // self.key_value_heads)
        object.__setattr__(self, "pair_layout_id", canonical_pair_layout(d).layout_id)
        key = repr(
            (
                self.batch_size, self.query_heads, self.key_value_heads, self.sequence_length, d,
                self.value_dimension, self.input_dtype, self.device, self.precision,
                self.requested_gradient_mask, self.token_block, self.options,
            )
        )
        object.__setattr__(self, "plan_id", hashlib.sha256(key.encode()).hexdigest()[:24])

    @property
    def geometry(self) -> tuple[int, int, int, int, int, int]:
        return (
            self.batch_size, self.query_heads, self.key_value_heads,
            self.sequence_length, self.head_dimension, self.value_dimension,
        )

    def __getattr__(self, name: str):
        for key, value in object.__getattribute__(self, "options"):
            if key == name:
                return value
        raise AttributeError(name)


def build_hd_block_gemm_plan(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    token_block: int = 128,
    feature_wave_blocks: int | None = None,
    precision: str = "fp32_ieee",
    requested_gradient_mask: tuple[bool, bool, bool, bool, bool, bool],
    memory_budget_bytes: int | None = None,
    model_residency_bytes: int = 0,
    require_positive_denominator: bool = True,
    **options: object,
) -> HDParallelBlockPlan:
    """Validate one geometry and freeze the requested options.

    Accepts every selector keyword of the reference planner and keeps it as a
    plan attribute; the HIP kernels schedule themselves, so the selectors do
    not change the arithmetic. ``precision`` must be ``fp32_ieee`` or
    ``bf16_tensorcore`` (``hd_block_gemm.py:132-153``).
    """
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor) or t.ndim != 4:
            raise ValueError(f"{name} must be a rank-4 tensor")
    b, hq, n, d = q.shape
    hkv, dv = k.shape[1], v.shape[-1]
    if d > 64 or dv > 64:
        raise ValueError("HD Block-GEMM supports head and value dimensions up to 64")
    if hq % hkv:
        raise ValueError("query head count must be divisible by KV head count")
    if not isinstance(token_block, int) or isinstance(token_block, bool) or token_block < 1:
        raise ValueError("token_block must be a positive int")
    nb = ceil(n / token_block)
    if feature_wave_blocks is None:
        feature_wave_blocks = nb
    if not isinstance(feature_wave_blocks, int) or feature_wave_blocks < 1:
        raise ValueError("feature_wave_blocks must be a positive int")
    if feature_wave_blocks > nb:
        raise ValueError("feature_wave_blocks cannot exceed the number of blocks")
    # the kernels run one token block, KERNEL_TOKEN_BLOCK (the library's
    # oal_chunk_size()); the plan reports that block and its block count, and
    # keeps the caller's request (results do not depend on the block size;
    # feature_wave_blocks, at most the requested block count, is at most the
    # kernel's as well)
    if precision not in _PRECISIONS:
        raise ValueError(f"precision must be one of {_PRECISIONS}")
    mask = tuple(bool(x) for x in requested_gradient_mask)
    if len(mask) != 6:
        raise ValueError("requested_gradient_mask must have six entries")
    return HDParallelBlockPlan(
        batch_size=b,
        query_heads=hq,
        key_value_heads=hkv,
        sequence_length=n,
        head_dimension=d,
        value_dimension=dv,
        input_dtype=str(q.dtype).replace("torch.", ""),
        device=str(q.device),
        precision=precision,
        requested_gradient_mask=mask,
        token_block=KERNEL_TOKEN_BLOCK,
        feature_wave_blocks=feature_wave_blocks,
        memory_budget_bytes=memory_budget_bytes,
        model_residency_bytes=model_residency_bytes,
        options=tuple(sorted((k_, v_ if not isinstance(v_, list) else tuple(v_)) for k_, v_ in options.items())),
        require_positive_denominator=bool(require_positive_denominator),
        requested_token_block=token_block,
    )


__all__ = (
    "CanonicalPairLayout",
    "HDParallelBlockPlan",
    "build_hd_block_gemm_plan",
    "canonical_pair_layout",
)
