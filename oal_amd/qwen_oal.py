"""Qwen2-shaped decoder with OAL grouped quadratic attention in every layer.

The benchmark's model-step workload (random init, no checkpoint is loaded): hidden
896, 24 layers, 14 query / 2 KV heads of dimension 64, SwiGLU MLP 4864, vocab
151936, RMSNorm (eps 1e-6), rotary embeddings (theta 1e6, rotate-half form),
tied input/output embeddings; LoRA of rank 16 on the q/k/v/o projections and a
trainable fp32 OAL factor per layer ([14, 45], one packed lower-triangular factor
per query head, as the reference's kernel parameter bank holds one nn.Parameter
per head, qwen_lora_experiment/kernel_parameters.py:115-128), all other weights
frozen; each decoder layer runs under non-reentrant activation checkpointing, so
the backward recomputes the attention forward. The training step therefore runs
the operator's coefficient-gradient kernels, as the reference's does.

It mirrors the reference adapter chain around the operator:
* the Qwen projection / RoPE shell (qwen_lora_experiment/attention/common.py:375-415,
  rotary 510-596): q, k, v are projected, reshaped head-first [B, H, N, 64], rotated;
* GroupedQuadraticQwenAttentionAdapter.head_attention (attention/grouped.py:182-258)
  -> grouped_quadratic_hd_attention (:88-122): the layer's live [14, 45] fp32 factor
  and [14, 64] int32 dim groups go to the HD family with scale 64^-1/2 and the
  layer's kernel epsilon, through a per-layer cached preparation as
  attention/hd_runtime.py:38-86 does (prepare once, run per call);
* activation checkpointing of each decoder layer (model_setup.py:621-665).

The attention runs in liboal_amd.so (precision "bf16_tensorcore": bf16 operands,
fp32 accumulation on the matrix cores); the projections, norms and MLP are torch.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn
from torch.utils.checkpoint import checkpoint

from .hd_block_gemm_adapters import prepare_grouped_hd_block_gemm, run_prepared_grouped_hd_block_gemm


@dataclass(frozen=True)
class QwenOALConfig:
    vocab_size: int = 151936
    hidden_size: int = 896
    intermediate_size: int = 4864
    num_layers: int = 24
    num_heads: int = 14
    num_kv_heads: int = 2
    head_dim: int = 64
    rope_theta: float = 1_000_000.0
    rms_eps: float = 1e-6
    lora_rank: int = 16
    lora_alpha: float = 32.0
    kernel_eps: float = 1e-6
    group_sizes: tuple = (2, 4, 6, 8, 10, 10, 12, 12)
    precision: str = "bf16_tensorcore"
    checkpointing: bool = True


class LoRALinear(nn.Module):
    """Frozen base projection plus a trainable rank-r update B A (B starts at zero)."""

    def __init__(self, in_features: int, out_features: int, *, bias: bool, rank: int, alpha: float):
        super().__init__()
        self.base = nn.Linear(in_features, out_features, bias=bias)
        self.base.requires_grad_(False)
        self.lora_a = nn.Parameter(torch.empty(rank, in_features))
        self.lora_b = nn.Parameter(torch.zeros(out_features, rank))
        nn.init.kaiming_uniform_(self.lora_a, a=math.sqrt(5))
        self.scaling = alpha / rank

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.base(x) + F.linear(F.linear(x, self.lora_a), self.lora_b) * self.scaling


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim), requires_grad=False)
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


def rotary_tables(seq_len: int, head_dim: int, theta: float, device, dtype):
    """cos, sin [N, head_dim] of the rotate-half rotary embedding."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
    t = torch.arange(seq_len, device=device, dtype=torch.float32)
    freqs = torch.outer(t, inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B, H, N, D]: x cos + rotate_half(x) sin."""
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos + rot * sin


def seeded_layer_groups(cfg: QwenOALConfig, gen: torch.Generator) -> torch.Tensor:
    """[Hq, 64] int32 labels: per head, the uneven group sizes over a seeded permutation."""
    rows = []
    for _ in range(cfg.num_heads):
        perm = torch.randperm(cfg.head_dim, generator=gen)
        lab = torch.empty(cfg.head_dim, dtype=torch.int32)
        start = 0
        for g, size in enumerate(cfg.group_sizes):
            lab[perm[start:start + size]] = g
            start += size
        rows.append(lab)
    return torch.stack(rows)


def seeded_layer_factor(cfg: QwenOALConfig, gen: torch.Generator) -> torch.Tensor:
    """[Hq, (G+1)(G+2)/2] fp32 packed lower-triangular factor L (row-major), unit-scale diagonal.

    kappa = ||[1, z] L||^2 + eps is positive for any inputs, so every denominator is.
    """
    side = len(cfg.group_sizes) + 1
    rows = []
    for _ in range(cfg.num_heads):
        low = torch.tril(torch.randn((side, side), generator=gen) * 0.15)
        low.diagonal().copy_(0.5 + 0.5 * torch.rand(side, generator=gen))
        r, c = torch.tril_indices(side, side)
        rows.append(low[r, c])
    return torch.stack(rows).float()


class OALAttention(nn.Module):
    def __init__(self, cfg: QwenOALConfig, layer_id: int, gen: torch.Generator):
        super().__init__()
        self.cfg = cfg
        self.layer_id = layer_id
        hq, hkv, d = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
        lora = dict(rank=cfg.lora_rank, alpha=cfg.lora_alpha)
        self.q_proj = LoRALinear(cfg.hidden_size, hq * d, bias=True, **lora)
        self.k_proj = LoRALinear(cfg.hidden_size, hkv * d, bias=True, **lora)
        self.v_proj = LoRALinear(cfg.hidden_size, hkv * d, bias=True, **lora)
        self.o_proj = LoRALinear(hq * d, cfg.hidden_size, bias=False, **lora)
        self.register_buffer("dim_groups", seeded_layer_groups(cfg, gen), persistent=True)
        # trainable, kept in fp32 whatever the model's compute dtype
        self.factor = nn.Parameter(seeded_layer_factor(cfg, gen))
        self.kernel_eps = cfg.kernel_eps
        # "triton": the configured fast precision (the matrix-core kernels by
        # default); "reference": the fp32 kernels, selected for a quality
        # evaluation by oal_amd.grouped_sessions.grouped_quadratic_reference_session
        # (the reference adapter's _grouped_execution, attention/grouped.py:182-258)
        self._grouped_execution = "triton"
        self._prepared = {}

    def execution_precision(self) -> str:
        """Planner precision of the current execution mode."""
        if self._grouped_execution == "triton":
            return self.cfg.precision
        if self._grouped_execution == "reference":
            return "fp32_ieee"
        from .grouped_sessions import GroupedQuadraticAttentionError

        raise GroupedQuadraticAttentionError(
            f"grouped quadratic operator layer={self.layer_id}: adapter has an invalid grouped execution mode")

    def head_attention(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """One grouped call with the layer's live factor, cached per call signature."""
        precision = self.execution_precision()
        sig = (tuple(q.shape), q.dtype, str(q.device), torch.is_grad_enabled(), q.requires_grad,
               k.requires_grad, v.requires_grad, self.factor.requires_grad, precision)
        prepared = self._prepared.get(sig)
        if prepared is None:
            prepared = prepare_grouped_hd_block_gemm(
                q, k, v, self.dim_groups, self.factor, scale=self.cfg.head_dim ** -0.5,
                kernel_eps=self.kernel_eps, precision=precision,
            )
            self._prepared[sig] = prepared
        out, _, _ = run_prepared_grouped_hd_block_gemm(prepared, q, k, v, self.factor)
        return out

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        b, n, _ = x.shape
        hq, hkv, d = self.cfg.num_heads, self.cfg.num_kv_heads, self.cfg.head_dim
        q = self.q_proj(x).view(b, n, hq, d).transpose(1, 2)
        k = self.k_proj(x).view(b, n, hkv, d).transpose(1, 2)
        v = self.v_proj(x).view(b, n, hkv, d).transpose(1, 2)
        q = apply_rotary(q, cos, sin).contiguous()
        k = apply_rotary(k, cos, sin).contiguous()
        o = self.head_attention(q, k, v.contiguous())
        return self.o_proj(o.transpose(1, 2).reshape(b, n, hq * d))


class MLP(nn.Module):
    def __init__(self, cfg: QwenOALConfig):
        super().__init__()
        self.gate = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.up = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.down = nn.Linear(cfg.intermediate_size, cfg.hidden_size, bias=False)
        self.requires_grad_(False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down(F.silu(self.gate(x)) * self.up(x))


class DecoderLayer(nn.Module):
    def __init__(self, cfg: QwenOALConfig, layer_id: int, gen: torch.Generator):
        super().__init__()
        self.input_norm = RMSNorm(cfg.hidden_size, cfg.rms_eps)
        self.attn = OALAttention(cfg, layer_id, gen)
        self.post_norm = RMSNorm(cfg.hidden_size, cfg.rms_eps)
        self.mlp = MLP(cfg)

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.input_norm(x), cos, sin)
        return x + self.mlp(self.post_norm(x))


class QwenOALModel(nn.Module):
    def __init__(self, cfg: QwenOALConfig, seed: int = 0):
        super().__init__()
        self.cfg = cfg
        torch.manual_seed(seed)
        gen = torch.Generator().manual_seed(seed)
        self.embed = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.embed.requires_grad_(False)
        self.layers = nn.ModuleList([DecoderLayer(cfg, i, gen) for i in range(cfg.num_layers)])
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_eps)
        self._init_weights()

    def _init_weights(self) -> None:
        for name, p in self.named_parameters():
            if name.endswith("lora_a") or name.endswith("lora_b") or "norm" in name:
                continue
            if p.ndim == 2:
                nn.init.normal_(p, std=0.02)
            else:
                nn.init.zeros_(p)

    def cast_parameters_(self, dtype: torch.dtype) -> "QwenOALModel":
        """Casts every parameter except the OAL factors (they stay fp32, as the
        reference's kernel bank keeps them; the dim-group buffers stay int32)."""
        for name, p in self.named_parameters():
            if not name.endswith("attn.factor"):
                p.data = p.data.to(dtype)
        return self

    def load_group_asset(self, asset) -> "QwenOALModel":
        """Sets the dim groups, factors and kernel epsilon of the asset's layers from an
        :class:`oal_amd.group_assets.OALGroupAsset` (the reference's released grouping)."""
        for layer_id in asset.layer_ids_zero_based:
            attn = self.layers[layer_id].attn
            attn.dim_groups = asset.dim_groups_for_layer(layer_id).to(attn.dim_groups.device)
            with torch.no_grad():
                attn.factor.copy_(asset.packed_grouped_factor_for_layer(layer_id))
            attn.kernel_eps = asset.epsilon
            attn._prepared.clear()
        return self

    def lora_parameters(self):
        return [p for n, p in self.named_parameters() if n.endswith("lora_a") or n.endswith("lora_b")]

    def oal_parameters(self):
        """The per-layer OAL factors (trainable, fp32)."""
        return [layer.attn.factor for layer in self.layers]

    def optimizer(self, lora_lr: float = 1e-4, kernel_lr: float = 1e-3) -> torch.optim.Optimizer:
        """AdamW with separate LoRA and OAL-factor groups (the reference's pilot optimizer
        keeps the two learning rates apart, qwen_lora_experiment/model_setup.py:462-560)."""
        return torch.optim.AdamW([
            {"params": self.lora_parameters(), "lr": lora_lr},
            {"params": self.oal_parameters(), "lr": kernel_lr},
        ])

    def forward(self, tokens: torch.Tensor) -> torch.Tensor:
        """tokens [B, N] -> logits [B, N, vocab] (output head tied to the embedding)."""
        x = self.embed(tokens)
        cos, sin = rotary_tables(tokens.shape[1], self.cfg.head_dim, self.cfg.rope_theta, x.device, x.dtype)
        for layer in self.layers:
            if self.cfg.checkpointing and torch.is_grad_enabled():
                x = checkpoint(layer, x, cos, sin, use_reentrant=False)
            else:
                x = layer(x, cos, sin)
        return F.linear(self.norm(x), self.embed.weight)


def causal_lm_loss(logits: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
    """Next-token cross entropy, computed in fp32."""
    return F.cross_entropy(logits[:, :-1].float().reshape(-1, logits.shape[-1]), tokens[:, 1:].reshape(-1))


def train_step(model: QwenOALModel, tokens: torch.Tensor, optimizer: torch.optim.Optimizer) -> torch.Tensor:
    """One LoRA training step: forward, loss, backward, optimizer update. Returns the loss."""
    optimizer.zero_grad(set_to_none=True)
    loss = causal_lm_loss(model(tokens), tokens)
    loss.backward()
    optimizer.step()
    return loss.detach()


__all__ = ("QwenOALConfig", "QwenOALModel", "causal_lm_loss", "train_step", "rotary_tables", "apply_rotary")
