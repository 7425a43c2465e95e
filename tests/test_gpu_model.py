"""The Qwen-shaped OAL model (the model-step benchmark's architecture) on the GPU.

A reduced copy (2 layers, vocab 512, MLP 256; hidden 896 = 14 heads x 64,
2 KV heads as in the full model) runs one forward + backward on the GPU with
the HIP operator, and the same weights run on the CPU with the attention
replaced by the dense token-pair oracle (oracle/grouped_oracle.py dense_forward,
differentiable by autograd). In fp32 mode the loss and every LoRA gradient must
agree to rel-L2 1e-4 (fp32 GEMMs and the 1e-5 fp32 operator through two layers);
in bf16 mode (bf16 weights and activations, matrix-core operator) the loss must
agree to 2e-2 relative and every gradient must be finite.
"""

import copy

import pytest
import torch

from oracle import grouped_oracle as go

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


def _twin_pair(precision):
    from oal_amd.qwen_oal import QwenOALConfig, QwenOALModel

    cfg = QwenOALConfig(vocab_size=512, num_layers=2, intermediate_size=256, precision=precision)
    cpu = QwenOALModel(cfg, seed=0)
    gen = torch.Generator().manual_seed(5)
    for p in cpu.lora_parameters():
        if p.shape[1] == cfg.lora_rank:  # lora_b: nonzero so that LoRA reaches the forward
            p.data.copy_(torch.randn(p.shape, generator=gen) * 0.02)
    for layer in cpu.layers:
        attn = layer.attn

        def oracle_head_attention(q, k, v, attn=attn):
            out, _, _ = go.dense_forward(q, k, v, attn.dim_groups, attn.factor, scale=cfg.head_dim ** -0.5,
                                         kernel_eps=cfg.kernel_eps)
            return out

        attn.head_attention = oracle_head_attention
    gpu = copy.deepcopy(cpu)
    for layer in gpu.layers:
        del layer.attn.head_attention  # back to the HIP operator
    return cfg, cpu, gpu


def _loss_and_grads(model, tokens):
    from oal_amd.qwen_oal import causal_lm_loss

    loss = causal_lm_loss(model(tokens), tokens)
    loss.backward()
    return loss.detach(), [p.grad for p in model.lora_parameters()]


def test_qwen_oal_model_fp32_matches_cpu_twin():
    dev = _dev()
    cfg, cpu, gpu = _twin_pair("fp32_ieee")
    tokens = torch.randint(0, cfg.vocab_size, (2, 96), generator=torch.Generator().manual_seed(1))
    loss_c, grads_c = _loss_and_grads(cpu, tokens)
    loss_g, grads_g = _loss_and_grads(gpu.to(dev), tokens.to(dev))
    errs = [_rel(g, c) for g, c in zip(grads_g, grads_c)]
    print(f"fp32 model: loss {loss_g.item():.6f} vs {loss_c.item():.6f}, max LoRA grad rel-L2 {max(errs):.2e}")
    assert abs(loss_g.item() - loss_c.item()) <= 1e-5 * abs(loss_c.item())
    assert max(errs) <= 1e-4, errs


def test_qwen_oal_model_bf16_step_is_close_and_finite():
    from oal_amd.qwen_oal import train_step

    dev = _dev()
    cfg, cpu, gpu = _twin_pair("bf16_tensorcore")
    tokens = torch.randint(0, cfg.vocab_size, (2, 160), generator=torch.Generator().manual_seed(2))
    loss_c, _ = _loss_and_grads(cpu, tokens)
    gpu = gpu.to(dev).cast_parameters_(torch.bfloat16)
    opt = torch.optim.AdamW(gpu.lora_parameters(), lr=1e-4)
    loss_g = train_step(gpu, tokens.to(dev), opt)
    grads = [p.grad for p in gpu.lora_parameters()]
    print(f"bf16 model step: loss {loss_g.item():.5f} vs fp32 CPU twin {loss_c.item():.5f}")
    assert abs(loss_g.item() - loss_c.item()) <= 2e-2 * abs(loss_c.item())
    assert all(g is not None and torch.isfinite(g.float()).all() for g in grads)
    assert any(g.float().abs().sum() > 0 for g in grads)
