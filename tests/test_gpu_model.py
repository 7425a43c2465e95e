"""The Qwen-shaped OAL model (the model-step benchmark's architecture) on the GPU.

The full configuration-4 step (24 layers, vocab 151936, B=4, N=4096, bf16, LoRA
r16 and trainable OAL factors) runs once; its properties are checked: the loss at
initialization is finite and near ln(151936) = 11.93 (random-init logits), and
every LoRA-B and OAL-factor gradient is finite and nonzero.

A reduced copy (2 layers, vocab 512, MLP 256; hidden 896 = 14 heads x 64,
2 KV heads as in the full model) runs one forward + backward on the GPU with
the HIP operator, and the same weights run on the CPU with the attention
replaced by the dense token-pair oracle (oracle/grouped_oracle.py dense_forward,
differentiable by autograd). In fp32 mode the loss and every LoRA gradient must
agree to rel-L2 1e-4 (fp32 GEMMs and the 1e-5 fp32 operator through two layers);
in bf16 mode (bf16 weights and activations, matrix-core operator) the loss must
agree to 2e-2 relative and every gradient must be finite. The OAL factors are
trainable parameters: their gradients (the operator's coefficient-gradient
kernels, chained through the factor expansion) are compared with the CPU twin's
autograd through the dense oracle, to 1e-4 in fp32 mode and 0.1 in bf16 mode
(bf16 weights and activations through two layers).
"""

import copy
import math

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
    return loss.detach(), [p.grad for p in model.lora_parameters()], [p.grad for p in model.oal_parameters()]


def test_qwen_oal_model_fp32_matches_cpu_twin():
    dev = _dev()
    cfg, cpu, gpu = _twin_pair("fp32_ieee")
    tokens = torch.randint(0, cfg.vocab_size, (2, 96), generator=torch.Generator().manual_seed(1))
    loss_c, grads_c, fgrads_c = _loss_and_grads(cpu, tokens)
    loss_g, grads_g, fgrads_g = _loss_and_grads(gpu.to(dev), tokens.to(dev))
    errs = [_rel(g, c) for g, c in zip(grads_g, grads_c)]
    ferrs = [_rel(g, c) for g, c in zip(fgrads_g, fgrads_c)]
    print(f"fp32 model: loss {loss_g.item():.6f} vs {loss_c.item():.6f}, max LoRA grad rel-L2 {max(errs):.2e}, "
          f"max OAL factor grad rel-L2 {max(ferrs):.2e}")
    assert abs(loss_g.item() - loss_c.item()) <= 1e-5 * abs(loss_c.item())
    assert max(errs) <= 1e-4, errs
    assert max(ferrs) <= 1e-4, ferrs


def test_qwen_oal_model_bf16_step_is_close_and_finite():
    from oal_amd.qwen_oal import train_step

    dev = _dev()
    cfg, cpu, gpu = _twin_pair("bf16_tensorcore")
    tokens = torch.randint(0, cfg.vocab_size, (2, 160), generator=torch.Generator().manual_seed(2))
    loss_c, _, fgrads_c = _loss_and_grads(cpu, tokens)
    gpu = gpu.to(dev).cast_parameters_(torch.bfloat16)
    assert all(p.dtype == torch.float32 for p in gpu.oal_parameters())
    opt = gpu.optimizer()
    before = [p.detach().clone() for p in gpu.oal_parameters()]
    loss_g = train_step(gpu, tokens.to(dev), opt)
    grads = [p.grad for p in gpu.lora_parameters()]
    fgrads = [p.grad for p in gpu.oal_parameters()]
    ferrs = [_rel(g, c) for g, c in zip(fgrads, fgrads_c)]
    print(f"bf16 model step: loss {loss_g.item():.5f} vs fp32 CPU twin {loss_c.item():.5f}; "
          f"OAL factor grad rel-L2 vs twin {[f'{e:.2e}' for e in ferrs]}")
    assert abs(loss_g.item() - loss_c.item()) <= 2e-2 * abs(loss_c.item())
    assert all(g is not None and torch.isfinite(g.float()).all() for g in grads)
    assert any(g.float().abs().sum() > 0 for g in grads)
    assert all(g is not None and torch.isfinite(g).all() and g.abs().sum() > 0 for g in fgrads)
    assert max(ferrs) <= 0.1, ferrs
    # the optimizer updated the factors
    assert all(not torch.equal(b, p.detach()) for b, p in zip(before, gpu.oal_parameters()))


def test_config4_full_model_step():
    """BASELINE configuration 4 at its workload: one bf16 LoRA + OAL-factor training step."""
    import time

    from oal_amd.qwen_oal import QwenOALConfig, QwenOALModel, train_step

    dev = _dev()
    cfg = QwenOALConfig()
    assert (cfg.num_layers, cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size) == (24, 151936, 896, 4864)
    model = QwenOALModel(cfg, seed=0).to(dev).cast_parameters_(torch.bfloat16)
    opt = model.optimizer()
    tokens = torch.randint(0, cfg.vocab_size, (4, 4096), generator=torch.Generator().manual_seed(0)).to(dev)
    t0 = time.perf_counter()
    loss = train_step(model, tokens, opt)
    torch.cuda.synchronize()
    lora_b = [p.grad for n, p in model.named_parameters() if n.endswith("lora_b")]
    fgrads = [p.grad for p in model.oal_parameters()]
    print(f"config 4 step: loss {loss.item():.4f} (ln V = {math.log(cfg.vocab_size):.4f}), "
          f"{time.perf_counter() - t0:.2f}s incl. first-call setup; factor grad norms "
          f"{min(float(g.norm()) for g in fgrads):.3e}..{max(float(g.norm()) for g in fgrads):.3e}", flush=True)
    assert math.isfinite(loss.item())
    assert abs(loss.item() - math.log(cfg.vocab_size)) <= 1.0
    assert len(lora_b) == 4 * cfg.num_layers and len(fgrads) == cfg.num_layers
    assert all(g is not None and torch.isfinite(g.float()).all() and g.float().abs().sum() > 0 for g in lora_b)
    assert all(g is not None and torch.isfinite(g).all() and g.abs().sum() > 0 for g in fgrads)
