"""Facts about the BASELINE config inputs, pinned on the CPU with the oracle.

The config coefficients (c0 = 1, lam ~ U(0.5, 1.5), Gam_gh ~ U(0, 0.5) for
g <= h, mirrored) do not form a PSD kernel: every
query head's Gam has a negative eigenvalue, so no packed factor L (Gam = L L^T)
exists for them and kappa can be negative. On the bf16-rounded q, k, v of
configs 1, 2 and 3 the fp32 oracle finds 1, 19 and 7 tokens with den <= 0 --
outputs the reference refuses (grouped_quadratic.py:386-394,
hd_block_gemm_runtime.py:392-408). The GPU tests and the benchmark run on these
inputs as BASELINE.json specifies them; their masked comparisons exclude at
most 0.1% of the tokens and print how many.
"""

import os

import pytest
import torch

from oracle import grouped_oracle as go


@pytest.mark.parametrize("config,nonpositive,min_den", [(1, 1, -2.08), (2, 19, -3.50), (3, 7, -0.94)])
def test_config_nonpositive_denominator_counts(config, nonpositive, min_den):
    torch.set_num_threads(min(8, len(os.sched_getaffinity(0))))
    inp = go.config_inputs(config)
    q, k, v = (inp[n].to(torch.bfloat16).float() for n in ("q", "k", "v"))
    wq = go.feature_coefficients(inp["groups"], inp["c0"], inp["lam"], inp["gam"], scale=inp["scale"], head_dim=64)
    _, _, den = go.chunked_forward(q, k, v, wq, chunk=64)
    assert int((den <= 0).sum()) == nonpositive
    assert abs(float(den.min()) - min_den) < 0.01
    assert int((den.abs() <= 1.0).sum()) <= 1e-3 * den.numel()


@pytest.mark.parametrize("config", [0, 1, 2, 3])
def test_config_gamma_is_not_psd(config):
    inp = go.config_inputs(config, seq_len=64)
    ev = torch.linalg.eigvalsh(inp["gam"].double())
    assert bool((ev.min(-1).values < 0).all())
