"""CPU oracle for the OAL grouped quadratic attention operator.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (``oal_amd``) may
import this package: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker or as the
timed CPU baseline, never as the thing measured or shipped.

Modules
-------
``grouped_oracle``
    Pure torch-CPU restatements of the reference algorithm:

    * ``materialized_forward``: the token-cumulative H0/H1/H2 state algorithm of
      ``oal_attention/grouped_reference.py:18-178`` (small shapes only; it
      materializes ``[B, H, N, D(D+1)/2, DV+1]``).
    * ``dense_forward``: the independent N^2 factor-form oracle of
      ``tests/operators/test_grouped_quadratic.py:31-84``.
    * ``chunked_forward`` / ``chunked_backward``: the chunked linear-attention
      form (per-chunk state totals, exclusive scan, readout plus intra-chunk
      term) with the closed-form vector-Jacobian products of
      ``oal_attention/hd_block_gemm_backward.py`` (normalization VJP :191-308,
      dCarry and right scan :764-908, query and KV sides :473-761,
      :911-1452).  This one runs at the full benchmark shapes.

Pinning (see ``tests/test_oracle.py``)
--------------------------------------
* the two golden fixtures shipped with the reference tests
  (``tests/operators/fixtures/grouped_quadratic/*.json``);
* materialized == dense == chunked on random fp64 cases (independent
  formulations: group-sum N^2 form, token-cumsum state form, feature form);
* ``torch.autograd.gradcheck`` of the materialized form, and the closed-form
  chunked backward against autograd of the dense form, including the
  coefficient gradients;
* the factor-expansion known-answer test of
  ``tests/operators/test_grouped_quadratic.py:476-488``;
* invariants: token 0 output equals v_0, q = 0 gives the causal running mean
  of v, chunk-size invariance, GQA equals K/V repeated per query head.

No function here is "parity unpinned".
"""
