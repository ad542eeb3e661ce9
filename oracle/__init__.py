"""CPU oracle for the window attention path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for the
baseline, as the timed CPU restatement of the reference's path).  The product
package ``neutrongt_amd`` never imports it and has no CPU fallback.

Modules
-------
attention  literal torch-CPU restatement of NeutronGT's CoreAttention
           (sparse_attention_bias, full_attention) + fp64 brute-force forms and
           the closed-form backward used to pin it.
graph      numpy restatements of the integer window preparation: COO -> CSR
           (both orientations), work lists, related-node selection,
           duplicate-node ordering, feature-cache indices, METIS edge weights.

Pinning status (what checks each function; see tests/test_oracle_*.py):
  sparse_attention_bias   fp64 brute force (dense masked formula), invariants
                          (empty row -> 0, single edge, q = 0 -> mean of V),
                          golden fixtures
  sparse backward         autograd vs closed form vs fp64 gradcheck/finite diff
  full_attention (+bwd)   fp64 softmax formula, gradcheck
  csr_from_coo            torch.sparse_coo_tensor(...).coalesce() on
                          duplicate-free inputs, brute-force sort
  merge_related_nodes     hand-derived answers incl. ties, brute force
  duplicate ordering      hand-derived answers
  adj weights             hand-derived answers
"""
