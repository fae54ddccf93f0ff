"""CPU oracle for the IVA1.0 paged KV-cache hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
directory; only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` use it, as the checker or as the timed CPU baseline.

Modules
  paged_kv        numpy restatement of append / gather / decode attention on the
                  paged layout (fp64 math), plus brute-force loop versions for
                  tiny inputs and the reference's index gather/scatter.
  reference_path  torch-CPU restatement of the reference's own contiguous path
                  (KVCache slice-append, torch.cat append, AttentionTorch math),
                  used as a second, independent formulation and as the CPU
                  baseline that bench.py times.

How each function is pinned (checks in tests/test_oracle.py):
  append/gather            brute-force loops over the documented address
                           formula; round trip gather(append(x)) == x bitwise;
                           agreement with the contiguous KVCache restatement;
                           canary pages untouched; page-permutation invariance.
  decode_attention         torch scaled_dot_product_attention (library routine)
                           in fp64; closed forms (one key -> v[0]; equal keys ->
                           mean of v; one dominant score -> its v row);
                           page-permutation invariance; brute-force visibility
                           sets for window/sink; agreement with reference_path.
  index_gather/scatter     torch advanced indexing; explicit loops.
  Planted mistakes in the oracle (dropped scale, wrong GQA map, window off by
  one, transposed K/V) are checked to fail at least one of the above.
Parity of the half-precision rounding trajectory of the reference's torch
kernels is not pinned (the reference cannot be imported: it does not parse);
it is covered by the stated tolerance instead.
"""
