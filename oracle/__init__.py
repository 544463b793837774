"""CPU oracle for the sparse shared-KV attention decode path.

TEST INFRASTRUCTURE ONLY. This package is the oracle the parity tests check
against: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it. The product path (``sparse_attn_sharedkv_amd``) never imports,
links or calls anything here, and fails loudly when its HIP library is
missing instead of falling back to this code.

Contents
--------
``golden_ref``  restatement of the reference's CPU golden math
                (``golden.py:28-204``), gathering KV rows straight from the
                paged pools instead of densifying them.
``gen``         seeded input generators (paged pools, block tables, top-k
                index sets) restating ``golden.py:315-473`` plus the
                workload builders for the benchmark shapes.
``checks``      the reference's tolerance rules as assertions
                (``test_sparse_attn_sharedkv.py:394-481``) and the stricter
                per-element bound used for this port.

Parity pinning (what fixes each function independently of this code):

* online softmax + sinks + LSE: closed-form one-shot softmax over
  ``scores ∪ {sink}`` evaluated in float64 (``golden.py:207-244``), the
  worked example of ``docs/OnlineSoftmax 原理详解.html`` (§5.1, §6.3, §7.2),
  and tile-size invariance;
* index resolution: brute-force set semantics on small inputs;
* paging: pack/unpack round trips against a dense tensor;
* split-KV merge: invariance of the merged result to the partition.
"""
