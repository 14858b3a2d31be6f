"""CPU oracle for the PACK3D attention hot path -- TEST INFRASTRUCTURE ONLY.

This package is the checker, never the thing measured or shipped.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package ``pack3d_amd`` never imports
anything from here and fails loudly when its HIP library is missing.

``oracle.pack3d_oracle`` restates, in PyTorch on the CPU, the reference
operator of amilworks/Pack3D (``src/pack3d``):

* geometry   -- ``geometry.py:53-126,129-266`` (layouts, Morton order,
  neighbour tables, reverse adjacency, repack transport)
* rope       -- ``rope.py:7-48`` (balanced pair allocation, axial RoPE)
* compression -- ``compression.py:7-44`` (learned fine pooling, coarse mean)
* core       -- ``reference.py:8-31`` (global + local softmax, fusion)
* attention  -- ``attention.py:24-89`` (the PACK3D layer)
* validation -- ``_validation.py:4-37`` (the core contract)

Differences from the reference, all deliberate:

* no dense-size guards (``reference.py:13-15``, ``compression.py:26-27``);
  the core is evaluated in query chunks instead, and can evaluate only a
  chosen subset of query rows (for sampled checks at full size);
* head_dim is not restricted to {16,32,64,128}: any even head_dim is
  accepted (the north star needs 48);
* the coarse mean is vectorised instead of looping over groups in Python
  (same arithmetic: a sum over the group, then a division by the count).

Pinning (see ``tests/test_oracle_*.py``): every function here is checked
against closed forms, the known answers in the reference docs and tests,
invariants (relative-position identity, repack equivariance, partition),
and brute-force pure-Python evaluation on tiny inputs.
"""
