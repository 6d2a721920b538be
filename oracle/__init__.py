"""CPU oracle for the quashkv_amd hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithms that the HIP
kernels in ``quashkv_amd/csrc`` replace.  It exists to CHECK the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package ``quashkv_amd`` never imports,
links or calls anything here, and has no CPU fallback of its own.

Pinning (how each function here is checked before it is trusted):

* ``ref_math.pack_bits/unpack_bits/packed_size`` -- golden bytes written by
  the reference (``tests/golden/packing.npz``), hand-derived known answers
  (``[0..7]@3b -> 88 C6 FA``, ``[0,1,2,3]@2b -> E4``, ``[1,2]@4b -> 21``,
  ``[1,0,1,1,0,0,0,1]@1b -> 8D``) and brute-force bit reconstruction.
* ``ref_math.quantize_boundary`` -- golden codes incl. exact ties
  (``tests/golden/compress.npz`` ``tie_*``) and equivalence with the
  nearest-centroid argmin.
* ``ref_math.random_orthogonal/random_signs`` -- golden Pi/S
  (``tests/golden/rotations.npz``) plus the QR characterisation
  ``Pi^T A`` upper-triangular with positive diagonal, ``Pi^T Pi = I``.
* ``ref_math.compress_* / decompress_*`` -- golden outputs on seeded inputs,
  the ``x = e_k`` special case (``y = Pi[:, k]``) that fixes the operand
  orientation, and norm/round-trip invariants.
* ``ref_math.attention_naive/attention_online`` -- golden engine and
  online-softmax outputs, naive == online, and the brute-force scalar loop
  ``attention_bruteforce`` on tiny inputs.
* ``ref_math.mixed_*`` -- golden calibration indices and codes.
* ``ref_math.index_search`` -- golden top-k indices/scores.
"""
