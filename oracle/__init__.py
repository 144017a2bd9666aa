"""CPU oracle for the fdwt hot path -- TEST INFRASTRUCTURE, NOT PART OF THE PRODUCT.

A plain PyTorch (CPU) restatement of the reference's own CPU fallback
(pytorch_morlet_fdwt: src/fdwt/reference.py:15-66, src/fdwt/dwt.py:85-171,
src/fdwt/cwt.py:54-203, 379-394, 512-612, src/fdwt/layers.py:26-262).  Every function
cites the reference lines it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this package, and only as the checker (or the timed CPU baseline): the
product package never imports it and never falls back to it.

How each part is pinned (see ``tests/test_oracle_*.py``):

* ``dwt``: PyWavelets 1.1.1 golden vectors (dwt / idwt / wavedec / waverec, all five
  modes), MATLAB R2012a known answers (PyWavelets' own KAT file), Haar closed form,
  dense-matrix brute force of the analysis operator on tiny sizes, adjointness
  <A x, y> = <x, A^T y> in every mode.
* ``cwt``: plan metadata and fast / direct outputs and gradients written by the
  reference's own CPU path (``tests/golden/make_cwt_golden.py``); the literal
  O(N^2) CWT definition for octave 0 / ``direct``; fast-vs-direct tolerance.
* ``mix`` / ``spectral_softmax`` / modules: reference-generated vectors plus the
  literal (unfused) definitions.
"""
