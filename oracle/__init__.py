"""CPU oracle for the packed-KV (k2b) decode path — TEST INFRASTRUCTURE ONLY.

This package restates, in plain torch-on-CPU (fp32) and numpy, the algorithms of
pherber3/bmx that the HIP product path replaces.  It is the checker, never the
product: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg
of ``bench.py`` may import it.  ``bmx_amd`` never imports anything from here.

Modules
  codecs     k2b key codec (low-rank + per-channel 3-bit RTN residual), per-head
             Hadamard/Lloyd value codec, the RTN arms, bpe accounting and the
             flush schedule  (reference: src/bmx/cache/codecs.py, quant/rtn.py,
             quant/hadamard.py, cache/streaming.py:144-151)
  attention  RoPE tables, naive dense oracle, chunked online-softmax path, tail
             partial and split-merge math (reference: cache/rope.py,
             cache/chunked_attention.py, cache/triton_dequant_attention.py)
  layout     numpy packer/unpacker for this build's 16-token physical page format
             (no reference counterpart: it restates the page format the HIP write
             kernel must produce, so the kernel's bytes can be checked exactly)

Pinning (every function is checked in tests/test_oracle.py):
  * against golden vectors written by the reference's own code
    (tests/golden/make_golden.py -> tests/golden/*.npz),
  * against closed forms (Sylvester Hadamard / sqrt(d), bpe formulas, the
    flush-schedule formula, exact online-softmax and split-merge identities),
  * against brute force on tiny inputs.
Parity unpinned: none of the functions used by the tests (each has a golden or
closed-form check).
"""
