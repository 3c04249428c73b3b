"""TEST INFRASTRUCTURE ONLY: the CPU oracle of bpdecode's constraint step.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker (or as
the timed CPU baseline).  The product (``bpdecode_amd``) never imports it.

* ``oracle.dense``  numpy restatement of the dense tok_next path
  (ops.py:143-197, 262-311; fsa.py:155-174).
* ``oracle.pda``    ctypes wrapper of ``liboracle_pda.so``, a plain-C
  restatement of pda.hpp:95-258 and pda_cpu.cpp:7-54.
* ``oracle.soft``   float64 numpy restatement of build_lookahead /
  apply_soft_ (ops.py:200-259) and of the prior-weighted lookahead.
* ``oracle.ref``    ctypes wrapper of ``_ref/libbpd_ref.so``, the reference's
  own mask_cpu.cpp / pda_cpu.cpp compiled from its sources (only present
  where the reference checkout exists); used to pin the restatements.
"""
