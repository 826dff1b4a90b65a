"""CPU oracle for the FA2-with-4D-mask hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
package: it is the checker used by ``tests/``, by ``__graft_entry__.smoke()``
and by the ``cpu_baseline`` leg of ``bench.py``.  The product path runs the
HIP kernels in ``fa2-with-4d-mask_amd/csrc`` and fails loudly when they are
not built.

Contents
--------
``eager``      restatement of the reference's eager fp32 attention and its
               autograd backward (benchmark/precision_check.py:133-180),
               plus a memory-light closed-form chunked variant for large
               shapes, diff statistics and pass rules
               (precision_check.py:183-206) and the FLOP convention
               (benchmark/throughput_check.py:85-92).
``inputs``     seeded input generators for every BASELINE config
               (precision_check.py:110-130 and the config text).
``bruteforce`` float64 scalar-loop attention used to pin ``eager`` on tiny
               inputs.

Parity status of each function is stated in its docstring ("pinned by ...").
"""
