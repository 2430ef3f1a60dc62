"""CPU oracle of omniasr-trt's speculative greedy verify step -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

A restatement in numpy (and, for the reference-order decode loop, plain PyTorch on the CPU) of the
reference's semantics for every function on the path; each function cites the reference file:line it
follows.  It is the checker of the HIP kernels: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and never as the thing measured or shipped.  The
product package (``omniasr-trt_amd``) does not import it and has no CPU fallback.

Modules:
  ``bf16``     -- bf16 rounding (round to nearest even) in numpy;
  ``verify``   -- RoPE + append, verify attention, log-softmax argmax, acceptance, proposal, step assembly,
                  CTC-frame drafts;
  ``reference``-- the reference-order greedy decode loop and a fp64 decoder forward (torch, CPU).

How each function is pinned (golden vectors, closed forms, invariants, brute force) is recorded next to it
and in the tests (tests/test_oracle.py).
"""
