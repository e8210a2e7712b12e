"""CPU oracle for the Mamba 4 memory read -- TEST INFRASTRUCTURE ONLY.

This package is the checker for the MI355X HIP implementation in
``mamba4_amd``.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only to check or to
time the CPU restatement.  The product path never calls it; the HIP library
raises when its shared object is missing instead of falling back here.

Every function restates the reference algorithm of tasmaikeni13/mamba4 in
NumPy and cites the reference ``file:line`` it follows.  How each function is
pinned (known answers, invariants, independent autodiff, finite differences)
is listed in ``memread.PINNED``; no function is left "parity unpinned".
"""

from oracle.memread import (  # noqa: F401
    PINNED,
    backward,
    cholesky_reciprocal,
    decode_step,
    dense_reference,
    factored_solve,
    forward,
)
