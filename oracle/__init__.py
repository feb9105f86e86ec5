"""CPU oracle for the TurboQuant compress / compressed-attention path.

TEST INFRASTRUCTURE ONLY. This package is a numpy restatement of the
reference algorithm (alex-rentel/mlx-turboquant) and exists to check the HIP
implementation. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker
(or, for ``cpu_baseline``, as the timed CPU restatement). The product package
never imports it and has no CPU fallback.

Every function cites the reference file:line it restates. Parity pinning of
each function (golden vectors, known answers, closed forms) lives in
``tests/test_oracle.py``.
"""

from .tq_oracle import *  # noqa: F401,F403
