"""CPU oracle for the LSA select+read path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this package, and only to check results. The product path
(``lsa_rocm_lab``) never imports it and has no CPU fallback.
"""

from oracle.lsa_oracle import *  # noqa: F401,F403
