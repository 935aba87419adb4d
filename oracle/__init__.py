"""CPU oracle for the PISA hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``nlogn_pisa_amd``) imports
this package; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker.
"""

from .pisa_oracle import *  # noqa: F401,F403
