"""CPU oracle for the Sol-Attn sparse attention path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker or the timed CPU baseline.
The product package never imports it.
"""

from .oracle import *  # noqa: F401,F403
