"""CPU oracle for the KV-cache hot path — TEST INFRASTRUCTURE.

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this package, and only as the checker (or the timed CPU baseline).
The product (``atomflow_amd``) never imports it.

``liboracle_kv.so`` is the scalar C++ restatement of the reference kernels
(``oracle_kv.cpp``, each function citing the reference file:line it follows);
``block_model`` is a pure-Python model of the paged BlockManager contract and
``sched_model`` one of the continuous-batching scheduler's rules.
"""
from .oracle import *  # noqa: F401,F403
from . import block_model  # noqa: F401
from . import sched_model  # noqa: F401
