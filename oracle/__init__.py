"""CPU oracle for the verify/decode paged-attention path.

TEST INFRASTRUCTURE ONLY.  This package restates, in numpy, the algorithm of
swiftLLM's Triton kernels for the path (paged attention, KV-cache store,
QK-RMSNorm, RoPE) and of the host code that defines the verify rows.  It is
imported only by ``tests/``, by ``__graft_entry__.smoke()`` (as the checker)
and by ``bench.py``'s ``cpu_baseline`` leg (as the timed CPU baseline).  The
product path (``nebulasd_amd``) never imports it and has no CPU fallback.

Every function cites the reference file:line it follows.  How each function
is pinned (closed forms, invariants, library routines, the reference's own
literal test cases) is listed in the headers of ``oracle/attention.py`` and
``oracle/blocks.py``, ``oracle/hostkv.py`` and ``oracle/layer.py``.
"""

from .attention import *  # noqa: F401,F403
from .blocks import *  # noqa: F401,F403
from .hostkv import *  # noqa: F401,F403
from .layer import *  # noqa: F401,F403
