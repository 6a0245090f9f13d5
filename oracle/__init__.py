"""CPU oracle for RECAP's corrected sparse-attention operator (test infrastructure).

This package is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg import it.  The
product path (``recap_amd``) never imports, links or calls anything here.
"""

from .recap_oracle import *  # noqa: F401,F403
