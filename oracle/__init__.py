"""CPU oracle for the Q8_0 linear path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this package.  It is the checker, never the product: the HIP
library in ``llmcp_amd`` does not import, link or call anything here.
"""
