"""CPU oracle (test infrastructure only; never called by the product path).

See `oracle.attention` for the restated algorithm and how it is pinned.
The CUDA reference itself cannot be compiled here (it needs nvcc and the CUDA
headers), so there is no `oracle/_ref` build.
"""
from .attention import *  # noqa: F401,F403
