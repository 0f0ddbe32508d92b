"""o1 MI355X engine: Python mirror of the C-ABI in include/*.h.

The compute path is libo1hip.so (HIP kernels for gfx950 + C++ host code);
this package only loads it through ctypes and passes device pointers that
torch allocated. Importing it never falls back to another implementation:
if the library is missing, load() raises.
"""
from .o1hip import *  # noqa: F401,F403
