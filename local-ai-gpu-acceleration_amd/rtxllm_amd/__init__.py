"""Host-side mirror of the reference runtime's decode path over the gfx950 C-ABI.

``_lib`` binds build/librtxllm.so; ``packs`` builds seeded synthetic resident
packs (host memory); ``ops`` launches the kernels on torch-allocated device
memory and torch's current HIP stream.
"""

from . import formats  # noqa: F401
from ._lib import HipError, check, lib  # noqa: F401
