"""MI355X-native Token2Wav hot path: the CFG Euler DiT solve and the HiFT vocoder on hand-written gfx950 HIP kernels.

Imported as ``t2w_amd`` (see the repository's ``t2w_amd.py``).  The compute lives in ``csrc/`` (compiled into
``libt2w_hip.so``, a C-ABI library); the Python modules here plan the packed ragged calls, own the stream state and
call the library through ctypes.  Nothing here falls back to a CPU path: without the built library every compute entry
point raises.
"""

from .config import DiTConfig, HiFTConfig  # noqa: F401
