"""Reference module name src/triton_kernel.py, served by gpusparse (HIP, gfx950)."""
import _path  # noqa: F401

from gpusparse.search import triton_fused_score  # noqa: F401
