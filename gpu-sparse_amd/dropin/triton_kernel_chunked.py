"""Reference module name src/triton_kernel_chunked.py, served by gpusparse (HIP, gfx950)."""
import _path  # noqa: F401

from gpusparse.chunked import build_chunk_boundaries, triton_chunked_score  # noqa: F401
