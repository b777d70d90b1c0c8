"""Reference module name src/fused_topk.py, served by gpusparse (HIP, gfx950)."""
import _path  # noqa: F401

from gpusparse.chunked import triton_chunked_score_fused  # noqa: F401
from gpusparse.search import compacted_topk  # noqa: F401
