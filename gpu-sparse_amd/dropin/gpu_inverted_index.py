"""Reference module name src/gpu_inverted_index.py, served by gpusparse (HIP, gfx950)."""
import _path  # noqa: F401

from gpusparse.index import (BLOCK_SIZE, GPUInvertedIndex, build_gpu_inverted_index,  # noqa: F401
                             build_gpu_inverted_index_from_sparse, index_memory_stats)
