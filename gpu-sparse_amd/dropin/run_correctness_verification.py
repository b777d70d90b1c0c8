"""Reference module name src/run_correctness_verification.py (its index builder only)."""
import _path  # noqa: F401

from gpusparse.index import VOCAB_SIZE, build_gpu_index_from_csr  # noqa: F401
