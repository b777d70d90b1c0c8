"""Reference module name src/run_correctness_verification.py: its index builder
and its harness helpers (query tensors from cached metadata, exact recall)."""
import _path  # noqa: F401

from gpusparse.index import VOCAB_SIZE, build_gpu_index_from_csr  # noqa: F401
from gpusparse.verification import compute_recall_exact, prepare_queries_from_meta  # noqa: F401
