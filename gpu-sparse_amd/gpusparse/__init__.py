"""gpusparse: exact learned-sparse (SPLADE) retrieval on MI355X (gfx950).

GPU inverted-index construction, batched exact scatter-add scoring and top-k
selection, behind the Python surface of ashutoshuiuc/gpu-sparse.  Compute runs
in hand-written HIP kernels (libgpusparse.so) called through a C ABI
(include/gpusparse.h); PyTorch provides device memory and streams.
"""
from .index import (BLOCK_SIZE, CSR, VOCAB_SIZE, GPUInvertedIndex, build_from_csr, build_gpu_index_from_csr,
                    build_gpu_inverted_index, build_gpu_inverted_index_from_sparse, build_index, check_lists,
                    index_memory_stats, require_ascending)
from .search import (MAX_K, MAX_T, PendingSearch, atomic_fused_score, compacted_topk, scatter_add, search, search_async,
                     search_counts, search_plan, timing_dict, topk_rows, triton_fused_score)
from .chunked import build_chunk_boundaries, triton_chunked_score, triton_chunked_score_fused
from .engine import determine_dimension, retrieve, run_engine, to_csr, to_query_tensors, write_run
from .storage import load_index, save_index
from .verification import compute_recall_exact, prepare_queries_from_meta

__all__ = [
    "BLOCK_SIZE", "CSR", "VOCAB_SIZE", "GPUInvertedIndex", "build_from_csr", "build_gpu_index_from_csr",
    "build_gpu_inverted_index", "build_gpu_inverted_index_from_sparse", "build_index", "check_lists",
    "index_memory_stats", "require_ascending", "MAX_K", "MAX_T", "PendingSearch", "atomic_fused_score", "compacted_topk",
    "scatter_add", "search", "search_async", "search_counts", "search_plan", "timing_dict", "topk_rows", "triton_fused_score", "build_chunk_boundaries",
    "triton_chunked_score", "triton_chunked_score_fused", "determine_dimension", "retrieve", "run_engine", "to_csr", "to_query_tensors",
    "write_run", "load_index", "save_index", "compute_recall_exact", "prepare_queries_from_meta",
]
