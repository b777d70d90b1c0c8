"""Test-only stand-in for the lsr-benchmark package: the one call the plug-in
makes on it (lsr_benchmark_engine/gpusparse_retrieval.py:178)."""

REGISTERED = []


def register_to_ir_datasets(dataset):
    REGISTERED.append(dataset)
