"""Test-only stand-in for tirex_tracker (lsr_benchmark_engine/gpusparse_retrieval.py:38):
metadata registration and a tracking context that writes a small metadata file."""
import contextlib
import enum
import time

METADATA = []


class ExportFormat(enum.Enum):
    IR_METADATA = "ir_metadata"


def register_metadata(meta):
    METADATA.append(dict(meta))


@contextlib.contextmanager
def tracking(export_file_path=None, export_format=ExportFormat.IR_METADATA):
    t0 = time.perf_counter()
    yield
    if export_file_path is not None:
        with open(export_file_path, "w") as f:
            f.write(f"format: {export_format.value}\nwall_s: {time.perf_counter() - t0:.6f}\n")
