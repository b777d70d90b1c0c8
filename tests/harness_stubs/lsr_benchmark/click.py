"""Test-only stand-in for lsr_benchmark.click.retrieve_command
(lsr_benchmark_engine/gpusparse_retrieval.py:175): the decorated engine entry
point takes (dataset, embedding, output, k) with `output` as a pathlib.Path."""
import functools
import pathlib


def retrieve_command():
    def wrap(fn):
        @functools.wraps(fn)
        def cli(dataset, embedding, output, k):
            return fn(dataset, embedding, pathlib.Path(output), int(k))
        return cli
    return wrap
