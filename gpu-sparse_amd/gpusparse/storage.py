"""On-disk index format: save and memory-mapped load of a GPUInvertedIndex.

The reference rebuilds its index from the document CSR on every run (numpy
argsort on the host, lsr_benchmark_engine/gpusparse_retrieval.py:81-115).  This
format stores the built index instead, so a later run maps the file and copies
the arrays straight to the GPU.

Layout of one index file:
  bytes [0, 8)        magic b"GSPIDX01"
  bytes [8, 16)       little-endian uint64: length of the JSON header
  bytes [16, ...)     the JSON header (UTF-8), zero-padded to ALIGN bytes
  then each array's raw little-endian bytes, each starting on an ALIGN boundary

JSON header: {"format": 1, "num_docs", "vocab_size", "weights": dtype name,
"arrays": [{"name", "dtype", "shape", "offset", "nbytes", "crc32"}, ...]}.
Arrays: the six GPUInvertedIndex tensors (doc_ids, scores, offsets, lengths,
padded_lengths, max_scores) and, when saved with ``forward=True`` and present,
the doc-major copy used by the exact rescoring (fwd_ptr, fwd_terms,
fwd_weights).
"""
from __future__ import annotations

import json
import os
import struct
import zlib

import numpy as np
import torch

from .index import GPUInvertedIndex

MAGIC = b"GSPIDX01"
FORMAT = 1
ALIGN = 4096
_CHUNK = 64 << 20  # bytes per staged host -> device copy

_INDEX_ARRAYS = ("doc_ids", "scores", "offsets", "lengths", "padded_lengths", "max_scores")
_FWD_ARRAYS = ("fwd_ptr", "fwd_terms", "fwd_weights")
_DTYPES = {"int32": np.int32, "int64": np.int64, "float32": np.float32, "float16": np.float16,
           "uint8": np.uint8}
_TORCH = {np.dtype(np.int32): torch.int32, np.dtype(np.int64): torch.int64, np.dtype(np.float32): torch.float32,
          np.dtype(np.float16): torch.float16, np.dtype(np.uint8): torch.uint8}


def save_index(index, path: str, *, forward: bool = False) -> dict:
    """Writes `index` to `path` (replaced atomically).  Returns the JSON header.
    With ``forward=True`` the doc-major copy is stored too (built first if the
    index has none)."""
    arrays = [(n, getattr(index, n)) for n in _INDEX_ARRAYS]
    if forward:
        from .index import ensure_search_state
        fwd = index.aux().get("fwd")
        if fwd is None:
            fwd = ensure_search_state(index).get("fwd")
        if fwd is None:
            raise ValueError("this index has no doc-major copy to store (uint8 weights, or no GPU memory for it)")
        nnz = int(index.lengths.sum().item())
        arrays += [("fwd_ptr", fwd[0]), ("fwd_terms", fwd[1][:nnz]), ("fwd_weights", fwd[2][:nnz])]
    host = [(n, t.detach().contiguous().cpu().numpy()) for n, t in arrays]
    entries = []
    for n, a in host:
        entries.append({"name": n, "dtype": str(a.dtype), "shape": list(a.shape), "offset": 0,
                        "nbytes": int(a.nbytes), "crc32": zlib.crc32(memoryview(a).cast("B")) & 0xFFFFFFFF})
    meta = {"format": FORMAT, "num_docs": int(index.num_docs), "vocab_size": int(index.vocab_size),
            "weights": str(host[1][1].dtype), "arrays": entries}
    # offsets depend on the header length, which depends on the offsets' digits:
    # settle them with a generous fixed header size
    blob = json.dumps(meta).encode()
    head = (16 + len(blob) + 64 * len(entries) + ALIGN - 1) // ALIGN * ALIGN
    off = head
    for e in entries:
        e["offset"] = off
        off = (off + e["nbytes"] + ALIGN - 1) // ALIGN * ALIGN
    blob = json.dumps(meta).encode()
    assert 16 + len(blob) <= head
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(MAGIC + struct.pack("<Q", len(blob)) + blob)
        for e, (_, a) in zip(entries, host):
            f.seek(e["offset"])
            f.write(memoryview(a).cast("B"))
        f.truncate(max(off, head))
    os.replace(tmp, path)
    return meta


def read_header(path: str) -> dict:
    """The JSON header of an index file, validated against the file size."""
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        pre = f.read(16)
        if len(pre) < 16 or pre[:8] != MAGIC:
            raise ValueError(f"{path}: not a gpusparse index file (bad magic)")
        (n,) = struct.unpack("<Q", pre[8:])
        if n > size - 16:
            raise ValueError(f"{path}: header length {n} exceeds the file")
        try:
            meta = json.loads(f.read(n).decode())
        except (UnicodeDecodeError, json.JSONDecodeError) as e:
            raise ValueError(f"{path}: unreadable header ({e})") from None
    if meta.get("format") != FORMAT:
        raise ValueError(f"{path}: format {meta.get('format')} is not {FORMAT}")
    names = [e.get("name") for e in meta.get("arrays", [])]
    if tuple(names[:6]) != _INDEX_ARRAYS or names[6:] not in ([], list(_FWD_ARRAYS)):
        raise ValueError(f"{path}: unexpected arrays {names}")
    V, N = int(meta["vocab_size"]), int(meta["num_docs"])
    for e in meta["arrays"]:
        dt = _DTYPES.get(e["dtype"])
        if dt is None:
            raise ValueError(f"{path}: array {e['name']} has unsupported dtype {e['dtype']}")
        if int(np.prod(e["shape"], dtype=np.int64)) * np.dtype(dt).itemsize != e["nbytes"]:
            raise ValueError(f"{path}: array {e['name']} size does not match its shape")
        if e["offset"] % ALIGN or e["offset"] + e["nbytes"] > size:
            raise ValueError(f"{path}: array {e['name']} lies outside the file (truncated?)")
    a = {e["name"]: e for e in meta["arrays"]}
    for n in ("offsets", "lengths", "padded_lengths", "max_scores"):
        if a[n]["shape"] != [V]:
            raise ValueError(f"{path}: {n} has shape {a[n]['shape']}, expected [{V}]")
    if a["doc_ids"]["shape"] != a["scores"]["shape"]:
        raise ValueError(f"{path}: doc_ids and scores differ in length")
    if "fwd_ptr" in a and a["fwd_ptr"]["shape"] != [N + 1]:
        raise ValueError(f"{path}: fwd_ptr has shape {a['fwd_ptr']['shape']}, expected [{N + 1}]")
    return meta


def _to_device(arr: np.ndarray, device: torch.device) -> torch.Tensor:
    """Copies a (memory-mapped) array to `device` through pinned staging buffers."""
    out = torch.empty(arr.shape, dtype=_TORCH[arr.dtype], device=device)
    if device.type != "cuda" or arr.nbytes <= _CHUNK:
        out.copy_(torch.from_numpy(np.array(arr)))
        return out
    flat_in = arr.reshape(-1).view(np.uint8)
    flat_out = out.view(-1).view(torch.uint8)
    bufs = [torch.empty(_CHUNK, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    done = [None, None]
    stream = torch.cuda.current_stream(device)
    for i, s in enumerate(range(0, flat_in.size, _CHUNK)):
        b = i & 1
        if done[b] is not None:
            done[b].synchronize()
        n = min(_CHUNK, flat_in.size - s)
        np.copyto(bufs[b].numpy()[:n], flat_in[s:s + n])
        flat_out[s:s + n].copy_(bufs[b][:n], non_blocking=True)
        done[b] = torch.cuda.Event()
        done[b].record(stream)
    stream.synchronize()
    return out


def _check_layout(path: str, m: dict):
    """Host-side bounds of the layout (the kernels index with these values): every
    list inside the slot arrays, and the doc-major rows inside their arrays."""
    n_slots = m["doc_ids"].shape[0]
    off, ln, pad = (m[n].astype(np.int64) for n in ("offsets", "lengths", "padded_lengths"))
    if np.any(ln < 0) or np.any(pad < ln) or np.any(off < 0) or np.any(off + pad > n_slots):
        raise ValueError(f"{path}: posting lists lie outside the slot arrays")
    if "fwd_ptr" in m:
        ptr = m["fwd_ptr"]
        nnz = int(ln.sum())
        if (ptr[0] != 0 or np.any(np.diff(ptr) < 0) or int(ptr[-1]) != nnz
                or m["fwd_terms"].shape[0] != nnz or m["fwd_weights"].shape[0] != nnz):
            raise ValueError(f"{path}: doc-major rows do not match the posting count")


def load_index(path: str, device=None, *, verify: bool = False) -> GPUInvertedIndex:
    """Maps an index file and copies its arrays to `device` (default: the current
    GPU).  The layout is bounds-checked on the host first; ``verify=True`` also
    checks every array's CRC-32.  Lists are checked for ascending order on first
    search, as for any index built elsewhere."""
    meta = read_header(path)
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    maps = {}
    for e in meta["arrays"]:
        dt = np.dtype(_DTYPES[e["dtype"]])
        m = np.memmap(path, dtype=dt, mode="r", offset=e["offset"], shape=tuple(e["shape"]))
        if verify and (zlib.crc32(memoryview(np.ascontiguousarray(m)).cast("B")) & 0xFFFFFFFF) != e["crc32"]:
            raise ValueError(f"{path}: array {e['name']} fails its CRC-32 check")
        maps[e["name"]] = m
    if maps["scores"].dtype.name not in ("float32", "float16", "uint8"):
        raise ValueError(f"{path}: posting weights must be float32, float16 or uint8")
    _check_layout(path, maps)
    arrays = {n: _to_device(m, dev) for n, m in maps.items()}
    ix = GPUInvertedIndex(doc_ids=arrays["doc_ids"], scores=arrays["scores"], offsets=arrays["offsets"],
                          lengths=arrays["lengths"], padded_lengths=arrays["padded_lengths"],
                          max_scores=arrays["max_scores"], num_docs=int(meta["num_docs"]),
                          vocab_size=int(meta["vocab_size"]), device=dev)
    if "fwd_ptr" in arrays:
        ix.aux()["fwd"] = (arrays["fwd_ptr"], arrays["fwd_terms"], arrays["fwd_weights"])
    return ix


__all__ = ["save_index", "load_index", "read_header", "MAGIC", "FORMAT"]
