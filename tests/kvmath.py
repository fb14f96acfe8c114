"""Independent numpy derivations used to pin the oracle and the HIP path.

Nothing here restates the offset arithmetic of the oracle or the kernels.
A pool is viewed as a numpy array whose axes are the layout's nesting
order, stated once by the reference: page -> layer -> tensor -> token ->
(head * dim) (crates/sglang-srt/src/kv_cache.rs:653-700 and the test name
``page_major_layout_matches_page_layer_tensor_token_order``,
crates/sglang-srt/tests/kv_cache.rs:64). Indexing that view is numpy's job,
so a dropped term, a swapped axis or a wrong stride in the C/HIP code shows
up as a mismatch here.
"""
from __future__ import annotations

import numpy as np


def pool_view(pool_bytes: np.ndarray, page_count: int, num_layers: int, tensors: int,
              page_size: int, row_bytes: int, heads: int = 1, hnd: bool = False) -> np.ndarray:
    """View of a uniform page-major pool.

    NHD: [page][layer][tensor][token][heads][chunk]
    HND: [page][layer][tensor][heads][token][chunk]
    where chunk = row_bytes // heads.
    """
    chunk = row_bytes // heads
    flat = pool_bytes.reshape(-1).view(np.uint8)
    if hnd:
        return flat.reshape(page_count, num_layers, tensors, heads, page_size, chunk)
    return flat.reshape(page_count, num_layers, tensors, page_size, heads, chunk)


def rows_from_view(view: np.ndarray, slots: np.ndarray, layer: int, tensor: int, page_size: int,
                   hnd: bool) -> np.ndarray:
    """The [len(slots)][row_bytes] rows of (layer, tensor) at `slots`, token-major."""
    slots = np.asarray(slots, dtype=np.int64)
    pages, pos = slots // page_size, slots % page_size
    if hnd:
        sel = view[pages, layer, tensor, :, pos, :]  # [n][heads][chunk]
    else:
        sel = view[pages, layer, tensor, pos, :, :]  # [n][heads][chunk]
    return sel.reshape(len(slots), -1)


def write_rows_to_view(view: np.ndarray, slots: np.ndarray, layer: int, tensor: int,
                       page_size: int, hnd: bool, rows: np.ndarray) -> None:
    slots = np.asarray(slots, dtype=np.int64)
    pages, pos = slots // page_size, slots % page_size
    heads = view.shape[3] if hnd else view.shape[4]
    r = rows.reshape(len(slots), heads, -1)
    if hnd:
        view[pages, layer, tensor, :, pos, :] = r
    else:
        view[pages, layer, tensor, pos, :, :] = r


def acceptance_rows(row_count: int, row_bytes: int, row_stride: int, seed: int):
    """strided_byte_rows (crates/sglang-srt/tests/cuda_backend.rs:158-176):
    byte b of row r is (seed + 37 r + 13 b) % 251; rows sit row_stride apart."""
    storage = np.zeros((row_count - 1) * row_stride + row_bytes, dtype=np.uint8)
    rows = []
    b = np.arange(row_bytes, dtype=np.int64)
    for r in range(row_count):
        row = ((seed + r * 37 + b * 13) % 251).astype(np.uint8)
        storage[r * row_stride: r * row_stride + row_bytes] = row
        rows.append(row)
    return storage, rows


def strided_rows(storage: np.ndarray, row_count: int, row_bytes: int, row_stride: int) -> np.ndarray:
    return np.stack([storage[r * row_stride: r * row_stride + row_bytes] for r in range(row_count)])


def slots_from_page_table(page_table: np.ndarray, spans: np.ndarray, page_size: int) -> np.ndarray:
    """Physical slot of every row covered by `spans`, by walking tokens one at
    a time in Python (small cases only)."""
    total = int(max((int(s["row_start"]) + int(s["token_count"]) for s in spans), default=0))
    out = np.full(total, -1, dtype=np.int64)
    for s in spans:
        for j in range(int(s["token_count"])):
            tok = int(s["token_offset"]) + j
            page = int(page_table[int(s["page_table_start"]) + tok // page_size])
            out[int(s["row_start"]) + j] = page * page_size + tok % page_size
    return out


def random_pool_bytes(rng: np.random.Generator, nbytes: int) -> np.ndarray:
    return rng.integers(0, 256, size=nbytes, dtype=np.uint8)
