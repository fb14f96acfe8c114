"""CPU oracle for the KV-cache transfer path (ctypes over libkv_oracle.so).

TEST INFRASTRUCTURE: only tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg import this package, and only as the checker. The
product library never loads it.

The C sources (kv_oracle.c) restate the reference's byte-movement
algorithm; the functions here marshal numpy arrays to them. The paged
attention restatement (floating point) is numpy, in float64. Build with
``make -C oracle``.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libkv_oracle.so")

FLAG_SLOT = 1
FLAG_PAGE = 2
FLAG_SPAN = 4
INVALID_SLOT = np.uint64(0xFFFFFFFFFFFFFFFF)

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u64 = ctypes.c_uint64


class OraLayout(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "page_size", "num_layers", "kv_tensors_per_token", "bytes_per_token",
        "page_size_bytes", "page_count")]


class OraPool(ctypes.Structure):
    _fields_ = [
        ("page_size", ctypes.c_uint64), ("page_stride", ctypes.c_uint64),
        ("page_count", ctypes.c_uint64), ("tensor_offset", ctypes.c_uint64 * 2),
        ("row_bytes", ctypes.c_uint64), ("tensors", ctypes.c_uint32),
        ("heads", ctypes.c_uint32), ("hnd", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
        ("value_row_bytes", ctypes.c_uint64),
    ]


class OraSpan(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "row_start", "token_offset", "token_count", "page_table_start")]


SPAN_DTYPE = np.dtype([("row_start", "<u4"), ("token_offset", "<u4"),
                       ("token_count", "<u4"), ("page_table_start", "<u4")])


def _load():
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(f"oracle library missing: run `make -C {_HERE}` ({_LIB_PATH})")
    lib = ctypes.CDLL(_LIB_PATH)
    lib.ora_tensor_token_byte_range.argtypes = [ctypes.POINTER(OraLayout), _u64, _u64, _u64, _u64, _u64p, _u64p]
    lib.ora_tensor_slot_byte_range.argtypes = [ctypes.POINTER(OraLayout), _u64, _u64, _u64, _u64p, _u64p]
    lib.ora_pair_tensor_token_byte_range.argtypes = [ctypes.POINTER(OraLayout), _u64, _u64, _u64, _u64, _u64, _u64, _u64p, _u64p]
    for name in ("ora_ref_gather_kv_pair_bytes", "ora_ref_scatter_kv_pair_bytes"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_uint32
    lib.ora_ref_gather_kv_pair_bytes.argtypes = [_u8p, _u64p, _u8p, _u8p] + [_u64] * 9
    lib.ora_ref_scatter_kv_pair_bytes.argtypes = [_u8p, _u8p, _u64p, _u8p] + [_u64] * 9
    lib.ora_resolve_slots.restype = ctypes.c_uint32
    lib.ora_resolve_slots.argtypes = [ctypes.POINTER(OraPool), _u64p, _i32p, _u64,
                                      ctypes.POINTER(OraSpan), ctypes.c_uint32, _u64, _u64p]
    lib.ora_pool_chunk_offset.restype = ctypes.c_uint64
    lib.ora_pool_chunk_offset.argtypes = [ctypes.POINTER(OraPool), _u64, ctypes.c_uint32, ctypes.c_uint32]
    lib.ora_pack.argtypes = [ctypes.POINTER(OraPool), _u8p, _u64p, _u64, _u8p, _u8p, _u64, _u64, ctypes.c_int]
    lib.ora_unpack.argtypes = [ctypes.POINTER(OraPool), _u8p, _u64p, _u64, _u8p, _u8p, _u64, _u64, ctypes.c_int]
    lib.ora_transfer.argtypes = [ctypes.POINTER(OraPool), _u8p, _u64p, ctypes.POINTER(OraPool),
                                 _u8p, _u64p, _u64, ctypes.c_int]
    lib.ora_transfer_page_indices.argtypes = [_u64, _u64p, _u64, _u64, _u64p, _u64p]
    lib.ora_f32_to_bf16.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_uint16), _u64]
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _p(a: np.ndarray, ctype):
    assert a.flags["C_CONTIGUOUS"], "oracle buffers must be C-contiguous"
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _bytes(a: np.ndarray) -> np.ndarray:
    """Flat uint8 view of a contiguous array (no copy)."""
    return a.reshape(-1).view(np.uint8)


# --- layout ---------------------------------------------------------------

def layout(page_size, num_layers, kv_tensors_per_token, bytes_per_token, page_size_bytes, page_count):
    return OraLayout(page_size, num_layers, kv_tensors_per_token, bytes_per_token,
                     page_size_bytes, page_count)


def tensor_token_byte_range(lay: OraLayout, page, layer, tensor, token):
    s, e = _u64(), _u64()
    rc = lib().ora_tensor_token_byte_range(ctypes.byref(lay), page, layer, tensor, token,
                                           ctypes.byref(s), ctypes.byref(e))
    return (rc, None) if rc else (0, (s.value, e.value))


def tensor_slot_byte_range(lay: OraLayout, layer, tensor, slot):
    s, e = _u64(), _u64()
    rc = lib().ora_tensor_slot_byte_range(ctypes.byref(lay), layer, tensor, slot,
                                          ctypes.byref(s), ctypes.byref(e))
    return (rc, None) if rc else (0, (s.value, e.value))


def pair_tensor_token_byte_range(lay: OraLayout, key_bytes, value_bytes, page, layer, tensor, token):
    s, e = _u64(), _u64()
    rc = lib().ora_pair_tensor_token_byte_range(ctypes.byref(lay), key_bytes, value_bytes, page,
                                                layer, tensor, token, ctypes.byref(s), ctypes.byref(e))
    return (rc, None) if rc else (0, (s.value, e.value))


# --- literal reference kernels ----------------------------------------------

def ref_gather_kv_pair_bytes(pool, slots, keys, values, *, slot_count, page_size, page_stride_bytes,
                             key_in_page_offset, value_in_page_offset, row_bytes,
                             key_row_stride_bytes, value_row_stride_bytes) -> int:
    slots = np.ascontiguousarray(slots, dtype=np.uint64)
    return lib().ora_ref_gather_kv_pair_bytes(
        _p(_bytes(pool), ctypes.c_uint8), _p(slots, ctypes.c_uint64),
        _p(_bytes(keys), ctypes.c_uint8), _p(_bytes(values), ctypes.c_uint8),
        len(slots), slot_count, page_size, page_stride_bytes, key_in_page_offset,
        value_in_page_offset, row_bytes, key_row_stride_bytes, value_row_stride_bytes)


def ref_scatter_kv_pair_bytes(keys, values, slots, pool, *, slot_count, page_size, page_stride_bytes,
                              key_in_page_offset, value_in_page_offset, row_bytes,
                              key_row_stride_bytes, value_row_stride_bytes) -> int:
    slots = np.ascontiguousarray(slots, dtype=np.uint64)
    return lib().ora_ref_scatter_kv_pair_bytes(
        _p(_bytes(keys), ctypes.c_uint8), _p(_bytes(values), ctypes.c_uint8),
        _p(slots, ctypes.c_uint64), _p(_bytes(pool), ctypes.c_uint8),
        len(slots), slot_count, page_size, page_stride_bytes, key_in_page_offset,
        value_in_page_offset, row_bytes, key_row_stride_bytes, value_row_stride_bytes)


# --- generalised pack / unpack ----------------------------------------------

@dataclass
class Pool:
    """One layer of a page-major pool (mirrors ``ora_pool``)."""
    page_size: int
    page_stride: int
    page_count: int
    tensor_offset: tuple
    row_bytes: int
    tensors: int
    heads: int
    hnd: bool
    value_row_bytes: int = 0   # tensor 1's width when it differs (tensor-pair layouts)

    def tensor_row_bytes(self, tensor: int) -> int:
        return self.value_row_bytes if tensor == 1 and self.value_row_bytes else self.row_bytes

    def c(self) -> OraPool:
        off = (ctypes.c_uint64 * 2)(*(list(self.tensor_offset) + [0, 0])[:2])
        return OraPool(self.page_size, self.page_stride, self.page_count, off, self.row_bytes,
                       self.tensors, self.heads, int(self.hnd), 0, self.value_row_bytes)


def resolve_slots(pool: Pool, row_count: int, slots=None, page_table=None, spans=None):
    out = np.empty(row_count, dtype=np.uint64)
    cpool = pool.c()
    if slots is not None:
        slots = np.ascontiguousarray(slots, dtype=np.uint64)
        flag = lib().ora_resolve_slots(ctypes.byref(cpool), _p(slots, ctypes.c_uint64), None, 0,
                                       None, 0, row_count, _p(out, ctypes.c_uint64))
    else:
        pt = np.ascontiguousarray(page_table, dtype=np.int32)
        sp = np.ascontiguousarray(spans, dtype=SPAN_DTYPE)
        flag = lib().ora_resolve_slots(ctypes.byref(cpool), None, _p(pt, ctypes.c_int32), len(pt),
                                       sp.ctypes.data_as(ctypes.POINTER(OraSpan)), len(sp),
                                       row_count, _p(out, ctypes.c_uint64))
    return out, flag


def pool_chunk_offset(pool: Pool, slot, tensor, head) -> int:
    cpool = pool.c()
    return lib().ora_pool_chunk_offset(ctypes.byref(cpool), slot, tensor, head)


def pack(pool: Pool, pool_bytes: np.ndarray, row_slots: np.ndarray, rows0: np.ndarray,
         rows1: np.ndarray | None, stride0: int, stride1: int = 0, threads: int = 1):
    row_slots = np.ascontiguousarray(row_slots, dtype=np.uint64)
    cpool = pool.c()
    lib().ora_pack(ctypes.byref(cpool), _p(_bytes(pool_bytes), ctypes.c_uint8),
                   _p(row_slots, ctypes.c_uint64), len(row_slots),
                   _p(_bytes(rows0), ctypes.c_uint8),
                   None if rows1 is None else _p(_bytes(rows1), ctypes.c_uint8),
                   stride0, stride1, threads)


def unpack(pool: Pool, pool_bytes: np.ndarray, row_slots: np.ndarray, rows0: np.ndarray,
           rows1: np.ndarray | None, stride0: int, stride1: int = 0, threads: int = 1):
    row_slots = np.ascontiguousarray(row_slots, dtype=np.uint64)
    cpool = pool.c()
    lib().ora_unpack(ctypes.byref(cpool), _p(_bytes(pool_bytes), ctypes.c_uint8),
                     _p(row_slots, ctypes.c_uint64), len(row_slots),
                     _p(_bytes(rows0), ctypes.c_uint8),
                     None if rows1 is None else _p(_bytes(rows1), ctypes.c_uint8),
                     stride0, stride1, threads)


def transfer(src: Pool, src_bytes, src_slots, dst: Pool, dst_bytes, dst_slots, threads: int = 1):
    src_slots = np.ascontiguousarray(src_slots, dtype=np.uint64)
    dst_slots = np.ascontiguousarray(dst_slots, dtype=np.uint64)
    assert len(src_slots) == len(dst_slots)
    cs, cd = src.c(), dst.c()
    lib().ora_transfer(ctypes.byref(cs), _p(_bytes(src_bytes), ctypes.c_uint8),
                       _p(src_slots, ctypes.c_uint64), ctypes.byref(cd),
                       _p(_bytes(dst_bytes), ctypes.c_uint8), _p(dst_slots, ctypes.c_uint64),
                       len(src_slots), threads)


def transfer_page_indices(token_offset: int, cache_slots, page_size: int):
    slots = np.ascontiguousarray(cache_slots, dtype=np.uint64)
    out = np.zeros(max(1, -(-len(slots) // max(page_size, 1))), dtype=np.uint64)
    n = _u64()
    rc = lib().ora_transfer_page_indices(token_offset, _p(slots, ctypes.c_uint64), len(slots),
                                         page_size, _p(out, ctypes.c_uint64), ctypes.byref(n))
    return rc, out[: n.value].tolist()


# --- scheduler-side plan metadata (pure Python restatement, small cases) ---------------------

PLAN_ZERO_PAGE_SIZE = 40
PLAN_CACHE_PAGE_COUNT_MISMATCH = 41
PLAN_TRAILING_CACHE_PAGES = 42
PLAN_NON_PREFILL_BATCH = 46


class RadixCache:
    """RadixCache (crates/sglang-srt/src/cache.rs:475-547) as nested dicts:
    a node is [cache_page or None, {token: child}]. insert (:485-504) gives
    every node on the path its token's page; match_prefix (:506-530) walks
    while the next token has a node with a page; match_prefix_page_aligned
    (:532-540) rounds the match down to whole pages."""

    def __init__(self):
        self.root = [None, {}]

    def insert(self, input_ids, cache_pages):
        assert len(input_ids) == len(cache_pages)
        node = self.root
        for tok, page in zip(input_ids, cache_pages):
            node = node[1].setdefault(int(tok), [None, {}])
            node[0] = int(page)

    def match_prefix_page_aligned(self, input_ids, page_size: int):
        """(matched_token_count, cache_pages, remaining_input_ids)."""
        assert page_size > 0
        node, pages = self.root, []
        for tok in input_ids:
            child = node[1].get(int(tok))
            if child is None or child[0] is None:
                break
            pages.append(child[0])
            node = child
        m = len(pages) // page_size * page_size
        return m, pages[:m], [int(t) for t in input_ids[m:]]


def transfer_plan_from_prefill_batch(input_token_counts, cached_token_counts, has_params, out_cache_pages,
                                     page_size: int, prefill: bool = True):
    """KvCacheTransferPlan::from_prefill_worker_batch_with_page_size
    (crates/sglang-srt/src/transfer.rs:604-668). Returns (0, spans) with a
    span = (request_index, token_offset, token_count, cache_pages,
    page_indices), or (code, None) with the error's status code."""
    if not prefill:
        return PLAN_NON_PREFILL_BATCH, None
    if page_size == 0:
        return PLAN_ZERO_PAGE_SIZE, None
    spans, offset = [], 0
    for r, count in enumerate(input_token_counts):
        end = offset + int(count)
        if end > len(out_cache_pages):
            return PLAN_CACHE_PAGE_COUNT_MISMATCH, None
        slots = [int(s) for s in out_cache_pages[offset:end]]
        offset = end
        if not has_params[r]:
            continue
        rc, pages = transfer_page_indices(int(cached_token_counts[r]), slots, page_size)
        if rc:
            return rc, None
        spans.append((r, int(cached_token_counts[r]), int(count), slots, pages))
    if offset != len(out_cache_pages):
        return PLAN_TRAILING_CACHE_PAGES, None
    return 0, spans


def f32_to_bf16(values: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(v.shape, dtype=np.uint16)
    lib().ora_f32_to_bf16(_p(v, ctypes.c_float), _p(out, ctypes.c_uint16), v.size)
    return out


# --- paged attention (float64 restatement, test infrastructure) -------------------------------

FLAG_ATTN_REQUEST = 1
FLAG_ATTN_SEQUENCE = 2
FLAG_ATTN_SLOT = 4


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def paged_attention(pool: np.ndarray, queries: np.ndarray, query_request_indices,
                    query_sequence_lengths, request_slot_offsets, sequence_slots, *,
                    page_size: int, page_stride: int, key_offset: int, value_offset: int,
                    kv_heads: int, dk: int, dv: int, scale: float, slot_count: int,
                    hnd: bool = False, with_abs: bool = False):
    """sglang_paged_attention_bf16 (crates/sglang-kernel/src/cuda_attention.rs:
    14-155) in float64: for query q of request r, softmax(scale * q.k) . v over
    the first len_q slots of r's slot list; query head h reads KV head
    h // (query_heads // kv_heads). Keys of KV head g at slot s start at byte
    (s // P) * page_stride + key_offset + (NHD) (s % P) * kv_heads*dk*2 + g*dk*2
    or (HND) g*P*dk*2 + (s % P)*dk*2; values alike.

    `pool` is the pool's bytes (uint8), `queries` bf16 bits [Q][QH][dk].
    Returns (out float64 [Q][QH][dv] with NaN rows for rejected queries,
    flags): the reference's metadata checks (:59-82) and slot check (:96-99)
    set flag bits 1, 2, 4 and skip the query. With `with_abs`, a third array
    holds sum_i w_i |v_i| per output element (w the softmax weights): the
    scale of the error that rounding the weights introduces.
    """
    q_bits = np.asarray(queries, dtype=np.uint16)
    nq, qh, _ = q_bits.shape
    group = qh // kv_heads
    pool16 = np.asarray(pool, dtype=np.uint8).view(np.uint16)
    qri = np.asarray(query_request_indices, dtype=np.uint64)
    qsl = np.asarray(query_sequence_lengths, dtype=np.uint64)
    rso = np.asarray(request_slot_offsets, dtype=np.uint64)
    slots_all = np.asarray(sequence_slots, dtype=np.uint64)
    request_count = len(rso) - 1
    out = np.full((nq, qh, dv), np.nan)
    absw = np.full((nq, qh, dv), np.nan)
    flags = 0
    for q in range(nq):
        r = int(qri[q])
        if r >= request_count:
            flags |= FLAG_ATTN_REQUEST
            continue
        s0, s1, n = int(rso[r]), int(rso[r + 1]), int(qsl[q])
        if s0 > s1 or s1 > len(slots_all) or n == 0 or n > s1 - s0:
            flags |= FLAG_ATTN_SEQUENCE
            continue
        sl = slots_all[s0:s0 + n].astype(np.int64)
        if (sl >= slot_count).any():
            flags |= FLAG_ATTN_SLOT
            continue
        page, pos = sl // page_size, sl % page_size
        for g in range(kv_heads):
            if hnd:
                kbyte = page * page_stride + key_offset + g * page_size * dk * 2 + pos * dk * 2
                vbyte = page * page_stride + value_offset + g * page_size * dv * 2 + pos * dv * 2
            else:
                kbyte = page * page_stride + key_offset + pos * kv_heads * dk * 2 + g * dk * 2
                vbyte = page * page_stride + value_offset + pos * kv_heads * dv * 2 + g * dv * 2
            k = bf16_to_f32(pool16[(kbyte // 2)[:, None] + np.arange(dk)]).astype(np.float64)
            v = bf16_to_f32(pool16[(vbyte // 2)[:, None] + np.arange(dv)]).astype(np.float64)
            qv = bf16_to_f32(q_bits[q, g * group:(g + 1) * group]).astype(np.float64)
            s = (qv @ k.T) * scale
            s -= s.max(axis=1, keepdims=True)
            w = np.exp(s)
            out[q, g * group:(g + 1) * group] = (w @ v) / w.sum(axis=1, keepdims=True)
            absw[q, g * group:(g + 1) * group] = (w @ np.abs(v)) / w.sum(axis=1, keepdims=True)
    return (out, flags, absw) if with_abs else (out, flags)
