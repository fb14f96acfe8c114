"""The KV-transfer workloads of the benchmark configurations, as seeded
generators of request lengths, slot maps and page tables.

Shapes follow the reference's model layouts: GQA models store K and V per
token per layer (``KvCacheModelLayout::multi_tensor``, crates/sglang-srt/src/
models/qwen.rs:234-239). The MLA workloads come in the three forms the
configurations and the reference use: one 576-wide latent row per token (a
single-tensor layout, as BASELINE's C4 words it), the DeepSeek-V3 adapter's
tensor pair of a 576-wide key and a 512-wide value
(``KvCacheModelLayout::tensor_pair``, models/deepseek.rs:360-369), and the
packed-MLA byte rows of 649 bytes (``KvCacheModelLayout::packed_mla``,
models/deepseek.rs:1035-1037). Slot maps stand in for the scheduler's
``out_cache_pages`` (crates/sglang-srt/src/model_executor.rs:158-175), page
tables for the decode side's ``dst_kv_indices``
(crates/sglang-srt/src/pd_bootstrap.rs:416-494).

All randomness comes from numpy's PCG64 seeded per workload; parity never
depends on it (the GPU result is compared with the CPU oracle on the same
bytes), it only fixes what is measured.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import HND, NHD, SPAN_DTYPE


@dataclass
class Shape:
    layers: int
    heads: int
    head_dim: int
    elt_bytes: int
    tensors: int  # 2 = K/V, 1 = MLA latent row
    value_head_dim: int = 0  # tensor 1's head dim when it differs (a tensor pair); 0 = head_dim

    def tensor_row_bytes(self, tensor: int) -> int:
        """Bytes per (token, layer) of `tensor`."""
        hd = self.value_head_dim if tensor == 1 and self.value_head_dim else self.head_dim
        return self.heads * hd * self.elt_bytes

    @property
    def row_bytes(self) -> int:
        """Tensor 0's row (every tensor's, unless a pair of unequal widths)."""
        return self.tensor_row_bytes(0)

    @property
    def layer_row_bytes(self) -> int:
        """Bytes one token owns in one layer, all tensors."""
        return sum(self.tensor_row_bytes(t) for t in range(self.tensors))

    @property
    def token_bytes(self) -> int:
        """Bytes one token owns across all layers and tensors."""
        return self.layers * self.layer_row_bytes


@dataclass
class PoolSpec:
    page_size: int
    page_count: int
    head_layout: int = NHD

    def page_stride(self, shape: Shape) -> int:
        return self.page_size * shape.token_bytes

    def byte_len(self, shape: Shape) -> int:
        return self.page_count * self.page_stride(shape)

    def tensor_offsets(self, shape: Shape, layer: int):
        """In-page offsets of the layer's tensor regions (kv_cache.rs:653-700;
        a pair's value region follows page_size key rows, :808-818)."""
        per_layer = self.page_size * shape.layer_row_bytes
        return tuple(layer * per_layer + t * self.page_size * shape.row_bytes
                     for t in range(shape.tensors))


@dataclass
class Transfer:
    """One transfer: rows [0, rows) move from src slots to dst slots."""
    name: str
    shape: Shape
    src: PoolSpec
    dst: PoolSpec
    lengths: np.ndarray          # uncached tokens moved per request
    src_slots: np.ndarray        # u64 per row
    dst_slots: np.ndarray        # u64 per row
    dst_page_table: np.ndarray   # i32, the decode side's pages, request after request
    dst_spans: np.ndarray        # SPAN_DTYPE per request
    prefix_tokens: np.ndarray = field(default=None)

    @property
    def rows(self) -> int:
        return int(len(self.src_slots))

    @property
    def payload_bytes(self) -> int:
        return self.rows * self.shape.token_bytes

    @property
    def algorithmic_bytes(self) -> int:
        """pack reads + writes the payload, unpack reads + writes it again."""
        return 4 * self.payload_bytes


def _page_table_slots(rng, lengths, prefix, page_size, page_count):
    """Random decode-side pages for each request; rows cover tokens
    [prefix, prefix + length) of each request."""
    need = [-(-(int(p) + int(n)) // page_size) for p, n in zip(prefix, lengths)]
    if sum(need) > page_count:
        raise ValueError(f"{sum(need)} pages needed, pool has {page_count}")
    perm = rng.permutation(page_count).astype(np.int32)
    table = perm[: sum(need)]
    spans = np.zeros(len(lengths), dtype=SPAN_DTYPE)
    slots = np.empty(int(np.sum(lengths)), dtype=np.uint64)
    row = pt = 0
    for i, (n, p) in enumerate(zip(lengths, prefix)):
        n, p = int(n), int(p)
        spans[i] = (row, p, n, pt)
        tok = p + np.arange(n, dtype=np.int64)
        slots[row: row + n] = (table[pt + tok // page_size].astype(np.int64) * page_size
                               + tok % page_size).astype(np.uint64)
        row += n
        pt += need[i]
    return table, spans, slots


def _token_slots(rng, rows, slot_count):
    """Distinct random slots of a page_size-1 pool (a seeded permutation)."""
    if rows > slot_count:
        raise ValueError(f"{rows} rows need more than {slot_count} slots")
    return rng.permutation(slot_count)[:rows].astype(np.uint64)


def c1(seed: int = 1) -> Transfer:
    """Qwen2-0.5B-like GQA transfer, the CPU-reference configuration."""
    rng = np.random.default_rng(seed)
    shape = Shape(24, 2, 64, 2, 2)
    lengths = rng.integers(100, 1001, size=8)
    rows = int(lengths.sum())
    src = PoolSpec(1, 65536)
    dst = PoolSpec(16, -(-65536 // 16))
    table, spans, dslots = _page_table_slots(rng, lengths, np.zeros(8, int), 16, dst.page_count)
    return Transfer("C1 qwen2-0.5b-like", shape, src, dst, lengths,
                    _token_slots(rng, rows, src.page_count), dslots, table, spans,
                    np.zeros(8, np.int64))


def c2(seed: int = 2) -> Transfer:
    """Llama-3-8B-shape GQA transfer: 64 requests x 2048 tokens (16 GiB of KV)."""
    rng = np.random.default_rng(seed)
    shape = Shape(32, 8, 128, 2, 2)
    lengths = np.full(64, 2048)
    src = PoolSpec(1, 262144)
    dst = PoolSpec(64, 4096)
    table, spans, dslots = _page_table_slots(rng, lengths, np.zeros(64, int), 64, dst.page_count)
    return Transfer("C2 llama-3-8b", shape, src, dst, lengths,
                    _token_slots(rng, int(lengths.sum()), src.page_count), dslots, table, spans,
                    np.zeros(64, np.int64))


def c3(seed: int = 3) -> Transfer:
    """One TP rank of Llama-3-70B (1 KV head): NHD page_size-1 -> HND page_size-64."""
    rng = np.random.default_rng(seed)
    shape = Shape(80, 1, 128, 2, 2)
    lengths = rng.integers(512, 8193, size=128)
    rows = int(lengths.sum())
    src = PoolSpec(1, rows + rows // 4)
    pages = sum(-(-int(n) // 64) for n in lengths)
    dst = PoolSpec(64, pages + pages // 4, HND)
    table, spans, dslots = _page_table_slots(rng, lengths, np.zeros(128, int), 64, dst.page_count)
    return Transfer("C3 llama-3-70b tp-rank hnd", shape, src, dst, lengths,
                    _token_slots(rng, rows, src.page_count), dslots, table, spans,
                    np.zeros(128, np.int64))


def c4(seed: int = 4, fp8: bool = False) -> Transfer:
    """MLA latent rows (576 wide) between two page_size-64 pools with
    independent random page tables."""
    rng = np.random.default_rng(seed)
    shape = Shape(61, 1, 576, 1 if fp8 else 2, 1)
    lengths = np.full(32, 8192)
    src = PoolSpec(64, 4096)
    dst = PoolSpec(64, 4096)
    _, _, sslots = _page_table_slots(rng, lengths, np.zeros(32, int), 64, src.page_count)
    table, spans, dslots = _page_table_slots(rng, lengths, np.zeros(32, int), 64, dst.page_count)
    return Transfer("C4 mla-576" + (" fp8" if fp8 else ""), shape, src, dst, lengths, sslots,
                    dslots, table, spans, np.zeros(32, np.int64))


def c4pair(seed: int = 4, fp8: bool = False, dst_page_size: int = 64) -> Transfer:
    """C4's requests over the pool the DeepSeek-V3 adapter allocates: the
    tensor pair of a 576-wide key (latent + rope) and a 512-wide value per
    token per layer (models/deepseek.rs:360-369; 1,152 + 1,024 bytes in
    bf16), page_size-64 source, destination page size `dst_page_size`."""
    rng = np.random.default_rng(seed)
    shape = Shape(61, 1, 576, 1 if fp8 else 2, 2, value_head_dim=512)
    lengths = np.full(32, 8192)
    src = PoolSpec(64, 4096)
    dst = PoolSpec(dst_page_size, -(-4096 * 64 // dst_page_size))
    _, _, sslots = _page_table_slots(rng, lengths, np.zeros(32, int), 64, src.page_count)
    table, spans, dslots = _page_table_slots(rng, lengths, np.zeros(32, int), dst_page_size,
                                             dst.page_count)
    return Transfer("C4 deepseek-v3 mla pair 576/512" + (" fp8" if fp8 else ""), shape, src, dst,
                    lengths, sslots, dslots, table, spans, np.zeros(32, np.int64))


def c4packed(seed: int = 4) -> Transfer:
    """C4's requests over packed-MLA rows: 649 bytes per token per layer
    (packed_mla(61, 512, 64), kv_cache.rs:201-224, as build_mla_moe_definition
    allocates it, models/deepseek.rs:1035-1037), page_size 64 on both sides."""
    rng = np.random.default_rng(seed)
    shape = Shape(61, 1, 649, 1, 1)
    lengths = np.full(32, 8192)
    src = PoolSpec(64, 4096)
    dst = PoolSpec(64, 4096)
    _, _, sslots = _page_table_slots(rng, lengths, np.zeros(32, int), 64, src.page_count)
    table, spans, dslots = _page_table_slots(rng, lengths, np.zeros(32, int), 64, dst.page_count)
    return Transfer("C4 packed-mla 649-byte rows", shape, src, dst, lengths, sslots, dslots, table,
                    spans, np.zeros(32, np.int64))


def chunks64(seed: int = 6, head_major: bool = True) -> Transfer:
    """Head chunks of 64 bytes: Llama-3.2-1B's KV shape (16 layers x 8 KV
    heads x 64 dims) stored in fp8 (one byte per element), so a 512-byte row
    is eight 64-byte head chunks. 64 requests x 2,048 tokens from a
    page_size-1 NHD pool into a page_size-64 pool with a random page table,
    head-major (HND: each head's chunks of a page contiguous, half a cache
    line per token) or token-major (NHD)."""
    rng = np.random.default_rng(seed)
    shape = Shape(16, 8, 64, 1, 2)
    lengths = np.full(64, 2048)
    src = PoolSpec(1, 262144)
    dst = PoolSpec(64, 4096, HND if head_major else NHD)
    table, spans, dslots = _page_table_slots(rng, lengths, np.zeros(64, int), 64, dst.page_count)
    return Transfer("llama-3.2-1b fp8, 64-byte head chunks, " + ("HND" if head_major else "NHD"),
                    shape, src, dst, lengths, _token_slots(rng, int(lengths.sum()), src.page_count),
                    dslots, table, spans, np.zeros(64, np.int64))


def c5(seed: int = 5, requests: int = 512) -> Transfer:
    """Ragged radix-prefix transfer: log-uniform lengths, a page-aligned
    prefix of each request already cached on the decode side."""
    rng = np.random.default_rng(seed)
    shape = Shape(32, 8, 128, 2, 2)
    total = np.exp(rng.uniform(np.log(16), np.log(32768), size=requests)).astype(np.int64)
    prefix = (rng.uniform(0, 0.9, size=requests) * total).astype(np.int64) // 64 * 64
    lengths = total - prefix
    rows = int(lengths.sum())
    src = PoolSpec(1, rows + rows // 8)
    pages = sum(-(-int(t) // 64) for t in total)
    dst = PoolSpec(64, pages + pages // 8)
    table, spans, dslots = _page_table_slots(rng, lengths, prefix, 64, dst.page_count)
    return Transfer("C5 ragged radix prefix", shape, src, dst, lengths,
                    _token_slots(rng, rows, src.page_count), dslots, table, spans, prefix)


def scaled(t: Transfer, max_rows: int, seed: int = 0) -> Transfer:
    """The first requests of `t` up to `max_rows` rows, with pools shrunk to
    what they cover (for sizes the CPU oracle checks in seconds)."""
    keep = int(np.searchsorted(np.cumsum(t.lengths), max_rows, side="right"))
    keep = max(1, keep)
    lengths = t.lengths[:keep]
    prefix = t.prefix_tokens[:keep] if t.prefix_tokens is not None else np.zeros(keep, np.int64)
    rng = np.random.default_rng(seed)
    rows = int(lengths.sum())
    if t.src.page_size == 1:
        src = PoolSpec(1, rows + rows // 4 + 1, t.src.head_layout)
        sslots = _token_slots(rng, rows, src.page_count)
    else:
        pages = sum(-(-int(n) // t.src.page_size) for n in lengths)
        src = PoolSpec(t.src.page_size, pages + pages // 4 + 1, t.src.head_layout)
        _, _, sslots = _page_table_slots(rng, lengths, np.zeros(keep, int), src.page_size,
                                         src.page_count)
    pages = sum(-(-(int(p) + int(n)) // t.dst.page_size) for p, n in zip(prefix, lengths))
    dst = PoolSpec(t.dst.page_size, pages + pages // 4 + 1, t.dst.head_layout)
    table, spans, dslots = _page_table_slots(rng, lengths, prefix, dst.page_size, dst.page_count)
    return Transfer(t.name + f" (first {rows} rows)", t.shape, src, dst, lengths, sslots, dslots,
                    table, spans, prefix)


def waves(t: Transfer, max_rows: int, max_pages: int, seed: int = 0):
    """Splits `t` into request waves whose rows fit a page_size-1 source pool
    of `max_rows` slots and whose pages (cached prefix included) fit a
    destination pool of `max_pages` pages; each wave gets fresh seeded slot
    maps inside those two fixed pools (the pools are reused wave after wave)."""
    rng = np.random.default_rng(seed)
    prefix = t.prefix_tokens if t.prefix_tokens is not None else np.zeros(len(t.lengths), np.int64)
    P = t.dst.page_size
    out, start = [], 0
    while start < len(t.lengths):
        rows = pages = 0
        end = start
        while end < len(t.lengths):
            r = int(t.lengths[end])
            pg = -(-(int(prefix[end]) + r) // P)
            if end > start and (rows + r > max_rows or pages + pg > max_pages):
                break
            rows, pages, end = rows + r, pages + pg, end + 1
        if rows > max_rows or pages > max_pages:
            raise ValueError(f"request {start} alone exceeds the wave pools")
        lengths, pre = t.lengths[start:end], prefix[start:end]
        src = PoolSpec(1, max_rows, t.src.head_layout)
        dst = PoolSpec(P, max_pages, t.dst.head_layout)
        table, spans, dslots = _page_table_slots(rng, lengths, pre, P, max_pages)
        out.append(Transfer(f"{t.name} wave {len(out)}", t.shape, src, dst, lengths,
                            _token_slots(rng, rows, max_rows), dslots, table, spans, pre))
        start = end
    return out
