"""Small seeded pack/unpack cases whose results are frozen as SHA-256 digests
in pool_digests.json (written by make_pool_digests.py).

Each case is one pool geometry on each side of a transfer: page-major pools
(page -> layer -> tensor -> token, crates/sglang-srt/src/kv_cache.rs:653-700),
tensor t of a layer holding rows of widths[t] bytes, token-major (NHD) or
head-major (HND) inside its page region. The inputs are pure functions of the
case: pool bytes from a splitmix64 stream, a source slot list of distinct
slots, and destination slots from a page table of distinct pages. Nothing here
depends on numpy's random generators, so the digests are stable across numpy
versions.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def splitmix64(seed: int, count: int) -> np.ndarray:
    """`count` outputs of splitmix64 (Steele, Lea, Flood 2014) from `seed`."""
    x = (np.uint64(seed) + np.arange(1, count + 1, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15))
    z = x.copy()
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def stream_bytes(seed: int, nbytes: int) -> np.ndarray:
    words = splitmix64(seed, (nbytes + 7) // 8)
    return words.view(np.uint8)[:nbytes].copy()


def distinct(seed: int, count: int, universe: int) -> np.ndarray:
    """`count` distinct values below `universe`: a Fisher-Yates shuffle of
    range(universe) driven by splitmix64, first `count` entries."""
    perm = np.arange(universe, dtype=np.uint64)
    r = splitmix64(seed, universe)
    for i in range(universe - 1, 0, -1):
        j = int(r[i] % np.uint64(i + 1))
        perm[i], perm[j] = perm[j], perm[i]
    return perm[:count]


@dataclass(frozen=True)
class Side:
    page_size: int
    page_count: int
    hnd: bool = False

    def page_stride(self, case: "Case") -> int:
        return self.page_size * case.layers * sum(case.widths)

    def byte_len(self, case: "Case") -> int:
        return self.page_count * self.page_stride(case)

    def tensor_offsets(self, case: "Case", layer: int):
        base = layer * self.page_size * sum(case.widths)
        return [base + self.page_size * sum(case.widths[:t]) for t in range(len(case.widths))]


@dataclass(frozen=True)
class Case:
    name: str
    layers: int
    widths: tuple        # row bytes of tensor 0 (and 1)
    heads: int           # head chunks per row (HND sides split rows into these)
    src: Side
    dst: Side
    tokens: int
    seed: int

    def src_slots(self) -> np.ndarray:
        return distinct(self.seed, self.tokens, self.src.page_size * self.src.page_count)

    def dst_slots(self) -> np.ndarray:
        P = self.dst.page_size
        pages = distinct(self.seed + 1, -(-self.tokens // P), self.dst.page_count)
        tok = np.arange(self.tokens, dtype=np.uint64)
        return pages[tok // np.uint64(P)] * np.uint64(P) + tok % np.uint64(P)

    def src_pool(self) -> np.ndarray:
        return stream_bytes(self.seed + 2, self.src.byte_len(self))

    def dst_pool(self) -> np.ndarray:
        return stream_bytes(self.seed + 3, self.dst.byte_len(self))

    def rows_bytes(self) -> int:
        """The transfer rows: [layer][tensor][token][widths[tensor]]."""
        return self.layers * self.tokens * sum(self.widths)

    def plane_offset(self, layer: int, tensor: int) -> int:
        return layer * self.tokens * sum(self.widths) + self.tokens * sum(self.widths[:tensor])


CASES = [
    # C1's geometry (Qwen2-0.5B-like: 2 heads x 64 dims, bf16 K and V), P1 -> P16.
    Case("c1_geometry", 24, (256, 256), 2, Side(1, 2048), Side(16, 64), 600, 101),
    # 8 heads x 128 dims, token-major P1 -> head-major P16 (the relayout C3 cannot show).
    Case("hnd_eight_heads", 4, (2048, 2048), 8, Side(1, 1024), Side(16, 32, True), 300, 202),
    # DeepSeek-V3's pair: 576-dim bf16 keys, 512-dim values, P64 -> P1.
    Case("mla_pair", 3, (1152, 1024), 1, Side(64, 16), Side(1, 1024), 500, 303),
    # Packed-MLA fp8 rows of 649 bytes (kv_cache.rs:201-224), P64 -> P64.
    Case("packed_mla_649", 3, (649,), 1, Side(64, 16), Side(64, 16), 400, 404),
    # One 576-byte fp8 latent row per token (the C4 fp8 form), P64 -> P64.
    Case("latent_576_fp8", 4, (576,), 1, Side(64, 12), Side(64, 12), 300, 505),
    # 64-byte head chunks (Llama-3.2-1B KV in fp8: 8 heads x 64 dims), P1 -> head-major P64.
    Case("hnd_64_byte_chunks", 2, (512, 512), 8, Side(1, 1024), Side(64, 8, True), 400, 606),
]


def numpy_pack_unpack(case: Case):
    """Rows and final destination pool by numpy indexing of views whose axes
    are the layout's nesting order (an independent route from the C oracle
    and the kernels)."""
    src, dst = case.src_pool(), case.dst_pool()
    ss, ds = case.src_slots().astype(np.int64), case.dst_slots().astype(np.int64)
    rows = np.zeros(case.rows_bytes(), dtype=np.uint8)

    def region(pool, side, tensor):
        # [page][layer][P * widths...] -> tensor t's [page][layer][P * w_t]
        per_layer = side.page_size * sum(case.widths)
        v = pool.reshape(side.page_count, case.layers, per_layer)
        lo = side.page_size * sum(case.widths[:tensor])
        return v[:, :, lo: lo + side.page_size * case.widths[tensor]]

    def tokens_view(pool, side, tensor):
        w = case.widths[tensor]
        r = region(pool, side, tensor)
        if side.hnd:  # [page][layer][head][P][chunk] -> [page][layer][P][head][chunk]
            c = w // case.heads
            return r.reshape(side.page_count, case.layers, case.heads, side.page_size, c).transpose(0, 1, 3, 2, 4)
        return r.reshape(side.page_count, case.layers, side.page_size, 1, w)

    for layer in range(case.layers):
        for t, w in enumerate(case.widths):
            sv = tokens_view(src, case.src, t)
            got = sv[ss // case.src.page_size, layer, ss % case.src.page_size].reshape(case.tokens, w)
            o = case.plane_offset(layer, t)
            rows[o: o + case.tokens * w] = got.reshape(-1)
            dv = tokens_view(dst, case.dst, t)  # a view: writes land in dst
            assert np.shares_memory(dv, dst)
            dv[ds // case.dst.page_size, layer, ds % case.dst.page_size] = got.reshape(
                case.tokens, dv.shape[3], dv.shape[4])
    return rows, dst
